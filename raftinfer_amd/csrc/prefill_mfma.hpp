// Causal gated GQA prefill attention on gfx950 bf16 MFMA (declaration).
#pragma once

#include "common.hpp"

namespace raftinfer::amd {

// q, gate, out: [tokens][16][256] bf16; cache: bf16 K plane then V plane
// holding positions 0..past+tokens-1 (already appended).  Enqueues on stream.
void launch_prefill_mfma(const bf16_bits *q, const bf16_bits *gate, bf16_bits *out,
                         const bf16_bits *cache, std::size_t tokens, std::size_t max_ctx,
                         std::size_t past, bool head_major, hipStream_t stream);

} // namespace raftinfer::amd
