// Causal gated GQA prefill attention on gfx950 bf16 MFMA (declaration).
#pragma once

#include "common.hpp"

namespace raftinfer::amd {

// q, gate, out: [tokens][16][256] bf16; key, value: [tokens][4][256] bf16;
// cache: bf16 K plane then V plane.  With fused_append (past must be 0) keys
// are read from key/value and each workgroup writes its tokens' cache rows;
// otherwise the cache must already hold positions 0..past+tokens-1.  Pointers
// to q, key, value and cache are 16-byte aligned, gate and out 8-byte.
// Enqueues on stream.
void launch_prefill_mfma(const bf16_bits *q, const bf16_bits *key, const bf16_bits *value,
                         const bf16_bits *gate, bf16_bits *out, bf16_bits *cache,
                         std::size_t tokens, std::size_t max_ctx, std::size_t past,
                         bool head_major, bool fused_append, hipStream_t stream);

} // namespace raftinfer::amd
