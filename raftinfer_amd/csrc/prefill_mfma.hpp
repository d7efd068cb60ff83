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

// The producers fused in (query_gate: the raw q projection [tokens][16][2][256];
// key: the raw k projection [tokens][4][256]): a key kernel normalises and
// rotates k and appends k and v at positions past..past+tokens-1, then the
// attention kernel normalises and rotates q while staging it and reads the
// gate from the projection's second half.  Bit-identical to the producers
// followed by launch_prefill_mfma.  Norm weights: 256 values, f32 (16-byte
// aligned) or bf16 (8-byte aligned); pairs = rotary_dim / 2, rotary_dim a
// multiple of 8; ratio = rope_base^(-2 / rotary_dim).
void launch_prefill_mfma_fused(const bf16_bits *query_gate, const bf16_bits *key,
                               const bf16_bits *value, bf16_bits *out, bf16_bits *cache,
                               std::size_t tokens, std::size_t max_ctx, std::size_t past,
                               bool head_major, const void *q_weight, const void *k_weight,
                               bool weight_f32, int pairs, double ratio, float epsilon,
                               hipStream_t stream);

} // namespace raftinfer::amd
