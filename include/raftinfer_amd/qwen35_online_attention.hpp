// Online (flash-style) attention entry points for gfx950.  Mirrors the
// reference's cpp/kernels/qwen35_online_attention.cuh:12-68 with hipStream_t.
// The decode plan and workspace layout are bit-identical to the reference's
// (cpp/kernels/qwen35_online_attention.cu:1071-1143).
#pragma once

#include "qwen35_attention.hpp"

#include <cstddef>
#include <cstdint>

namespace raftinfer::kernels {

struct Qwen35OnlineDecodePlan {
  Qwen35DecodeAttentionMode resolved_mode{Qwen35DecodeAttentionMode::single_block};
  std::size_t partition_tokens{};
  std::size_t split_k_threshold_tokens{};
  std::size_t context_bucket_tokens{};
  std::size_t active_partition_capacity{1};

  bool operator==(const Qwen35OnlineDecodePlan &) const = default;
};

struct Qwen35OnlineDecodeWorkspaceLayout {
  std::size_t partial_count{};
  std::size_t max_offset_bytes{};
  std::size_t sum_offset_bytes{};
  std::size_t value_offset_bytes{};
  std::size_t bytes{};

  bool operator==(const Qwen35OnlineDecodeWorkspaceLayout &) const = default;
};

Qwen35OnlineDecodePlan qwen35_online_decode_plan(Qwen35AttentionShape shape,
                                                 Qwen35DecodeAttentionMode requested,
                                                 std::size_t context_tokens);

Qwen35OnlineDecodeWorkspaceLayout
qwen35_online_decode_workspace_layout(Qwen35AttentionShape shape,
                                      Qwen35DecodeAttentionMode resolved_mode);

bool qwen35_online_attention_prefill_supported(Qwen35AttentionShape shape,
                                               RaftInferDataType activation_dtype,
                                               Qwen35AttentionLaunchPolicy policy) noexcept;

std::size_t qwen35_online_attention_workspace_bytes(Qwen35AttentionShape shape) noexcept;

void qwen35_online_attention_prefill(const void *query, const void *key, const void *value,
                                     const void *gate, void *output, void *kv_cache,
                                     std::size_t kv_cache_bytes, Qwen35AttentionShape shape,
                                     RaftInferDataType activation_dtype,
                                     Qwen35KvCacheDType cache_dtype,
                                     Qwen35KvCacheLayout cache_layout, hipStream_t stream);

void qwen35_online_attention_decode(const void *query, const void *key, const void *value,
                                    const void *gate, void *output, void *kv_cache,
                                    std::size_t kv_cache_bytes, void *workspace,
                                    std::size_t workspace_bytes, Qwen35AttentionShape shape,
                                    RaftInferDataType activation_dtype,
                                    Qwen35KvCacheDType cache_dtype,
                                    Qwen35KvCacheLayout cache_layout, Qwen35OnlineDecodePlan plan,
                                    const std::uint32_t *device_position, hipStream_t stream);

void qwen35_online_attention_decode(const void *query, const void *key, const void *value,
                                    const void *gate, void *output, void *kv_cache,
                                    std::size_t kv_cache_bytes, Qwen35AttentionShape shape,
                                    RaftInferDataType activation_dtype,
                                    Qwen35KvCacheDType cache_dtype,
                                    Qwen35KvCacheLayout cache_layout,
                                    const std::uint32_t *device_position, hipStream_t stream);

// ---- Additive: batched ragged decode (no counterpart in the reference). ----
// `sequences` independent Qwen3.5-shape (16/4/256) decodes in one enqueue.
// Each sequence b owns a BF16 head-major cache of `max_context_tokens`
// positions at kv_cache + b * cache_stride_bytes (layout as the single-sequence
// path).  context_lengths (device, uint32[sequences]) gives each sequence's
// context including the new token, which is appended at position length-1.
// Per-sequence policy: length <= single_block_max_tokens runs the
// single-block path, otherwise split-K with 256-token partitions and an LSE
// merge.  q/gate/out: [sequences][16][256]; k/v: [sequences][4][256].
// query, kv_cache and workspace must be 16-byte aligned.
struct Qwen35BatchedDecodeShape {
  std::size_t sequences;
  std::size_t max_context_tokens;
  std::size_t cache_stride_bytes;
  std::size_t single_block_max_tokens;
};
std::size_t qwen35_batched_decode_workspace_bytes(Qwen35BatchedDecodeShape shape);
void qwen35_online_attention_decode_batched(const void *query, const void *key,
                                            const void *value, const void *gate, void *output,
                                            void *kv_cache, std::size_t kv_cache_bytes,
                                            const std::uint32_t *context_lengths,
                                            void *workspace, std::size_t workspace_bytes,
                                            Qwen35BatchedDecodeShape shape,
                                            RaftInferDataType activation_dtype,
                                            hipStream_t stream);

// ---- Additive: producers fused into the attention (no counterpart in the
// reference). ----
// The RMSNorm + NeoX partial RoPE of q and k (qwen35_qk_norm_rope) and the
// q / gate split (qwen35_split_full_query_gate), which the reference runs as
// separate kernels before the attention (cpp/execution/qwen35_executor.cu:
// 1989-2013), done inside the attention kernels: the raw projections are read
// once and no intermediate q / gate / k buffer exists.  Results are bit-
// identical to the producers followed by the unfused call.  bf16 activations
// and a bf16 KV cache, the model signature, rotary_dim a multiple of 8 (at
// most 256); RoPE positions are past_tokens + t (decode: the device position
// when one is given).
struct Qwen35FusedNormRope {
  const void *query_norm_weight; // [head_dim]
  const void *key_norm_weight;   // [head_dim]
  RaftInferDataType weight_dtype; // bf16 or f32
  std::size_t rotary_dim;
  float rope_base;
  float epsilon;
};
// query_gate: [16][2][256] (query half then gate half per head, the q
// projection's layout); key: the raw k projection [4][256]; value [4][256].
// Otherwise as qwen35_online_attention_decode with a plan.
void qwen35_online_attention_decode_fused(const void *query_gate, const void *key,
                                          const void *value, void *output, void *kv_cache,
                                          std::size_t kv_cache_bytes, void *workspace,
                                          std::size_t workspace_bytes, Qwen35AttentionShape shape,
                                          Qwen35FusedNormRope norm, Qwen35KvCacheDType cache_dtype,
                                          Qwen35KvCacheLayout cache_layout,
                                          Qwen35OnlineDecodePlan plan,
                                          const std::uint32_t *device_position, hipStream_t stream);

// query_gate: [tokens][16][2][256]; key: the raw k projection [tokens][4][256];
// value [tokens][4][256].  The keys are normalised, rotated and appended with
// the values at past_tokens .. past_tokens + tokens - 1, then the causal gated
// attention runs as qwen35_online_attention_prefill.  A bf16 KV cache.
void qwen35_online_attention_prefill_fused(const void *query_gate, const void *key,
                                           const void *value, void *output, void *kv_cache,
                                           std::size_t kv_cache_bytes, Qwen35AttentionShape shape,
                                           Qwen35FusedNormRope norm, Qwen35KvCacheDType cache_dtype,
                                           Qwen35KvCacheLayout cache_layout, hipStream_t stream);

// Allocation-free decode (no counterpart in the reference): for callers that
// cannot allocate device memory (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc).  Same arguments and behaviour as
// qwen35_online_attention_decode with a plan, except that the split-K
// workspace is a library-owned static device array of
// qwen35_online_attention_static_workspace_bytes() bytes per GPU (8,454,144:
// max_context_tokens <= 131072 at split_k_256, <= 262144 at split_k_512); a
// larger plan is rejected with Qwen35PrimitiveError.  Nothing is allocated.
// Every call on one GPU shares that array, so calls that overlap on one GPU
// (different streams, or different host threads) race; serialize them.  The
// first call on each device looks up the array's address and must not be
// under stream capture (it throws there); later calls may be captured.
std::size_t qwen35_online_attention_static_workspace_bytes() noexcept;
void qwen35_online_attention_decode_static_workspace(
    const void *query, const void *key, const void *value, const void *gate, void *output,
    void *kv_cache, std::size_t kv_cache_bytes, Qwen35AttentionShape shape,
    RaftInferDataType activation_dtype, Qwen35KvCacheDType cache_dtype,
    Qwen35KvCacheLayout cache_layout, Qwen35OnlineDecodePlan plan,
    const std::uint32_t *device_position, hipStream_t stream);

// Measurement entry points (no counterpart in the reference): validate
// exactly like qwen35_online_attention_decode / _prefill, then enqueue only the
// dominant kernel -- the split-K partition kernel of a split plan, or the
// prefill attention kernel without the K/V append -- so a benchmark can time
// it alone with events on the same stream.
void qwen35_online_attention_decode_partition_only(
    const void *query, const void *key, const void *value, const void *gate, void *output,
    void *kv_cache, std::size_t kv_cache_bytes, void *workspace, std::size_t workspace_bytes,
    Qwen35AttentionShape shape, RaftInferDataType activation_dtype,
    Qwen35KvCacheDType cache_dtype, Qwen35KvCacheLayout cache_layout, Qwen35OnlineDecodePlan plan,
    const std::uint32_t *device_position, hipStream_t stream);
void qwen35_online_attention_prefill_kernel_only(
    const void *query, const void *key, const void *value, const void *gate, void *output,
    void *kv_cache, std::size_t kv_cache_bytes, Qwen35AttentionShape shape,
    RaftInferDataType activation_dtype, Qwen35KvCacheDType cache_dtype,
    Qwen35KvCacheLayout cache_layout, hipStream_t stream);

// Device-side capacity guard.  Where the reference merge kernel traps when a
// device-read position needs more partitions than the plan's capacity
// (cpp/kernels/qwen35_online_attention.cu:714-717), this build writes NaN to
// the affected heads, records the condition in a device flag and exits
// normally; the new K/V row is still appended when the position is inside the
// cache.  The batched decode counts a sequence whose length is 0 or above its
// maximum context the same way (its output rows become NaN).  Returns the
// number of such events since the last call and clears the flag
// (synchronizes the current device).
std::uint32_t qwen35_online_attention_consume_capacity_errors();

} // namespace raftinfer::kernels
