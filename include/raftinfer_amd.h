/*
 * raftinfer_amd: C ABI of the gfx950 attention / gated-delta hot path.
 *
 * Plain pointers and sizes only.  Every entry point returns a status code and
 * leaves a thread-local message readable through
 * raftinfer_amd_last_error_message() (the convention of the reference's C ABI,
 * cpp/src/c_api.cpp:44, :173-175).  Each wraps the C++ drop-in boundary in
 * the headers under include/raftinfer_amd/, which keeps the reference kernel signatures
 * (cpp/kernels/qwen35_attention.cuh, qwen35_online_attention.cuh,
 * qwen35_delta.cuh) with hipStream_t in place of cudaStream_t.
 *
 * Ownership: the caller owns every buffer (activations, KV cache, workspace,
 * convolution / recurrent state).  No entry point allocates device memory,
 * creates a stream or synchronizes, except
 * raftinfer_amd_consume_capacity_errors().  `stream` is a hipStream_t and must
 * not be null.
 */
#ifndef RAFTINFER_AMD_H
#define RAFTINFER_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum raftinfer_amd_status {
  RAFTINFER_AMD_OK = 0,
  /* Validation failure: Qwen35PrimitiveError / Qwen35DeltaError before launch. */
  RAFTINFER_AMD_INVALID_ARGUMENT = 1,
  /* A kernel launch reported an error. */
  RAFTINFER_AMD_LAUNCH_FAILED = 2,
  RAFTINFER_AMD_INTERNAL_ERROR = 3
} raftinfer_amd_status;

/* Enum values equal the reference's uint8 enumerators
 * (cpp/execution/qwen35_execution_policy.hpp:7-27). */
enum {
  RAFTINFER_AMD_IMPL_MATERIALIZED = 0,
  RAFTINFER_AMD_IMPL_ONLINE_TILED = 1,
  RAFTINFER_AMD_DECODE_AUTO = 0,
  RAFTINFER_AMD_DECODE_SINGLE_BLOCK = 1,
  RAFTINFER_AMD_DECODE_SPLIT_K_256 = 2,
  RAFTINFER_AMD_DECODE_SPLIT_K_512 = 3,
  RAFTINFER_AMD_CACHE_F32 = 0,
  RAFTINFER_AMD_CACHE_BF16 = 1,
  RAFTINFER_AMD_LAYOUT_TOKEN_MAJOR = 0,
  RAFTINFER_AMD_LAYOUT_HEAD_MAJOR = 1,
  RAFTINFER_AMD_DTYPE_F32 = 1,
  RAFTINFER_AMD_DTYPE_F16 = 2,
  RAFTINFER_AMD_DTYPE_BF16 = 3
};

/* Qwen35AttentionShape (cpp/kernels/qwen35_attention.cuh:14-21). */
typedef struct raftinfer_amd_attention_shape {
  size_t tokens, query_heads, kv_heads, head_dim, max_context_tokens, past_tokens;
} raftinfer_amd_attention_shape;

/* Qwen35AttentionLaunchPolicy (cpp/kernels/qwen35_attention.cuh:23-27). */
typedef struct raftinfer_amd_attention_policy {
  uint8_t implementation, kv_cache_dtype, kv_cache_layout;
} raftinfer_amd_attention_policy;

/* Qwen35OnlineDecodePlan (cpp/kernels/qwen35_online_attention.cuh:12-21). */
typedef struct raftinfer_amd_decode_plan {
  uint8_t resolved_mode;
  size_t partition_tokens, split_k_threshold_tokens, context_bucket_tokens,
      active_partition_capacity;
} raftinfer_amd_decode_plan;

/* Qwen35OnlineDecodeWorkspaceLayout (cpp/kernels/qwen35_online_attention.cuh:23-31). */
typedef struct raftinfer_amd_decode_layout {
  size_t partial_count, max_offset_bytes, sum_offset_bytes, value_offset_bytes, bytes;
} raftinfer_amd_decode_layout;

/* GatedDeltaShape (cpp/kernels/qwen35_delta.cuh:20-29). */
typedef struct raftinfer_amd_delta_shape {
  size_t tokens, hidden_size, key_heads, value_heads, key_dim, value_dim, conv_width;
  float epsilon;
} raftinfer_amd_delta_shape;

/* GatedDeltaLaunchPolicy (cpp/kernels/qwen35_delta.cuh:37-41). */
typedef struct raftinfer_amd_delta_policy {
  uint8_t schedule; /* 0 current, 1 prefill candidate (chunked), 2 decode candidate */
  uint32_t warps_per_block;
  uint8_t transposed_boundary_state;
} raftinfer_amd_delta_policy;

/* Batched ragged decode shape (additive; no reference counterpart). */
typedef struct raftinfer_amd_batched_decode_shape {
  size_t sequences, max_context_tokens, cache_stride_bytes, single_block_max_tokens;
} raftinfer_amd_batched_decode_shape;

/* cpp/kernels/qwen35_primitives.cuh:34-41 */
typedef struct raftinfer_amd_qk_norm_rope_shape {
  size_t tokens, heads, head_dim, rotary_dim, position_offset;
  float rope_base;
} raftinfer_amd_qk_norm_rope_shape;

typedef struct raftinfer_amd_delta_core_shape {
  size_t tokens, key_heads, value_heads, key_dim, value_dim;
} raftinfer_amd_delta_core_shape;

const char *raftinfer_amd_last_error_message(void);

/* ---- sizing / planning (host only, no device calls) ---- */
/* qwen35_attention.cuh:29-30 */
int raftinfer_amd_attention_workspace_floats(raftinfer_amd_attention_shape shape, size_t *out);
/* qwen35_attention.cuh:31-36 */
int raftinfer_amd_attention_cache_bytes(raftinfer_amd_attention_shape shape,
                                        raftinfer_amd_attention_policy policy, size_t *out);
int raftinfer_amd_attention_workspace_bytes(raftinfer_amd_attention_shape shape,
                                            raftinfer_amd_attention_policy policy, size_t *out);
/* qwen35_online_attention.cuh:33-35 */
int raftinfer_amd_online_decode_plan(raftinfer_amd_attention_shape shape, uint8_t requested_mode,
                                     size_t context_tokens, raftinfer_amd_decode_plan *out);
/* qwen35_online_attention.cuh:37-38 */
int raftinfer_amd_online_decode_workspace_layout(raftinfer_amd_attention_shape shape,
                                                 uint8_t resolved_mode,
                                                 raftinfer_amd_decode_layout *out);
/* qwen35_online_attention.cuh:40-42; returns 1 / 0. */
int raftinfer_amd_online_attention_prefill_supported(raftinfer_amd_attention_shape shape,
                                                     int activation_dtype,
                                                     raftinfer_amd_attention_policy policy);
/* qwen35_delta.cuh:64 */
int raftinfer_amd_gated_delta_workspace_bytes(raftinfer_amd_delta_shape shape, size_t *out);
/* qwen35_delta.cuh:69-71; writes the selected policy. */
int raftinfer_amd_gated_delta_select_policy(raftinfer_amd_delta_shape shape, size_t bucket_tokens,
                                            raftinfer_amd_delta_policy *out);
int raftinfer_amd_batched_decode_workspace_bytes(raftinfer_amd_batched_decode_shape shape,
                                                 size_t *out);

/* ---- enqueue ---- */
/* qwen35_attention.cuh:38-45 (qwen35_causal_attention with a policy). */
int raftinfer_amd_causal_attention(const void *query, const void *key, const void *value,
                                   const void *gate, void *output, void *kv_cache,
                                   size_t kv_cache_bytes, void *workspace, size_t workspace_bytes,
                                   raftinfer_amd_attention_shape shape, int activation_dtype,
                                   raftinfer_amd_attention_policy policy, void *stream);
/* qwen35_attention.cuh:47-51 (materialized convenience overload). */
int raftinfer_amd_causal_attention_materialized(const void *query, const void *key,
                                                const void *value, const void *gate, void *output,
                                                float *kv_cache, float *logits_workspace,
                                                size_t logits_workspace_floats,
                                                raftinfer_amd_attention_shape shape, int dtype,
                                                void *stream);
/* qwen35_online_attention.cuh:47-52 */
int raftinfer_amd_online_attention_prefill(const void *query, const void *key, const void *value,
                                           const void *gate, void *output, void *kv_cache,
                                           size_t kv_cache_bytes,
                                           raftinfer_amd_attention_shape shape,
                                           int activation_dtype, uint8_t cache_dtype,
                                           uint8_t cache_layout, void *stream);
/* qwen35_online_attention.cuh:54-61 (with plan; device_position may be null). */
int raftinfer_amd_online_attention_decode(const void *query, const void *key, const void *value,
                                          const void *gate, void *output, void *kv_cache,
                                          size_t kv_cache_bytes, void *workspace,
                                          size_t workspace_bytes,
                                          raftinfer_amd_attention_shape shape,
                                          int activation_dtype, uint8_t cache_dtype,
                                          uint8_t cache_layout, raftinfer_amd_decode_plan plan,
                                          const uint32_t *device_position, void *stream);
/* qwen35_online_attention.cuh:63-68 (single-block, no plan). */
int raftinfer_amd_online_attention_decode_single(const void *query, const void *key,
                                                 const void *value, const void *gate,
                                                 void *output, void *kv_cache,
                                                 size_t kv_cache_bytes,
                                                 raftinfer_amd_attention_shape shape,
                                                 int activation_dtype, uint8_t cache_dtype,
                                                 uint8_t cache_layout,
                                                 const uint32_t *device_position, void *stream);
/* Additive: batched ragged decode; see qwen35_online_attention.hpp. */
int raftinfer_amd_online_attention_decode_batched(
    const void *query, const void *key, const void *value, const void *gate, void *output,
    void *kv_cache, size_t kv_cache_bytes, const uint32_t *context_lengths, void *workspace,
    size_t workspace_bytes, raftinfer_amd_batched_decode_shape shape, int activation_dtype,
    void *stream);
/* Producers fused into the attention (additive; see qwen35_online_attention.hpp):
 * q / gate split + RMSNorm + partial RoPE of q and k done inside the attention
 * kernels, bit-identical to qwen35_split_query_gate_norm_rope /
 * qwen35_qk_norm_rope followed by the unfused call. */
typedef struct raftinfer_amd_fused_norm_rope {
  const void *query_norm_weight, *key_norm_weight;
  int weight_dtype; /* RAFTINFER_AMD_DTYPE_BF16 or _F32 */
  size_t rotary_dim;
  float rope_base, epsilon;
} raftinfer_amd_fused_norm_rope;
int raftinfer_amd_online_attention_decode_fused(
    const void *query_gate, const void *key, const void *value, void *output, void *kv_cache,
    size_t kv_cache_bytes, void *workspace, size_t workspace_bytes,
    raftinfer_amd_attention_shape shape, raftinfer_amd_fused_norm_rope norm, uint8_t cache_dtype,
    uint8_t cache_layout, raftinfer_amd_decode_plan plan, const uint32_t *device_position,
    void *stream);

int raftinfer_amd_online_attention_prefill_fused(
    const void *query_gate, const void *key, const void *value, void *output, void *kv_cache,
    size_t kv_cache_bytes, raftinfer_amd_attention_shape shape, raftinfer_amd_fused_norm_rope norm,
    uint8_t cache_dtype, uint8_t cache_layout, void *stream);

/* Allocation-free decode.  No counterpart in the reference: for callers that
 * cannot allocate device memory (HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  As raftinfer_amd_online_attention_decode
 * with a plan, but the split-K workspace is a library-owned static device
 * array of raftinfer_amd_online_attention_static_workspace_bytes() bytes per
 * GPU (8,454,144: max_context_tokens <= 131072 at split_k_256, <= 262144 at
 * split_k_512); larger plans return RAFTINFER_AMD_INVALID_ARGUMENT.  Calls
 * that overlap on one GPU share that array and race.  The first call on each
 * device looks up the array's address and must not be under stream capture
 * (it returns RAFTINFER_AMD_INVALID_ARGUMENT there); later calls may be
 * captured. */
size_t raftinfer_amd_online_attention_static_workspace_bytes(void);
int raftinfer_amd_online_attention_decode_static_workspace(
    const void *query, const void *key, const void *value, const void *gate, void *output,
    void *kv_cache, size_t kv_cache_bytes, raftinfer_amd_attention_shape shape,
    int activation_dtype, uint8_t cache_dtype, uint8_t cache_layout,
    raftinfer_amd_decode_plan plan, const uint32_t *device_position, void *stream);
/* Measurement entry points (no reference counterpart): validate like the
 * calls above, then enqueue only the dominant kernel (the split-K partition
 * kernel; the prefill attention kernel without the K/V append). */
int raftinfer_amd_online_attention_decode_partition_only(
    const void *query, const void *key, const void *value, const void *gate, void *output,
    void *kv_cache, size_t kv_cache_bytes, void *workspace, size_t workspace_bytes,
    raftinfer_amd_attention_shape shape, int activation_dtype, uint8_t cache_dtype,
    uint8_t cache_layout, raftinfer_amd_decode_plan plan, const uint32_t *device_position,
    void *stream);
int raftinfer_amd_online_attention_prefill_kernel_only(
    const void *query, const void *key, const void *value, const void *gate, void *output,
    void *kv_cache, size_t kv_cache_bytes, raftinfer_amd_attention_shape shape,
    int activation_dtype, uint8_t cache_dtype, uint8_t cache_layout, void *stream);
/* Device capacity-guard counter (replaces the reference merge kernel's trap,
 * qwen35_online_attention.cu:714-717); also counts batched-decode sequences
 * whose length is 0 or above the maximum context.  Synchronizes the device. */
int raftinfer_amd_consume_capacity_errors(uint32_t *out);

/* ---- decode graphs (include/raftinfer_amd/hip_graph_decode.hpp) ---- */
/* Buffers of one decode-attention step (qwen35_executor.cu:2027-2057). */
typedef struct raftinfer_amd_decode_buffers {
  const void *query, *key, *value, *gate;
  void *output, *kv_cache;
  size_t kv_cache_bytes;
  void *workspace;
  size_t workspace_bytes;
  const uint32_t *device_position;
} raftinfer_amd_decode_buffers;
/* Captures one decode-attention graph per context-bucket plan, as
 * qwen35_executor.cu:2191-2226 builds its variants (CudaGraphDecode,
 * cuda_graph_decode.cu:20-61, on hipGraph).  Writes an opaque handle. */
int raftinfer_amd_decode_graphs_create(int device_id, void *stream,
                                       raftinfer_amd_attention_shape shape, uint8_t mode,
                                       int activation_dtype, uint8_t cache_dtype,
                                       uint8_t cache_layout, raftinfer_amd_decode_buffers buffers,
                                       void **out_handle);
int raftinfer_amd_decode_graphs_variant_count(void *handle, size_t *out);
int raftinfer_amd_decode_graphs_variant_for(void *handle, size_t position, size_t *out);
/* Replays the step of `position`; *device_position must already equal it on the stream. */
int raftinfer_amd_decode_graphs_replay(void *handle, size_t position);
void raftinfer_amd_decode_graphs_destroy(void *handle);

/* qwen35_delta.cuh:96-102 (qwen35_gated_delta with a policy). */
int raftinfer_amd_gated_delta(const void *input, const void *conv_weight, const void *recurrent_a,
                              const void *dt_bias, const void *output_norm_weight, void *output,
                              float *convolution_state, float *recurrent_state, void *workspace,
                              size_t workspace_bytes, raftinfer_amd_delta_shape shape,
                              raftinfer_amd_delta_policy policy, int dtype, int weight_dtype,
                              void *stream);
/* qwen35_delta.cuh:88-94 (policy chosen by qwen35_gated_delta_select_policy). */
int raftinfer_amd_gated_delta_auto(const void *input, const void *conv_weight,
                                   const void *recurrent_a, const void *dt_bias,
                                   const void *output_norm_weight, void *output,
                                   float *convolution_state, float *recurrent_state,
                                   void *workspace, size_t workspace_bytes,
                                   raftinfer_amd_delta_shape shape, int dtype, int weight_dtype,
                                   void *stream);
/* Additive: qwen35_pack_linear_delta_input (qwen35_primitives.cu:388-420)
 * fused into qwen35_gated_delta; the four projection outputs are read in place
 * (see qwen35_delta.hpp). */
int raftinfer_amd_gated_delta_unpacked(const void *qkv, const void *beta, const void *alpha,
                                       const void *gate, const void *conv_weight,
                                       const void *recurrent_a, const void *dt_bias,
                                       const void *output_norm_weight, void *output,
                                       float *convolution_state, float *recurrent_state,
                                       void *workspace, size_t workspace_bytes,
                                       raftinfer_amd_delta_shape shape,
                                       raftinfer_amd_delta_policy policy, int dtype,
                                       int weight_dtype, void *stream);
/* Additive: the recurrence alone; see qwen35_delta.hpp. */
int raftinfer_amd_gated_delta_core_workspace_bytes(raftinfer_amd_delta_core_shape shape,
                                                   size_t *out);
int raftinfer_amd_gated_delta_core(const void *q, const void *k, const void *v, const float *beta,
                                   const float *log_decay, float q_scale, float *state,
                                   void *output, void *workspace, size_t workspace_bytes,
                                   raftinfer_amd_delta_core_shape shape, int chunked,
                                   void *stream);

/* ---- attention producers ---- */
/* qwen35_primitives.cuh:63-67 (qwen35_qk_norm_rope; device_position may be null). */
int raftinfer_amd_qk_norm_rope(const void *input, const void *weight, void *output,
                               raftinfer_amd_qk_norm_rope_shape shape, float epsilon, int dtype,
                               int weight_dtype, void *stream, const uint32_t *device_position);
/* qwen35_primitives.cuh:93-96 (qwen35_split_full_query_gate). */
int raftinfer_amd_split_full_query_gate(const void *query_gate, void *query, void *gate,
                                        size_t tokens, size_t heads, size_t head_dim, int dtype,
                                        void *stream);
/* qwen35_primitives.cuh:98-102 (qwen35_pack_linear_delta_input). */
int raftinfer_amd_pack_linear_delta_input(const void *qkv, const void *beta, const void *alpha,
                                          const void *gate, void *packed, size_t tokens,
                                          size_t qkv_width, size_t beta_width, size_t alpha_width,
                                          size_t gate_width, int dtype, void *stream);
/* Additive: the split and the query's norm + RoPE in one pass. */
int raftinfer_amd_split_query_gate_norm_rope(const void *query_gate, const void *weight,
                                             void *query, void *gate,
                                             raftinfer_amd_qk_norm_rope_shape shape, float epsilon,
                                             int dtype, int weight_dtype, void *stream,
                                             const uint32_t *device_position);

#ifdef __cplusplus
}
#endif
#endif
