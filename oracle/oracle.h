/*
 * CPU oracle for the Qwen3.5 attention / gated-delta hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the
 * reference's CPU truth (cpp/reference/qwen35.cpp, cpp/reference/bf16.hpp)
 * and of the integer bookkeeping of its split-K decode path
 * (cpp/kernels/qwen35_online_attention.cu).  Only tests/, the smoke check and
 * the bench's cpu_baseline leg may load it, and only as the checker or the
 * CPU baseline.  The product library never links or calls it.
 *
 * Every function names the reference lines it follows.  How each function is
 * pinned (known-answer vectors, the HF fixture, the compiled reference in
 * oracle/_ref, closed forms) is listed in oracle/README.md; no function here is
 * left "parity unpinned".
 */
#ifndef RAFTINFER_AMD_ORACLE_H
#define RAFTINFER_AMD_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- bf16 round-to-nearest-even (cpp/reference/bf16.hpp:16-32) ---- */
uint16_t orc_f32_to_bf16(float value);
float orc_bf16_to_f32(uint16_t bits);
void orc_bf16_round_array(const float *in, float *out, size_t n);

/* ---- decode plan / workspace layout
 *      (cpp/kernels/qwen35_online_attention.cu:171-196, :1071-1143) ---- */
enum {
  ORC_MODE_AUTO = 0,
  ORC_MODE_SINGLE_BLOCK = 1,
  ORC_MODE_SPLIT_K_256 = 2,
  ORC_MODE_SPLIT_K_512 = 3
};
typedef struct {
  int resolved_mode;
  size_t partition_tokens;
  size_t split_k_threshold_tokens;
  size_t context_bucket_tokens;
  size_t active_partition_capacity;
} orc_decode_plan_t;
typedef struct {
  size_t partial_count;
  size_t max_offset_bytes;
  size_t sum_offset_bytes;
  size_t value_offset_bytes;
  size_t bytes;
} orc_decode_layout_t;
/* Return 0 on success, -1 where the reference throws. */
int orc_decode_plan(size_t tokens, size_t query_heads, size_t kv_heads,
                    size_t head_dim, size_t max_context_tokens, int requested,
                    size_t context_tokens, orc_decode_plan_t *out);
int orc_decode_workspace_layout(size_t tokens, size_t query_heads,
                                size_t kv_heads, size_t head_dim,
                                size_t max_context_tokens, int resolved_mode,
                                orc_decode_layout_t *out);

/* ---- gated causal attention core (cpp/reference/qwen35.cpp:316-370) ----
 * q, gate, out: [tokens][Hq][D]; keys, values: [past+tokens][Hkv][D].
 * Query row t sees keys 0..past+t.  Double dot products, float logits,
 * double softmax sum, float probabilities, float PV, sigmoid gate. */
void orc_attention_core(const float *q, const float *keys, const float *values,
                        const float *gate, float *out, size_t tokens,
                        size_t query_heads, size_t kv_heads, size_t head_dim,
                        size_t past_tokens);

/* Full reference block: per-head RMSNorm + partial RoPE on q/k, the core,
 * sigmoid gate and the [in,out] output projection
 * (cpp/reference/qwen35.cpp:254-382).  input: [tokens][q,k,v,gate]. */
void orc_gated_full_attention(const float *input, const float *q_norm_weight,
                              const float *k_norm_weight,
                              const float *output_weight, float *output,
                              size_t tokens, size_t hidden_size,
                              size_t query_heads, size_t kv_heads,
                              size_t head_dim, size_t rotary_dim,
                              size_t position_offset, float rope_base,
                              float epsilon);

/* ---- split-K decode partials and merge
 *      (cpp/kernels/qwen35_online_attention.cu:354-405, :602-756) ----
 * q: [Hq][D]; keys/values: [ctx][Hkv][D] as the cache holds them.
 * Writes partial max/sum/value at index qh*max_partitions + p for the
 * ceil(ctx/P) active partitions (per-token online recurrence in float). */
void orc_decode_partials(const float *q, const float *keys,
                         const float *values, size_t context_tokens,
                         size_t query_heads, size_t kv_heads, size_t head_dim,
                         size_t partition_tokens, size_t max_partitions,
                         float *partial_max, float *partial_sum,
                         float *partial_value);
/* Sequential log-sum-exp merge over the active partitions plus gate. */
void orc_decode_merge(const float *gate, const float *partial_max,
                      const float *partial_sum, const float *partial_value,
                      size_t context_tokens, size_t query_heads,
                      size_t head_dim, size_t partition_tokens,
                      size_t max_partitions, float *out);

/* ---- gated delta rule (cpp/reference/qwen35.cpp:384-549) ---- */
/* One token: input [conv_dim + 2*Hv + hidden] = [q,k,v,b,a,z]. */
void orc_gated_delta_step(const float *input, const float *conv_weight,
                          const float *recurrent_a, const float *dt_bias,
                          const float *output_norm_weight, float *output,
                          float *conv_state, float *recurrent_state,
                          size_t hidden_size, size_t key_heads,
                          size_t value_heads, size_t key_dim, size_t value_dim,
                          size_t conv_width, float epsilon);
/* Token-sequential prefill (:528-549). */
void orc_gated_delta_prefill(const float *input, const float *conv_weight,
                             const float *recurrent_a, const float *dt_bias,
                             const float *output_norm_weight, float *output,
                             float *conv_state, float *recurrent_state,
                             size_t tokens, size_t hidden_size,
                             size_t key_heads, size_t value_heads,
                             size_t key_dim, size_t value_dim,
                             size_t conv_width, float epsilon);
/* The recurrence alone (:459-518), for already-convolved, normalised q/k:
 * q,k: [T][Hk][dk]; v: [T][Hv][dv]; beta, log_decay: [T][Hv].
 * decay = expf(log_decay); q is multiplied by q_scale first.
 * state: [Hv][dk][dv]; raw_out: [T][Hv][dv]. */
void orc_delta_core(const float *q, const float *k, const float *v,
                    const float *beta, const float *log_decay, float q_scale,
                    float *state, float *raw_out, size_t tokens,
                    size_t key_heads, size_t value_heads, size_t key_dim,
                    size_t value_dim);

/* ---- metrics (cpp/reference/correctness.cpp:18-78) ----
 * out[0]=max_abs, out[1]=max_rel, out[2]=cosine, out[3]=nonfinite mismatches,
 * out[4]=relative L2 = ||a-b||2/||b||2 (not defined by the reference). */
/* ---- attention producers (the step before the attention kernels) ---- */
/* Per (token, head) vector of head_dim: RMSNorm with weight (qwen35.cpp:125-148,
 * weight base 0), then NeoX partial RoPE at position position_offset + token
 * (qwen35.cpp:169-186): the q/k processing of qwen35.cpp:297-312, computed by
 * the kernel qwen35_qk_norm_rope (cpp/kernels/qwen35_primitives.cu:158-210). */
void orc_qk_norm_rope(const float *input, const float *weight, float *output,
                      size_t tokens, size_t heads, size_t head_dim,
                      size_t rotary_dim, size_t position_offset,
                      float rope_base, float epsilon);
/* [tokens][heads][2][head_dim] -> query, gate [tokens][heads][head_dim]
 * (cpp/kernels/qwen35_primitives.cu:366-386). */
void orc_split_full_query_gate(const float *query_gate, float *query,
                               float *gate, size_t tokens, size_t heads,
                               size_t head_dim);

/* Row concatenation [qkv | beta | alpha | gate] per token
 * (cpp/kernels/qwen35_primitives.cu:388-420). */
void orc_pack_linear_delta_input(const float *qkv, const float *beta,
                                 const float *alpha, const float *gate,
                                 float *packed, size_t tokens, size_t qkv_width,
                                 size_t beta_width, size_t alpha_width,
                                 size_t gate_width);

void orc_compare(const float *candidate, const float *reference, size_t n,
                 double relative_floor, double *out);

#ifdef __cplusplus
}
#endif
#endif
