// extern "C" layer over the C++ drop-in boundary.  Exceptions never cross the
// ABI: validation errors map to RAFTINFER_AMD_INVALID_ARGUMENT, launch errors
// to RAFTINFER_AMD_LAUNCH_FAILED, with the message kept per thread (the
// convention of the reference's cpp/src/c_api.cpp:44, :173-175).
#include "raftinfer_amd.h"

#include "raftinfer_amd/hip_graph_decode.hpp"
#include "raftinfer_amd/qwen35_delta.hpp"
#include "raftinfer_amd/qwen35_online_attention.hpp"
#include "raftinfer_amd/qwen35_primitives.hpp"

#include <cstring>
#include <exception>
#include <string>

namespace {

using namespace raftinfer;
using namespace raftinfer::kernels;

thread_local std::string g_last_error;

template <typename Fn> int guarded(Fn &&fn) {
  try {
    fn();
    g_last_error.clear();
    return RAFTINFER_AMD_OK;
  } catch (const Qwen35PrimitiveError &e) {
    g_last_error = e.what();
  } catch (const Qwen35DeltaError &e) {
    g_last_error = e.what();
  } catch (const std::exception &e) {
    g_last_error = e.what();
    return RAFTINFER_AMD_INTERNAL_ERROR;
  } catch (...) {
    g_last_error = "unknown error";
    return RAFTINFER_AMD_INTERNAL_ERROR;
  }
  return g_last_error.find("launch failed") != std::string::npos ? RAFTINFER_AMD_LAUNCH_FAILED
                                                                  : RAFTINFER_AMD_INVALID_ARGUMENT;
}

Qwen35AttentionShape to_shape(raftinfer_amd_attention_shape s) {
  return {s.tokens, s.query_heads, s.kv_heads, s.head_dim, s.max_context_tokens, s.past_tokens};
}
Qwen35AttentionLaunchPolicy to_policy(raftinfer_amd_attention_policy p) {
  return {static_cast<Qwen35AttentionImplementation>(p.implementation),
          static_cast<Qwen35KvCacheDType>(p.kv_cache_dtype),
          static_cast<Qwen35KvCacheLayout>(p.kv_cache_layout)};
}
Qwen35OnlineDecodePlan to_plan(raftinfer_amd_decode_plan p) {
  return {static_cast<Qwen35DecodeAttentionMode>(p.resolved_mode), p.partition_tokens,
          p.split_k_threshold_tokens, p.context_bucket_tokens, p.active_partition_capacity};
}
GatedDeltaShape to_delta(raftinfer_amd_delta_shape s) {
  return {s.tokens, s.hidden_size, s.key_heads, s.value_heads,
          s.key_dim, s.value_dim, s.conv_width, s.epsilon};
}
GatedDeltaLaunchPolicy to_delta_policy(raftinfer_amd_delta_policy p) {
  return {static_cast<GatedDeltaSchedule>(p.schedule), p.warps_per_block,
          p.transposed_boundary_state != 0};
}
hipStream_t to_stream(void *s) { return static_cast<hipStream_t>(s); }
// The result of a sizing / planning call is written through a caller pointer;
// a null one is an invalid argument, not a crash.
template <typename T> T &out_ref(T *p) {
  if (p == nullptr) throw Qwen35PrimitiveError("raftinfer_amd result pointer is null");
  return *p;
}
RaftInferDataType to_dtype(int d) { return static_cast<RaftInferDataType>(d); }
Qwen35FusedNormRope to_norm(raftinfer_amd_fused_norm_rope n) {
  return {n.query_norm_weight, n.key_norm_weight, static_cast<RaftInferDataType>(n.weight_dtype),
          n.rotary_dim, n.rope_base, n.epsilon};
}

} // namespace

extern "C" {

const char *raftinfer_amd_last_error_message(void) { return g_last_error.c_str(); }

int raftinfer_amd_attention_workspace_floats(raftinfer_amd_attention_shape shape, size_t *out) {
  return guarded([&] { out_ref(out) = qwen35_attention_workspace_floats(to_shape(shape)); });
}

int raftinfer_amd_attention_cache_bytes(raftinfer_amd_attention_shape shape,
                                        raftinfer_amd_attention_policy policy, size_t *out) {
  return guarded([&] { out_ref(out) = qwen35_attention_cache_bytes(to_shape(shape), to_policy(policy)); });
}

int raftinfer_amd_attention_workspace_bytes(raftinfer_amd_attention_shape shape,
                                            raftinfer_amd_attention_policy policy, size_t *out) {
  return guarded(
      [&] { out_ref(out) = qwen35_attention_workspace_bytes(to_shape(shape), to_policy(policy)); });
}

int raftinfer_amd_online_decode_plan(raftinfer_amd_attention_shape shape, uint8_t requested,
                                     size_t context_tokens, raftinfer_amd_decode_plan *out) {
  return guarded([&] {
    const auto p = qwen35_online_decode_plan(
        to_shape(shape), static_cast<Qwen35DecodeAttentionMode>(requested), context_tokens);
    out_ref(out) = {static_cast<uint8_t>(p.resolved_mode), p.partition_tokens,
            p.split_k_threshold_tokens, p.context_bucket_tokens, p.active_partition_capacity};
  });
}

int raftinfer_amd_online_decode_workspace_layout(raftinfer_amd_attention_shape shape,
                                                 uint8_t resolved, raftinfer_amd_decode_layout *out) {
  return guarded([&] {
    const auto l = qwen35_online_decode_workspace_layout(
        to_shape(shape), static_cast<Qwen35DecodeAttentionMode>(resolved));
    out_ref(out) = {l.partial_count, l.max_offset_bytes, l.sum_offset_bytes, l.value_offset_bytes, l.bytes};
  });
}

int raftinfer_amd_online_attention_prefill_supported(raftinfer_amd_attention_shape shape,
                                                     int act, raftinfer_amd_attention_policy policy) {
  return qwen35_online_attention_prefill_supported(to_shape(shape), to_dtype(act), to_policy(policy))
             ? 1
             : 0;
}

int raftinfer_amd_gated_delta_workspace_bytes(raftinfer_amd_delta_shape shape, size_t *out) {
  return guarded([&] { out_ref(out) = qwen35_gated_delta_workspace_bytes(to_delta(shape)); });
}

int raftinfer_amd_gated_delta_select_policy(raftinfer_amd_delta_shape shape, size_t bucket,
                                            raftinfer_amd_delta_policy *out) {
  return guarded([&] {
    const auto p = qwen35_gated_delta_select_policy(to_delta(shape), bucket);
    out_ref(out) = {static_cast<uint8_t>(p.schedule), p.warps_per_block,
            static_cast<uint8_t>(p.transposed_boundary_state)};
  });
}

int raftinfer_amd_batched_decode_workspace_bytes(raftinfer_amd_batched_decode_shape s, size_t *out) {
  return guarded([&] {
    out_ref(out) = qwen35_batched_decode_workspace_bytes(
        {s.sequences, s.max_context_tokens, s.cache_stride_bytes, s.single_block_max_tokens});
  });
}

int raftinfer_amd_causal_attention(const void *q, const void *k, const void *v, const void *g,
                                   void *o, void *cache, size_t cache_bytes, void *ws,
                                   size_t ws_bytes, raftinfer_amd_attention_shape shape, int act,
                                   raftinfer_amd_attention_policy policy, void *stream) {
  return guarded([&] {
    qwen35_causal_attention(q, k, v, g, o, cache, cache_bytes, ws, ws_bytes, to_shape(shape),
                            to_dtype(act), to_policy(policy), to_stream(stream));
  });
}

int raftinfer_amd_causal_attention_materialized(const void *q, const void *k, const void *v,
                                                const void *g, void *o, float *cache,
                                                float *logits, size_t logits_floats,
                                                raftinfer_amd_attention_shape shape, int dtype,
                                                void *stream) {
  return guarded([&] {
    qwen35_causal_attention(q, k, v, g, o, cache, logits, logits_floats, to_shape(shape),
                            to_dtype(dtype), to_stream(stream));
  });
}

int raftinfer_amd_online_attention_prefill(const void *q, const void *k, const void *v,
                                           const void *g, void *o, void *cache, size_t cache_bytes,
                                           raftinfer_amd_attention_shape shape, int act,
                                           uint8_t cache_dtype, uint8_t cache_layout, void *stream) {
  return guarded([&] {
    qwen35_online_attention_prefill(q, k, v, g, o, cache, cache_bytes, to_shape(shape),
                                    to_dtype(act), static_cast<Qwen35KvCacheDType>(cache_dtype),
                                    static_cast<Qwen35KvCacheLayout>(cache_layout),
                                    to_stream(stream));
  });
}

int raftinfer_amd_online_attention_decode(const void *q, const void *k, const void *v,
                                          const void *g, void *o, void *cache, size_t cache_bytes,
                                          void *ws, size_t ws_bytes,
                                          raftinfer_amd_attention_shape shape, int act,
                                          uint8_t cache_dtype, uint8_t cache_layout,
                                          raftinfer_amd_decode_plan plan,
                                          const uint32_t *device_position, void *stream) {
  return guarded([&] {
    qwen35_online_attention_decode(q, k, v, g, o, cache, cache_bytes, ws, ws_bytes,
                                   to_shape(shape), to_dtype(act),
                                   static_cast<Qwen35KvCacheDType>(cache_dtype),
                                   static_cast<Qwen35KvCacheLayout>(cache_layout), to_plan(plan),
                                   device_position, to_stream(stream));
  });
}

int raftinfer_amd_online_attention_decode_single(const void *q, const void *k, const void *v,
                                                 const void *g, void *o, void *cache,
                                                 size_t cache_bytes,
                                                 raftinfer_amd_attention_shape shape, int act,
                                                 uint8_t cache_dtype, uint8_t cache_layout,
                                                 const uint32_t *device_position, void *stream) {
  return guarded([&] {
    qwen35_online_attention_decode(q, k, v, g, o, cache, cache_bytes, to_shape(shape),
                                   to_dtype(act), static_cast<Qwen35KvCacheDType>(cache_dtype),
                                   static_cast<Qwen35KvCacheLayout>(cache_layout), device_position,
                                   to_stream(stream));
  });
}

int raftinfer_amd_online_attention_decode_batched(const void *q, const void *k, const void *v,
                                                  const void *g, void *o, void *cache,
                                                  size_t cache_bytes, const uint32_t *lengths,
                                                  void *ws, size_t ws_bytes,
                                                  raftinfer_amd_batched_decode_shape s, int act,
                                                  void *stream) {
  return guarded([&] {
    qwen35_online_attention_decode_batched(
        q, k, v, g, o, cache, cache_bytes, lengths, ws, ws_bytes,
        {s.sequences, s.max_context_tokens, s.cache_stride_bytes, s.single_block_max_tokens},
        to_dtype(act), to_stream(stream));
  });
}

int raftinfer_amd_online_attention_decode_partition_only(
    const void *q, const void *k, const void *v, const void *g, void *o, void *cache,
    size_t cache_bytes, void *ws, size_t ws_bytes, raftinfer_amd_attention_shape shape, int act,
    uint8_t cache_dtype, uint8_t cache_layout, raftinfer_amd_decode_plan plan,
    const uint32_t *device_position, void *stream) {
  return guarded([&] {
    qwen35_online_attention_decode_partition_only(
        q, k, v, g, o, cache, cache_bytes, ws, ws_bytes, to_shape(shape), to_dtype(act),
        static_cast<Qwen35KvCacheDType>(cache_dtype), static_cast<Qwen35KvCacheLayout>(cache_layout),
        to_plan(plan), device_position, to_stream(stream));
  });
}

int raftinfer_amd_online_attention_decode_fused(
    const void *qg, const void *k, const void *v, void *o, void *cache, size_t cache_bytes, void *ws,
    size_t ws_bytes, raftinfer_amd_attention_shape shape, raftinfer_amd_fused_norm_rope norm,
    uint8_t cache_dtype, uint8_t cache_layout, raftinfer_amd_decode_plan plan,
    const uint32_t *device_position, void *stream) {
  return guarded([&] {
    qwen35_online_attention_decode_fused(
        qg, k, v, o, cache, cache_bytes, ws, ws_bytes, to_shape(shape), to_norm(norm),
        static_cast<Qwen35KvCacheDType>(cache_dtype), static_cast<Qwen35KvCacheLayout>(cache_layout),
        to_plan(plan), device_position, to_stream(stream));
  });
}

int raftinfer_amd_online_attention_prefill_fused(
    const void *qg, const void *k, const void *v, void *o, void *cache, size_t cache_bytes,
    raftinfer_amd_attention_shape shape, raftinfer_amd_fused_norm_rope norm, uint8_t cache_dtype,
    uint8_t cache_layout, void *stream) {
  return guarded([&] {
    qwen35_online_attention_prefill_fused(
        qg, k, v, o, cache, cache_bytes, to_shape(shape), to_norm(norm),
        static_cast<Qwen35KvCacheDType>(cache_dtype), static_cast<Qwen35KvCacheLayout>(cache_layout),
        to_stream(stream));
  });
}

size_t raftinfer_amd_online_attention_static_workspace_bytes(void) {
  return qwen35_online_attention_static_workspace_bytes();
}

int raftinfer_amd_online_attention_decode_static_workspace(
    const void *q, const void *k, const void *v, const void *g, void *o, void *cache,
    size_t cache_bytes, raftinfer_amd_attention_shape shape, int act, uint8_t cache_dtype,
    uint8_t cache_layout, raftinfer_amd_decode_plan plan, const uint32_t *device_position,
    void *stream) {
  return guarded([&] {
    qwen35_online_attention_decode_static_workspace(
        q, k, v, g, o, cache, cache_bytes, to_shape(shape), to_dtype(act),
        static_cast<Qwen35KvCacheDType>(cache_dtype), static_cast<Qwen35KvCacheLayout>(cache_layout),
        to_plan(plan), device_position, to_stream(stream));
  });
}

int raftinfer_amd_online_attention_prefill_kernel_only(
    const void *q, const void *k, const void *v, const void *g, void *o, void *cache,
    size_t cache_bytes, raftinfer_amd_attention_shape shape, int act, uint8_t cache_dtype,
    uint8_t cache_layout, void *stream) {
  return guarded([&] {
    qwen35_online_attention_prefill_kernel_only(
        q, k, v, g, o, cache, cache_bytes, to_shape(shape), to_dtype(act),
        static_cast<Qwen35KvCacheDType>(cache_dtype), static_cast<Qwen35KvCacheLayout>(cache_layout),
        to_stream(stream));
  });
}

int raftinfer_amd_decode_graphs_create(int device_id, void *stream,
                                       raftinfer_amd_attention_shape shape, uint8_t mode, int act,
                                       uint8_t cache_dtype, uint8_t cache_layout,
                                       raftinfer_amd_decode_buffers b, void **out_handle) {
  return guarded([&] {
    auto &handle = out_ref(out_handle);
    handle = new Qwen35DecodeAttentionGraphs(
        device_id, to_stream(stream), to_shape(shape), static_cast<Qwen35DecodeAttentionMode>(mode),
        to_dtype(act), static_cast<Qwen35KvCacheDType>(cache_dtype),
        static_cast<Qwen35KvCacheLayout>(cache_layout),
        Qwen35DecodeAttentionBuffers{b.query, b.key, b.value, b.gate, b.output, b.kv_cache,
                                     b.kv_cache_bytes, b.workspace, b.workspace_bytes,
                                     b.device_position});
  });
}

int raftinfer_amd_decode_graphs_variant_count(void *handle, size_t *out) {
  return guarded([&] {
    if (handle == nullptr) throw Qwen35PrimitiveError("decode graph handle is null");
    out_ref(out) = static_cast<Qwen35DecodeAttentionGraphs *>(handle)->variant_count();
  });
}

int raftinfer_amd_decode_graphs_variant_for(void *handle, size_t position, size_t *out) {
  return guarded([&] {
    if (handle == nullptr) throw Qwen35PrimitiveError("decode graph handle is null");
    out_ref(out) = static_cast<Qwen35DecodeAttentionGraphs *>(handle)->variant_for(position);
  });
}

int raftinfer_amd_decode_graphs_replay(void *handle, size_t position) {
  return guarded([&] {
    if (handle == nullptr) throw Qwen35PrimitiveError("decode graph handle is null");
    static_cast<Qwen35DecodeAttentionGraphs *>(handle)->replay(position);
  });
}

void raftinfer_amd_decode_graphs_destroy(void *handle) {
  delete static_cast<Qwen35DecodeAttentionGraphs *>(handle);
}

int raftinfer_amd_consume_capacity_errors(uint32_t *out) {
  return guarded([&] { out_ref(out) = qwen35_online_attention_consume_capacity_errors(); });
}

int raftinfer_amd_gated_delta(const void *input, const void *conv_weight, const void *a,
                              const void *dt_bias, const void *norm_w, void *output,
                              float *conv_state, float *rec_state, void *ws, size_t ws_bytes,
                              raftinfer_amd_delta_shape shape, raftinfer_amd_delta_policy policy,
                              int dtype, int weight_dtype, void *stream) {
  return guarded([&] {
    qwen35_gated_delta(input, conv_weight, a, dt_bias, norm_w, output, conv_state, rec_state, ws,
                       ws_bytes, to_delta(shape), to_delta_policy(policy), to_dtype(dtype),
                       to_dtype(weight_dtype), to_stream(stream));
  });
}

int raftinfer_amd_gated_delta_auto(const void *input, const void *conv_weight, const void *a,
                                   const void *dt_bias, const void *norm_w, void *output,
                                   float *conv_state, float *rec_state, void *ws, size_t ws_bytes,
                                   raftinfer_amd_delta_shape shape, int dtype, int weight_dtype,
                                   void *stream) {
  return guarded([&] {
    qwen35_gated_delta(input, conv_weight, a, dt_bias, norm_w, output, conv_state, rec_state, ws,
                       ws_bytes, to_delta(shape), to_dtype(dtype), to_dtype(weight_dtype),
                       to_stream(stream));
  });
}

int raftinfer_amd_gated_delta_unpacked(const void *qkv, const void *beta, const void *alpha,
                                       const void *gate, const void *conv_weight,
                                       const void *recurrent_a, const void *dt_bias,
                                       const void *norm_w, void *output, float *conv_state,
                                       float *rec_state, void *workspace, size_t workspace_bytes,
                                       raftinfer_amd_delta_shape shape,
                                       raftinfer_amd_delta_policy policy, int dtype,
                                       int weight_dtype, void *stream) {
  return guarded([&] {
    qwen35_gated_delta_unpacked(qkv, beta, alpha, gate, conv_weight, recurrent_a, dt_bias, norm_w,
                                output, conv_state, rec_state, workspace, workspace_bytes,
                                to_delta(shape), to_delta_policy(policy), to_dtype(dtype),
                                to_dtype(weight_dtype), to_stream(stream));
  });
}

int raftinfer_amd_gated_delta_core_workspace_bytes(raftinfer_amd_delta_core_shape s, size_t *out) {
  return guarded([&] {
    out_ref(out) = qwen35_gated_delta_core_workspace_bytes(
        {s.tokens, s.key_heads, s.value_heads, s.key_dim, s.value_dim});
  });
}

int raftinfer_amd_gated_delta_core(const void *q, const void *k, const void *v, const float *beta,
                                   const float *log_decay, float q_scale, float *state, void *out,
                                   void *ws, size_t ws_bytes, raftinfer_amd_delta_core_shape s,
                                   int chunked, void *stream) {
  return guarded([&] {
    qwen35_gated_delta_core(q, k, v, beta, log_decay, q_scale, state, out, ws, ws_bytes,
                            {s.tokens, s.key_heads, s.value_heads, s.key_dim, s.value_dim},
                            chunked != 0, to_stream(stream));
  });
}

int raftinfer_amd_qk_norm_rope(const void *input, const void *weight, void *output,
                               raftinfer_amd_qk_norm_rope_shape s, float epsilon, int dtype,
                               int weight_dtype, void *stream, const uint32_t *device_position) {
  return guarded([&] {
    qwen35_qk_norm_rope(input, weight, output,
                        {s.tokens, s.heads, s.head_dim, s.rotary_dim, s.position_offset, s.rope_base},
                        epsilon, static_cast<RaftInferDataType>(dtype),
                        static_cast<RaftInferDataType>(weight_dtype), to_stream(stream),
                        device_position);
  });
}

int raftinfer_amd_split_full_query_gate(const void *query_gate, void *query, void *gate,
                                        size_t tokens, size_t heads, size_t head_dim, int dtype,
                                        void *stream) {
  return guarded([&] {
    qwen35_split_full_query_gate(query_gate, query, gate, tokens, heads, head_dim,
                                 static_cast<RaftInferDataType>(dtype), to_stream(stream));
  });
}

int raftinfer_amd_pack_linear_delta_input(const void *qkv, const void *beta, const void *alpha,
                                          const void *gate, void *packed, size_t tokens,
                                          size_t qkv_width, size_t beta_width, size_t alpha_width,
                                          size_t gate_width, int dtype, void *stream) {
  return guarded([&] {
    qwen35_pack_linear_delta_input(qkv, beta, alpha, gate, packed, tokens, qkv_width, beta_width,
                                   alpha_width, gate_width, static_cast<RaftInferDataType>(dtype),
                                   to_stream(stream));
  });
}

int raftinfer_amd_split_query_gate_norm_rope(const void *query_gate, const void *weight,
                                             void *query, void *gate,
                                             raftinfer_amd_qk_norm_rope_shape s, float epsilon,
                                             int dtype, int weight_dtype, void *stream,
                                             const uint32_t *device_position) {
  return guarded([&] {
    qwen35_split_query_gate_norm_rope(
        query_gate, weight, query, gate,
        {s.tokens, s.heads, s.head_dim, s.rotary_dim, s.position_offset, s.rope_base}, epsilon,
        static_cast<RaftInferDataType>(dtype), static_cast<RaftInferDataType>(weight_dtype),
        to_stream(stream), device_position);
  });
}

} // extern "C"
