// Gated DeltaNet entry points for gfx950.  Mirrors the reference's
// cpp/kernels/qwen35_delta.cuh:14-102 with hipStream_t; adds a chunked
// prefill schedule and a core-only entry.
#pragma once

#include "tensor.h"

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

namespace raftinfer::kernels {

class Qwen35DeltaError : public std::runtime_error {
public:
  explicit Qwen35DeltaError(const std::string &message) : std::runtime_error(message) {}
};

struct GatedDeltaShape {
  std::size_t tokens;
  std::size_t hidden_size;
  std::size_t key_heads;
  std::size_t value_heads;
  std::size_t key_dim;
  std::size_t value_dim;
  std::size_t conv_width;
  float epsilon;
};

// The enumerator names are the reference's; on gfx950 the *_sm120 values
// select this build's chunked (prefill) and single-token (decode) schedules.
enum class GatedDeltaSchedule : std::uint8_t {
  register_resident_current,
  register_resident_prefill_sm120,
  register_resident_decode_sm120,
};

struct GatedDeltaLaunchPolicy {
  GatedDeltaSchedule schedule{GatedDeltaSchedule::register_resident_current};
  std::uint32_t warps_per_block{4};
  bool transposed_boundary_state{false};
};

struct GatedDeltaScheduleDiagnostic {
  std::size_t bucket_tokens{};
  std::size_t key_dim{};
  std::size_t value_dim{};
  GatedDeltaSchedule candidate_schedule{GatedDeltaSchedule::register_resident_current};
  GatedDeltaSchedule schedule{GatedDeltaSchedule::register_resident_current};
  std::uint32_t warps_per_block{};
  bool transposed_boundary_state{};
  bool candidate_accepted{};
  bool correctness_passed{};
  float current_median_ms{};
  float candidate_median_ms{};
  std::string rejection_reason;

  bool operator==(const GatedDeltaScheduleDiagnostic &) const = default;
};

std::size_t qwen35_gated_delta_workspace_bytes(const GatedDeltaShape &shape);

GatedDeltaLaunchPolicy qwen35_gated_delta_select_policy(const GatedDeltaShape &shape,
                                                        std::size_t bucket_tokens) noexcept;

GatedDeltaScheduleDiagnostic
qwen35_gated_delta_schedule_diagnostic(const GatedDeltaShape &shape,
                                       std::size_t bucket_tokens) noexcept;

void qwen35_gated_delta(const void *input, const void *conv_weight, const void *recurrent_a,
                        const void *dt_bias, const void *output_norm_weight, void *output,
                        float *convolution_state, float *recurrent_state, void *workspace,
                        std::size_t workspace_bytes, GatedDeltaShape shape,
                        RaftInferDataType dtype, RaftInferDataType weight_dtype,
                        hipStream_t stream);

void qwen35_gated_delta(const void *input, const void *conv_weight, const void *recurrent_a,
                        const void *dt_bias, const void *output_norm_weight, void *output,
                        float *convolution_state, float *recurrent_state, void *workspace,
                        std::size_t workspace_bytes, GatedDeltaShape shape,
                        GatedDeltaLaunchPolicy policy, RaftInferDataType dtype,
                        RaftInferDataType weight_dtype, hipStream_t stream);

// ---- Additive: the delta input pack fused into the layer (no counterpart in
// the reference). ----
// The same computation as qwen35_pack_linear_delta_input
// (cpp/kernels/qwen35_primitives.cu:388-420) followed by qwen35_gated_delta,
// without the packed copy: the kernels read the four projection outputs in
// place.  qkv: [tokens][2 * key_heads * key_dim + value_heads * value_dim],
// beta and alpha: [tokens][value_heads], gate: [tokens][hidden_size], all in
// the activation dtype.  Workspace, states, policy, errors and alignment rules
// are qwen35_gated_delta's, with the four pointers checked in place of input.
void qwen35_gated_delta_unpacked(const void *qkv, const void *beta, const void *alpha,
                                 const void *gate, const void *conv_weight, const void *recurrent_a,
                                 const void *dt_bias, const void *output_norm_weight, void *output,
                                 float *convolution_state, float *recurrent_state, void *workspace,
                                 std::size_t workspace_bytes, GatedDeltaShape shape,
                                 GatedDeltaLaunchPolicy policy, RaftInferDataType dtype,
                                 RaftInferDataType weight_dtype, hipStream_t stream);

// ---- Additive: the recurrence alone (no counterpart in the reference). ----
// q, k: bf16 [tokens][key_heads][key_dim] (already L2-normalised; q is
// multiplied by q_scale), v: bf16 [tokens][value_heads][value_dim],
// beta, log_decay: f32 [tokens][value_heads] (beta already a probability,
// decay = exp(log_decay)).  state: f32 [value_heads][key_dim][value_dim],
// updated in place.  out: bf16 [tokens][value_heads][value_dim] = S_t^T q_t.
// chunked selects the chunk-64 schedule (key_dim = value_dim = 128 only);
// the workspace is needed by the chunked schedule only.
struct GatedDeltaCoreShape {
  std::size_t tokens;
  std::size_t key_heads;
  std::size_t value_heads;
  std::size_t key_dim;
  std::size_t value_dim;
};
std::size_t qwen35_gated_delta_core_workspace_bytes(GatedDeltaCoreShape shape);
void qwen35_gated_delta_core(const void *q, const void *k, const void *v, const float *beta,
                             const float *log_decay, float q_scale, float *state, void *output,
                             void *workspace, std::size_t workspace_bytes,
                             GatedDeltaCoreShape shape, bool chunked, hipStream_t stream);

} // namespace raftinfer::kernels
