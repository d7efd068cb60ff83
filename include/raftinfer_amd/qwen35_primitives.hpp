// The attention producers of cpp/kernels/qwen35_primitives.cuh (lines 15-19,
// 34-41, 63-67, 93-96) for gfx950, with hipStream_t in place of cudaStream_t:
// the query/gate split of the q projection and the per-head RMSNorm + partial
// RoPE of q and k, the steps right before the attention kernels
// (cpp/execution/qwen35_executor.cu:1989-2013).  Validation failures throw
// Qwen35PrimitiveError before any launch.  Nothing allocates or synchronizes.
#pragma once

#include "tensor.h"

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

namespace raftinfer::kernels {

// cpp/kernels/qwen35_primitives.cuh:15-19
class Qwen35PrimitiveError : public std::runtime_error {
public:
  explicit Qwen35PrimitiveError(const std::string &message) : std::runtime_error(message) {}
};

// cpp/kernels/qwen35_primitives.cuh:34-41
struct QkNormRopeShape {
  std::size_t tokens;
  std::size_t heads;
  std::size_t head_dim;
  std::size_t rotary_dim;
  std::size_t position_offset;
  float rope_base;
};

// cpp/kernels/qwen35_primitives.cuh:63-67.  input, output: [tokens][heads][head_dim];
// weight: [head_dim].  Position of token t: (*device_position or
// position_offset) + t.
void qwen35_qk_norm_rope(const void *input, const void *weight, void *output,
                         QkNormRopeShape shape, float epsilon, RaftInferDataType dtype,
                         RaftInferDataType weight_dtype, hipStream_t stream,
                         const std::uint32_t *device_position = nullptr);

// cpp/kernels/qwen35_primitives.cuh:93-96.  query_gate: [tokens][heads][2][head_dim]
// -> query, gate: [tokens][heads][head_dim].
void qwen35_split_full_query_gate(const void *query_gate, void *query, void *gate,
                                  std::size_t tokens, std::size_t heads, std::size_t head_dim,
                                  RaftInferDataType dtype, hipStream_t stream);

// cpp/kernels/qwen35_primitives.cuh:98-102.  Each source [tokens][width];
// packed [tokens][qkv | beta | alpha | gate], the input rows of qwen35_gated_delta.
void qwen35_pack_linear_delta_input(const void *qkv, const void *beta, const void *alpha,
                                    const void *gate, void *packed, std::size_t tokens,
                                    std::size_t qkv_width, std::size_t beta_width,
                                    std::size_t alpha_width, std::size_t gate_width,
                                    RaftInferDataType dtype, hipStream_t stream);

// Additive (no counterpart in the reference): both steps in one pass over the
// q projection, query_gate -> RMSNorm + RoPE'd query and gate, equal to
// qwen35_split_full_query_gate followed by qwen35_qk_norm_rope on the query.
void qwen35_split_query_gate_norm_rope(const void *query_gate, const void *weight, void *query,
                                       void *gate, QkNormRopeShape shape, float epsilon,
                                       RaftInferDataType dtype, RaftInferDataType weight_dtype,
                                       hipStream_t stream,
                                       const std::uint32_t *device_position = nullptr);

} // namespace raftinfer::kernels
