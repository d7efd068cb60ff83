// HIP-graph decode capture for gfx950.
//
// HipGraphDecode mirrors the reference's CudaGraphDecode
// (cpp/execution/cuda_graph_decode.hpp, cuda_graph_decode.cu:20-97): capture a
// body enqueued on one stream into a graph, instantiate it, replay it.
//
// Qwen35DecodeAttentionGraphs is the per-context-bucket variant table the
// reference executor builds around it (cpp/execution/qwen35_executor.cu:
// 2191-2226): one variant for the single-block plan of short contexts, then
// one per distinct qwen35_online_decode_plan over the positions from the
// split threshold - 1 to max_context - 1 (split_k_256 / split_k_512 only:
// auto_select and single_block keep the single-block variant at every
// position, as the reference's table does).  Each variant holds one captured
// decode-attention step (qwen35_online_attention_decode with that plan and a
// device-resident position), so a serving loop writes the position on the
// device and replays the variant of the current position.
#pragma once

#include "qwen35_online_attention.hpp"

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <functional>
#include <memory>
#include <vector>

namespace raftinfer {

class HipGraphDecode {
public:
  using CaptureBody = std::function<void()>;

  HipGraphDecode(int device_id, hipStream_t stream);
  ~HipGraphDecode() noexcept;

  void capture(CaptureBody body);
  void replay();
  void replay_on_current_device();
  void reset() noexcept;
  bool captured() const noexcept;

  HipGraphDecode(const HipGraphDecode &) = delete;
  HipGraphDecode &operator=(const HipGraphDecode &) = delete;

private:
  int device_id_{};
  hipStream_t stream_{};
  hipGraph_t graph_{};
  hipGraphExec_t exec_{};
};

namespace kernels {

// Caller-owned buffers of one decode-attention step, as the executor passes
// them to qwen35_online_attention_decode (qwen35_executor.cu:2027-2057).
// `workspace` must hold the split-K layout of `shape`'s maximum context
// (qwen35_online_decode_workspace_layout); `device_position` is read by the
// kernels at replay time.
struct Qwen35DecodeAttentionBuffers {
  const void *query{};
  const void *key{};
  const void *value{};
  const void *gate{};
  void *output{};
  void *kv_cache{};
  std::size_t kv_cache_bytes{};
  void *workspace{};
  std::size_t workspace_bytes{};
  const std::uint32_t *device_position{};
};

class Qwen35DecodeAttentionGraphs {
public:
  // shape: the model signature with max_context_tokens set (tokens = 1,
  // past_tokens ignored).  Captures every variant on `stream` (nothing runs).
  Qwen35DecodeAttentionGraphs(int device_id, hipStream_t stream, Qwen35AttentionShape shape,
                              Qwen35DecodeAttentionMode mode, RaftInferDataType activation_dtype,
                              Qwen35KvCacheDType cache_dtype, Qwen35KvCacheLayout cache_layout,
                              Qwen35DecodeAttentionBuffers buffers);

  std::size_t variant_count() const noexcept { return variants_.size(); }
  std::size_t variant_for(std::size_t position) const;
  const Qwen35OnlineDecodePlan &plan_for(std::size_t position) const;
  // Replays the step of `position`; the caller has made *device_position ==
  // position visible to `stream` (written earlier on the same stream).
  void replay(std::size_t position);

private:
  struct Variant {
    Qwen35OnlineDecodePlan plan;
    std::unique_ptr<HipGraphDecode> graph;
  };
  std::vector<Variant> variants_;
  std::vector<std::size_t> by_position_;
};

} // namespace kernels
} // namespace raftinfer
