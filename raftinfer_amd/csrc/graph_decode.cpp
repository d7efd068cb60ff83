// HIP-graph decode capture: the HipGraphDecode wrapper
// (cpp/execution/cuda_graph_decode.cu:20-97) and the per-bucket decode
// attention variants (cpp/execution/qwen35_executor.cu:2191-2226).
#include "raftinfer_amd/hip_graph_decode.hpp"

#include <stdexcept>
#include <string>

namespace raftinfer {
namespace {

void check_hip(hipError_t status, const char *operation) {
  if (status != hipSuccess)
    throw std::runtime_error(std::string{"HIP graph decode "} + operation + ": " +
                             hipGetErrorString(status));
}

} // namespace

HipGraphDecode::HipGraphDecode(int device_id, hipStream_t stream)
    : device_id_(device_id), stream_(stream) {
  if (stream_ == nullptr) throw std::runtime_error("HIP graph decode stream is null");
}

HipGraphDecode::~HipGraphDecode() noexcept { reset(); }

void HipGraphDecode::capture(CaptureBody body) {
  if (!body) throw std::runtime_error("HIP graph decode capture body is empty");
  reset();
  check_hip(hipSetDevice(device_id_), "device selection failed");
  check_hip(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "capture begin failed");
  try {
    body();
  } catch (...) {
    hipGraph_t abandoned{};
    if (hipStreamEndCapture(stream_, &abandoned) == hipSuccess && abandoned != nullptr)
      (void)hipGraphDestroy(abandoned);
    throw;
  }
  hipGraph_t graph{};
  const hipError_t end_status = hipStreamEndCapture(stream_, &graph);
  if (end_status != hipSuccess) {
    if (graph != nullptr) (void)hipGraphDestroy(graph);
    check_hip(end_status, "capture end failed");
  }
  hipGraphExec_t exec{};
  const hipError_t inst = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  if (inst != hipSuccess) {
    (void)hipGraphDestroy(graph);
    check_hip(inst, "instantiate failed");
  }
  graph_ = graph;
  exec_ = exec;
}

void HipGraphDecode::replay() {
  if (!captured()) throw std::runtime_error("HIP graph decode has not been captured");
  check_hip(hipSetDevice(device_id_), "device selection failed");
  check_hip(hipGraphLaunch(exec_, stream_), "launch failed");
}

void HipGraphDecode::replay_on_current_device() {
  if (!captured()) throw std::runtime_error("HIP graph decode has not been captured");
  check_hip(hipGraphLaunch(exec_, stream_), "launch failed");
}

void HipGraphDecode::reset() noexcept {
  (void)hipSetDevice(device_id_);
  if (exec_ != nullptr) {
    (void)hipGraphExecDestroy(exec_);
    exec_ = nullptr;
  }
  if (graph_ != nullptr) {
    (void)hipGraphDestroy(graph_);
    graph_ = nullptr;
  }
}

bool HipGraphDecode::captured() const noexcept { return graph_ != nullptr && exec_ != nullptr; }

namespace kernels {

Qwen35DecodeAttentionGraphs::Qwen35DecodeAttentionGraphs(
    int device_id, hipStream_t stream, Qwen35AttentionShape shape, Qwen35DecodeAttentionMode mode,
    RaftInferDataType act, Qwen35KvCacheDType cache_dtype, Qwen35KvCacheLayout layout,
    Qwen35DecodeAttentionBuffers b) {
  if (stream == nullptr) throw Qwen35PrimitiveError("HIP graph decode stream is null");
  if (b.device_position == nullptr)
    throw Qwen35PrimitiveError("decode graph variants need a device position");
  if (shape.max_context_tokens == 0)
    throw Qwen35PrimitiveError("decode graph variants need a maximum context");
  const std::size_t max_ctx = shape.max_context_tokens;
  auto shape_at = [&](std::size_t position) {
    Qwen35AttentionShape s = shape;
    s.tokens = 1;
    s.past_tokens = position;
    return s;
  };
  // Variant 0: the single-block plan every position below the split
  // threshold replays (qwen35_executor.cu:2192-2198).
  by_position_.assign(max_ctx, 0);
  variants_.push_back({qwen35_online_decode_plan(shape_at(0), Qwen35DecodeAttentionMode::single_block, 1),
                       std::make_unique<HipGraphDecode>(device_id, stream)});
  // As the reference executor: only the explicit split modes add split-K
  // variants; auto_select and single_block replay variant 0 at every position.
  const std::size_t threshold = mode == Qwen35DecodeAttentionMode::split_k_256   ? 256
                                : mode == Qwen35DecodeAttentionMode::split_k_512 ? 512
                                                                                 : 0;
  if (threshold != 0) {
    std::size_t active = 0;
    for (std::size_t position = threshold - 1; position < max_ctx; ++position) {
      const auto plan = qwen35_online_decode_plan(shape_at(position), mode, position + 1);
      if (active == 0 || variants_[active].plan != plan) {
        variants_.push_back({plan, std::make_unique<HipGraphDecode>(device_id, stream)});
        active = variants_.size() - 1;
      }
      by_position_[position] = active;
    }
  }
  // Capture each variant: one decode-attention step with the device position.
  // Validation runs for the variant's smallest position; every kernel of the
  // plan is enqueued and selects itself on the device.
  for (std::size_t v = 0; v < variants_.size(); ++v) {
    std::size_t first = 0;
    while (first < max_ctx && by_position_[first] != v) ++first;
    const Qwen35AttentionShape s = shape_at(first < max_ctx ? first : 0);
    const Qwen35OnlineDecodePlan plan = variants_[v].plan;
    const bool single = plan.resolved_mode == Qwen35DecodeAttentionMode::single_block;
    variants_[v].graph->capture([&] {
      qwen35_online_attention_decode(b.query, b.key, b.value, b.gate, b.output, b.kv_cache,
                                     b.kv_cache_bytes, single ? nullptr : b.workspace,
                                     single ? 0 : b.workspace_bytes, s, act, cache_dtype, layout,
                                     plan, b.device_position, stream);
    });
  }
}

std::size_t Qwen35DecodeAttentionGraphs::variant_for(std::size_t position) const {
  if (position >= by_position_.size())
    throw Qwen35PrimitiveError("decode graph position exceeds the maximum context");
  return by_position_[position];
}

const Qwen35OnlineDecodePlan &Qwen35DecodeAttentionGraphs::plan_for(std::size_t position) const {
  return variants_[variant_for(position)].plan;
}

void Qwen35DecodeAttentionGraphs::replay(std::size_t position) {
  variants_[variant_for(position)].graph->replay(); // selects the capture device
}

} // namespace kernels
} // namespace raftinfer
