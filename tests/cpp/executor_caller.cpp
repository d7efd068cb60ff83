// A C++ caller of the drop-in headers, written the way the reference
// executor calls the kernel layer (cpp/execution/qwen35_executor.cu:2017-2057
// for attention, :2105-2126 for the gated delta).  It compiles against
// include/raftinfer_amd/*.hpp and links libraftinfer_amd.so, so the headers'
// types, defaulted operator==, noexcept and overload sets are exercised by a
// real C++ translation unit.
//
//   executor_caller host        sizing, plans, validation errors (no GPU)
//   executor_caller gpu DIR     one decode, one prefill and one gated-delta
//                               call on the GPU; inputs and outputs are
//                               written to DIR as raw float32 files for the
//                               test to check against the CPU oracle.
#include "raftinfer_amd/hip_graph_decode.hpp"
#include "raftinfer_amd/qwen35_attention.hpp"
#include "raftinfer_amd/qwen35_delta.hpp"
#include "raftinfer_amd/qwen35_online_attention.hpp"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <string>
#include <type_traits>
#include <vector>

using namespace raftinfer;
using namespace raftinfer::kernels;

namespace {

int g_failures = 0;

void expect(bool ok, const char *what) {
  if (!ok) {
    std::fprintf(stderr, "FAILED: %s\n", what);
    ++g_failures;
  }
}

template <typename E, typename Fn> void expect_throw(Fn &&fn, const char *what) {
  try {
    fn();
  } catch (const E &) {
    return;
  } catch (...) {
    std::fprintf(stderr, "FAILED (wrong exception type): %s\n", what);
    ++g_failures;
    return;
  }
  std::fprintf(stderr, "FAILED (no exception): %s\n", what);
  ++g_failures;
}

// The header contract a caller relies on, checked at compile time.
static_assert(noexcept(qwen35_online_attention_workspace_bytes(Qwen35AttentionShape{})));
static_assert(noexcept(qwen35_online_attention_prefill_supported(
    Qwen35AttentionShape{}, RAFTINFER_DTYPE_BF16, Qwen35AttentionLaunchPolicy{})));
static_assert(noexcept(qwen35_gated_delta_select_policy(GatedDeltaShape{}, 1)));
static_assert(std::is_base_of_v<std::runtime_error, Qwen35PrimitiveError>);
static_assert(std::is_base_of_v<std::runtime_error, Qwen35DeltaError>);
static_assert(std::is_same_v<decltype(Qwen35OnlineDecodePlan{} == Qwen35OnlineDecodePlan{}), bool>);

Qwen35AttentionShape decode_shape(std::size_t max_ctx, std::size_t past) {
  return Qwen35AttentionShape{.tokens = 1, .query_heads = 16, .kv_heads = 4, .head_dim = 256,
                              .max_context_tokens = max_ctx, .past_tokens = past};
}

GatedDeltaShape delta_shape(std::size_t tokens) {
  return GatedDeltaShape{.tokens = tokens, .hidden_size = 4096, .key_heads = 16, .value_heads = 32,
                         .key_dim = 128, .value_dim = 128, .conv_width = 4, .epsilon = 1e-6f};
}

int host_checks() {
  // plan / layout values of the reference test table (qwen35_cuda_attention_test.cu:283-317)
  const auto shape = decode_shape(4096, 4095);
  const auto plan = qwen35_online_decode_plan(shape, Qwen35DecodeAttentionMode::auto_select, 4096);
  const Qwen35OnlineDecodePlan want{Qwen35DecodeAttentionMode::split_k_256, 256, 256, 4096, 16};
  expect(plan == want, "auto plan at ctx 4096");
  expect(!(plan == Qwen35OnlineDecodePlan{}), "plan inequality");
  const auto layout = qwen35_online_decode_workspace_layout(shape, plan.resolved_mode);
  const Qwen35OnlineDecodeWorkspaceLayout want_layout{256, 0, 1024, 2048, 264192};
  expect(layout == want_layout, "split-K workspace layout at max_ctx 4096");
  expect(qwen35_online_attention_workspace_bytes(shape) == 0, "online workspace is zero");
  const Qwen35AttentionLaunchPolicy policy{Qwen35AttentionImplementation::online_tiled,
                                           Qwen35KvCacheDType::bf16, Qwen35KvCacheLayout::head_major};
  expect(qwen35_attention_cache_bytes(shape, policy) == 2u * 4096 * 4 * 256 * 2, "cache bytes");
  expect(qwen35_attention_workspace_bytes(shape, policy) == 0, "online attention workspace bytes");
  expect(qwen35_attention_workspace_floats(shape) == 16u * 4096, "materialized workspace floats");
  expect(qwen35_online_attention_prefill_supported(
             Qwen35AttentionShape{512, 16, 4, 256, 512, 0}, RAFTINFER_DTYPE_BF16, policy),
         "prefill supported at PP512");
  const auto dshape = delta_shape(512);
  expect(qwen35_gated_delta_workspace_bytes(dshape) >= 512u * (8192 + 4096) * 4,
         "delta workspace at least the reference's");
  const auto dpol = qwen35_gated_delta_select_policy(dshape, 512);
  expect(dpol.schedule == GatedDeltaSchedule::register_resident_current, "delta policy");
  // validation throws the reference's error types before any launch
  std::vector<char> dummy(64);
  expect_throw<Qwen35PrimitiveError>(
      [&] {
        qwen35_online_attention_decode(dummy.data(), dummy.data(), dummy.data(), dummy.data(),
                                       dummy.data(), dummy.data(), dummy.size(), nullptr, 0, shape,
                                       RAFTINFER_DTYPE_BF16, Qwen35KvCacheDType::bf16,
                                       Qwen35KvCacheLayout::head_major, plan, nullptr, nullptr);
      },
      "decode with a null stream");
  expect_throw<Qwen35PrimitiveError>(
      [&] {
        qwen35_online_decode_plan(shape, Qwen35DecodeAttentionMode::split_k_256, 5000);
      },
      "plan beyond the maximum context");
  expect_throw<Qwen35DeltaError>(
      [&] {
        auto bad = delta_shape(4);
        bad.value_heads = 30;
        (void)qwen35_gated_delta_workspace_bytes(bad);
      },
      "delta shape with value_heads not divisible by key_heads");
  // the plan-less single-block overload resolves and validates too
  expect_throw<Qwen35PrimitiveError>(
      [&] {
        qwen35_online_attention_decode(dummy.data(), dummy.data(), dummy.data(), dummy.data(),
                                       dummy.data(), dummy.data(), dummy.size(), shape,
                                       RAFTINFER_DTYPE_BF16, Qwen35KvCacheDType::bf16,
                                       Qwen35KvCacheLayout::head_major, nullptr, nullptr);
      },
      "single-block overload with a null stream");
  std::printf(g_failures == 0 ? "host checks ok\n" : "host checks FAILED\n");
  return g_failures == 0 ? 0 : 1;
}

// ------------------------------------------------------------- GPU mode
std::uint16_t to_bf16(float x) {
  std::uint32_t u;
  std::memcpy(&u, &x, 4);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<std::uint16_t>(u >> 16);
}
float from_bf16(std::uint16_t b) {
  const std::uint32_t u = static_cast<std::uint32_t>(b) << 16;
  float x;
  std::memcpy(&x, &u, 4);
  return x;
}

struct Bf16Buffer {
  std::vector<std::uint16_t> host;
  void *dev{};
  explicit Bf16Buffer(std::size_t n) : host(n, 0) {
    if (hipMalloc(&dev, n * 2) != hipSuccess) throw std::runtime_error("hipMalloc failed");
  }
  ~Bf16Buffer() { (void)hipFree(dev); }
  void fill(std::mt19937 &gen, std::size_t count) {
    std::normal_distribution<float> nd;
    for (std::size_t i = 0; i < count; ++i) host[i] = to_bf16(nd(gen));
  }
  void upload() { check(hipMemcpy(dev, host.data(), host.size() * 2, hipMemcpyHostToDevice)); }
  void download() { check(hipMemcpy(host.data(), dev, host.size() * 2, hipMemcpyDeviceToHost)); }
  void save(const std::string &path) const {
    std::vector<float> f(host.size());
    for (std::size_t i = 0; i < f.size(); ++i) f[i] = from_bf16(host[i]);
    FILE *fp = std::fopen(path.c_str(), "wb");
    std::fwrite(f.data(), 4, f.size(), fp);
    std::fclose(fp);
  }
  static void check(hipError_t e) {
    if (e != hipSuccess) throw std::runtime_error(hipGetErrorString(e));
  }
};

int gpu_run(const std::string &dir) {
  hipStream_t stream{};
  Bf16Buffer::check(hipStreamCreate(&stream));
  std::mt19937 gen(0x5241);
  // ---- decode, as qwen35_executor.cu:2027-2045 (tokens == 1, online_tiled)
  {
    const std::size_t max_ctx = 1024, position = 700;
    const auto attention_shape = decode_shape(max_ctx, position);
    Bf16Buffer q(16 * 256), k(4 * 256), v(4 * 256), g(16 * 256), out(16 * 256),
        cache(2 * max_ctx * 4 * 256);
    q.fill(gen, q.host.size());
    k.fill(gen, k.host.size());
    v.fill(gen, v.host.size());
    g.fill(gen, g.host.size());
    std::normal_distribution<float> nd;
    for (int plane = 0; plane < 2; ++plane)
      for (std::size_t h = 0; h < 4; ++h)
        for (std::size_t t = 0; t < position; ++t)
          for (std::size_t d = 0; d < 256; ++d)
            cache.host[plane * max_ctx * 1024 + (h * max_ctx + t) * 256 + d] = to_bf16(nd(gen));
    for (auto *b : {&q, &k, &v, &g, &cache}) b->upload();
    const auto plan = kernels::qwen35_online_decode_plan(
        attention_shape, Qwen35DecodeAttentionMode::auto_select, position + 1);
    const auto decode_workspace_bytes =
        kernels::qwen35_online_decode_workspace_layout(attention_shape, plan.resolved_mode).bytes;
    void *attention_workspace{};
    Bf16Buffer::check(hipMalloc(&attention_workspace, decode_workspace_bytes));
    kernels::qwen35_online_attention_decode(
        q.dev, k.dev, v.dev, g.dev, out.dev, cache.dev, cache.host.size() * 2,
        decode_workspace_bytes == 0 ? nullptr : attention_workspace, decode_workspace_bytes,
        attention_shape, RAFTINFER_DTYPE_BF16, Qwen35KvCacheDType::bf16,
        Qwen35KvCacheLayout::head_major, plan, nullptr, stream);
    Bf16Buffer::check(hipStreamSynchronize(stream));
    out.download();
    cache.download();
    q.save(dir + "/decode_q.f32");
    k.save(dir + "/decode_k.f32");
    v.save(dir + "/decode_v.f32");
    g.save(dir + "/decode_g.f32");
    cache.save(dir + "/decode_cache.f32");
    out.save(dir + "/decode_out.f32");
    (void)hipFree(attention_workspace);
  }
  // ---- prefill, as qwen35_executor.cu:2046-2054 (qwen35_causal_attention)
  {
    const std::size_t T = 40;
    const Qwen35AttentionShape attention_shape{T, 16, 4, 256, T, 0};
    const Qwen35AttentionLaunchPolicy policy{Qwen35AttentionImplementation::online_tiled,
                                             Qwen35KvCacheDType::bf16, Qwen35KvCacheLayout::head_major};
    Bf16Buffer q(T * 16 * 256), k(T * 4 * 256), v(T * 4 * 256), g(T * 16 * 256),
        out(T * 16 * 256), cache(2 * T * 4 * 256);
    for (auto *b : {&q, &k, &v, &g}) {
      b->fill(gen, b->host.size());
      b->upload();
    }
    cache.upload();
    const std::size_t prefill_attention_workspace_bytes =
        kernels::qwen35_attention_workspace_bytes(attention_shape, policy);
    kernels::qwen35_causal_attention(q.dev, k.dev, v.dev, g.dev, out.dev, cache.dev,
                                     cache.host.size() * 2, nullptr,
                                     prefill_attention_workspace_bytes, attention_shape,
                                     RAFTINFER_DTYPE_BF16, policy, stream);
    Bf16Buffer::check(hipStreamSynchronize(stream));
    out.download();
    q.save(dir + "/prefill_q.f32");
    k.save(dir + "/prefill_k.f32");
    v.save(dir + "/prefill_v.f32");
    g.save(dir + "/prefill_g.f32");
    out.save(dir + "/prefill_out.f32");
  }
  // ---- gated delta, as qwen35_executor.cu:2105-2126
  {
    const std::size_t tokens = 5;
    const auto shape = delta_shape(tokens);
    Bf16Buffer input(tokens * 12352), conv(8192 * 4), a(32), dt(32), norm(128), out(tokens * 4096);
    input.fill(gen, input.host.size());
    std::normal_distribution<float> nd;
    for (auto &x : conv.host) x = to_bf16(0.3f * nd(gen));
    for (auto &x : a.host) x = to_bf16(-std::exp(0.5f * nd(gen)));
    dt.fill(gen, dt.host.size());
    norm.fill(gen, norm.host.size());
    for (auto *b : {&input, &conv, &a, &dt, &norm}) b->upload();
    float *conv_state{}, *rec_state{};
    void *delta_workspace{};
    Bf16Buffer::check(hipMalloc(reinterpret_cast<void **>(&conv_state), 8192 * 3 * 4));
    Bf16Buffer::check(hipMalloc(reinterpret_cast<void **>(&rec_state), 32 * 128 * 128 * 4));
    Bf16Buffer::check(hipMemset(conv_state, 0, 8192 * 3 * 4));
    Bf16Buffer::check(hipMemset(rec_state, 0, 32 * 128 * 128 * 4));
    const std::size_t ws_bytes = kernels::qwen35_gated_delta_workspace_bytes(shape);
    Bf16Buffer::check(hipMalloc(&delta_workspace, ws_bytes));
    kernels::qwen35_gated_delta(input.dev, conv.dev, a.dev, dt.dev, norm.dev, out.dev, conv_state,
                                rec_state, delta_workspace, ws_bytes, shape,
                                kernels::qwen35_gated_delta_select_policy(shape, tokens),
                                RAFTINFER_DTYPE_BF16, RAFTINFER_DTYPE_BF16, stream);
    Bf16Buffer::check(hipStreamSynchronize(stream));
    out.download();
    std::vector<float> rec(32 * 128 * 128);
    Bf16Buffer::check(hipMemcpy(rec.data(), rec_state, rec.size() * 4, hipMemcpyDeviceToHost));
    input.save(dir + "/delta_input.f32");
    conv.save(dir + "/delta_conv_w.f32");
    a.save(dir + "/delta_a.f32");
    dt.save(dir + "/delta_dt.f32");
    norm.save(dir + "/delta_norm_w.f32");
    out.save(dir + "/delta_out.f32");
    FILE *fp = std::fopen((dir + "/delta_rec.f32").c_str(), "wb");
    std::fwrite(rec.data(), 4, rec.size(), fp);
    std::fclose(fp);
    (void)hipFree(conv_state);
    (void)hipFree(rec_state);
    (void)hipFree(delta_workspace);
  }
  Bf16Buffer::check(hipStreamDestroy(stream));
  std::printf("gpu run ok\n");
  return 0;
}

} // namespace

int main(int argc, char **argv) {
  const std::string mode = argc > 1 ? argv[1] : "host";
  try {
    if (mode == "host") return host_checks();
    if (mode == "gpu" && argc > 2) return gpu_run(argv[2]);
  } catch (const std::exception &e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 2;
  }
  std::fprintf(stderr, "usage: executor_caller host | gpu DIR\n");
  return 2;
}
