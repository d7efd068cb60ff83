// Public attention dispatcher, cache/workspace sizing, the materialized
// fallback path and the online prefill entry point.
//
// Host semantics follow cpp/kernels/qwen35_attention.cu:103-613 and
// cpp/kernels/qwen35_online_attention.cu:27-94, :1145-1218.  The online
// prefill runs the bf16 MFMA kernel (attention_prefill_mfma.hip) for the
// Qwen3.5 signature with bf16 activations and cache, and a generic fp32
// wave-per-row kernel for every other supported shape / dtype / layout.
#include <cmath>
#include "decode_scan.hpp"
#include "prefill_mfma.hpp"
#include "raftinfer_amd/qwen35_online_attention.hpp"

namespace raftinfer::kernels {
namespace {

using namespace raftinfer::amd;
using Err = Qwen35PrimitiveError;

constexpr int kBlockSize = 256;
constexpr std::size_t kPrefillRowsPerBlock = 4;
constexpr std::size_t kMaxGridY = 65535;

bool multiplication_fits(std::size_t a, std::size_t b) noexcept {
  return a == 0 || b <= std::numeric_limits<std::size_t>::max() / a;
}

void require_dtype(RaftInferDataType dtype) {
  require<Err>(dtype == RAFTINFER_DTYPE_F32 || dtype == RAFTINFER_DTYPE_F16 ||
                   dtype == RAFTINFER_DTYPE_BF16,
               "unsupported Qwen3.5 attention dtype");
}

std::size_t current_context_tokens(Qwen35AttentionShape s) {
  return checked_add<Err>(s.past_tokens, s.tokens, "attention context length overflow");
}
std::size_t hidden_size(Qwen35AttentionShape s) {
  return checked_mul<Err>(s.query_heads, s.head_dim, "attention hidden size overflow");
}
std::size_t kv_vector_size(Qwen35AttentionShape s) {
  return checked_mul<Err>(s.kv_heads, s.head_dim, "attention kv vector size overflow");
}

// cpp/kernels/qwen35_attention.cu:113-131
void validate_shape(Qwen35AttentionShape s) {
  require<Err>(s.tokens > 0, "attention tokens must be positive");
  require<Err>(s.query_heads > 0, "attention query_heads must be positive");
  require<Err>(s.kv_heads > 0, "attention kv_heads must be positive");
  require<Err>(s.head_dim > 0, "attention head_dim must be positive");
  require<Err>(s.max_context_tokens > 0, "attention max_context_tokens must be positive");
  require<Err>(s.query_heads % s.kv_heads == 0,
               "attention query_heads must be divisible by kv_heads");
  require<Err>(current_context_tokens(s) <= s.max_context_tokens,
               "attention context exceeds cache capacity");
  (void)checked_mul<Err>(s.tokens, hidden_size(s), "attention output shape overflow");
  (void)checked_mul<Err>(2,
                         checked_mul<Err>(s.max_context_tokens, kv_vector_size(s),
                                          "attention cache shape overflow"),
                         "attention cache shape overflow");
}

void validate_launch_policy(Qwen35AttentionLaunchPolicy p) {
  require<Err>(p.implementation == Qwen35AttentionImplementation::materialized_reference ||
                   p.implementation == Qwen35AttentionImplementation::online_tiled,
               "unsupported Qwen3.5 attention implementation");
  require<Err>(p.kv_cache_dtype == Qwen35KvCacheDType::f32 ||
                   p.kv_cache_dtype == Qwen35KvCacheDType::bf16,
               "unsupported Qwen3.5 KV cache dtype");
  require<Err>(p.kv_cache_layout == Qwen35KvCacheLayout::token_major ||
                   p.kv_cache_layout == Qwen35KvCacheLayout::head_major,
               "unsupported Qwen3.5 KV cache layout");
}

std::size_t kv_cache_element_bytes(Qwen35KvCacheDType dtype) {
  return dtype == Qwen35KvCacheDType::f32 ? sizeof(float) : sizeof(bf16_bits);
}

void validate_attention_pointers(const void *q, const void *k, const void *v, const void *g,
                                 void *o, void *cache, void *workspace,
                                 std::size_t required_workspace, hipStream_t stream) {
  require<Err>(q != nullptr, "attention query pointer is null");
  require<Err>(k != nullptr, "attention key pointer is null");
  require<Err>(v != nullptr, "attention value pointer is null");
  require<Err>(g != nullptr, "attention gate pointer is null");
  require<Err>(o != nullptr, "attention output pointer is null");
  require<Err>(cache != nullptr, "attention kv_cache pointer is null");
  require<Err>(required_workspace == 0 || workspace != nullptr,
               "attention workspace pointer is null");
  require<Err>(stream != nullptr, "HIP stream is null");
}

// cpp/kernels/qwen35_online_attention.cu:27-94
bool online_prefill_signature_supported(Qwen35AttentionShape s, RaftInferDataType act,
                                        Qwen35KvCacheDType cache_dtype,
                                        Qwen35KvCacheLayout layout) noexcept {
  if (s.tokens <= 1 || s.query_heads == 0 || s.kv_heads == 0 || s.head_dim == 0 ||
      s.head_dim > 256 || s.max_context_tokens == 0 || s.query_heads % s.kv_heads != 0 ||
      s.past_tokens > s.max_context_tokens || s.tokens > s.max_context_tokens - s.past_tokens)
    return false;
  if (act != RAFTINFER_DTYPE_F32 && act != RAFTINFER_DTYPE_BF16) return false;
  std::size_t eb = 0;
  switch (cache_dtype) {
  case Qwen35KvCacheDType::f32: eb = 4; break;
  case Qwen35KvCacheDType::bf16: eb = 2; break;
  default: return false;
  }
  if (layout != Qwen35KvCacheLayout::token_major && layout != Qwen35KvCacheLayout::head_major)
    return false;
  const auto int_limit = static_cast<std::size_t>(std::numeric_limits<int>::max());
  const std::size_t query_tiles = ceil_div_unchecked(s.tokens, kPrefillRowsPerBlock);
  if (s.query_heads > int_limit || query_tiles > kMaxGridY ||
      !multiplication_fits(s.kv_heads, s.head_dim))
    return false;
  const std::size_t kv_size = s.kv_heads * s.head_dim;
  if (!multiplication_fits(s.tokens, kv_size) || !multiplication_fits(s.max_context_tokens, kv_size) ||
      !multiplication_fits(s.query_heads, s.head_dim))
    return false;
  const std::size_t kv_elements = s.tokens * kv_size;
  if (ceil_div_unchecked(kv_elements, kBlockSize) > int_limit ||
      !multiplication_fits(s.tokens, s.query_heads * s.head_dim))
    return false;
  const std::size_t plane = s.max_context_tokens * kv_size;
  return multiplication_fits(2, plane) && multiplication_fits(2 * plane, eb);
}

// ------------------------------------------------------------ kernels

template <typename CacheT>
__device__ __forceinline__ std::size_t cache_index(bool head_major, std::size_t token,
                                                   std::size_t kvh, std::size_t dim,
                                                   std::size_t max_ctx, std::size_t kv_heads,
                                                   std::size_t head_dim) {
  return head_major ? (kvh * max_ctx + token) * head_dim + dim
                    : (token * kv_heads + kvh) * head_dim + dim;
}

// Appends T tokens of K and V at past..past+T-1 with the layout's index
// (cpp/kernels/qwen35_online_attention.cu:295-321); RNE cast for bf16.
template <typename ActT, typename CacheT>
__global__ __launch_bounds__(kBlockSize) void append_prefill_kernel(
    const ActT *__restrict__ key, const ActT *__restrict__ value, CacheT *__restrict__ cache,
    std::size_t tokens, std::size_t kv_heads, std::size_t head_dim, std::size_t max_ctx,
    std::size_t past, bool head_major) {
  const std::size_t e = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const std::size_t kv_size = kv_heads * head_dim;
  if (e >= tokens * kv_size) return;
  const std::size_t t = e / kv_size;
  const std::size_t within = e - t * kv_size;
  const std::size_t kvh = within / head_dim;
  const std::size_t d = within - kvh * head_dim;
  const std::size_t idx =
      cache_index<CacheT>(head_major, past + t, kvh, d, max_ctx, kv_heads, head_dim);
  const std::size_t plane = max_ctx * kv_size;
  Elem<CacheT>::store(cache, idx, Elem<ActT>::load(key, e));
  Elem<CacheT>::store(cache, plane + idx, Elem<ActT>::load(value, e));
}

// Generic online prefill: one wave per (query token, query head), lane owns
// dims lane + 64*i.  Keys are read from the cache in 16-key tiles with an
// fp32 running max / sum (cpp/kernels/qwen35_online_attention.cu:758-867).
template <typename ActT, typename CacheT>
__global__ __launch_bounds__(kBlockSize) void prefill_generic_kernel(
    const ActT *__restrict__ query, const ActT *__restrict__ gate, ActT *__restrict__ output,
    const CacheT *__restrict__ cache, std::size_t tokens, std::size_t query_heads,
    std::size_t kv_heads, std::size_t head_dim, std::size_t max_ctx, std::size_t past,
    bool head_major) {
  constexpr int kKTile = 16;
  const int lane = threadIdx.x & 63;
  const std::size_t t = static_cast<std::size_t>(blockIdx.y) * kPrefillRowsPerBlock + (threadIdx.x >> 6);
  if (t >= tokens) return;
  const std::size_t h = blockIdx.x;
  const std::size_t kvh = h / (query_heads / kv_heads);
  const std::size_t visible = past + t + 1;
  const std::size_t plane = max_ctx * kv_heads * head_dim;
  const std::size_t qbase = (t * query_heads + h) * head_dim;
  const float scale = rsqrtf(static_cast<float>(head_dim));
  float q[4], acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const std::size_t d = lane + 64 * i;
    q[i] = d < head_dim ? Elem<ActT>::load(query, qbase + d) : 0.f;
    acc[i] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  for (std::size_t k0 = 0; k0 < visible; k0 += kKTile) {
    float s[kKTile];
    float tmax = -INFINITY;
#pragma unroll
    for (int j = 0; j < kKTile; ++j) {
      s[j] = -INFINITY;
      if (k0 + j < visible) {
        const std::size_t base =
            cache_index<CacheT>(head_major, k0 + j, kvh, 0, max_ctx, kv_heads, head_dim);
        float dot = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const std::size_t d = lane + 64 * i;
          if (d < head_dim) dot = fmaf(q[i], Elem<CacheT>::load(cache, base + d), dot);
        }
        s[j] = wave_sum(dot) * scale;
        tmax = fmaxf(tmax, s[j]);
      }
    }
    const float mn = fmaxf(m, tmax);
    const float so = m == -INFINITY ? 0.f : __expf(m - mn);
    l *= so;
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] *= so;
#pragma unroll
    for (int j = 0; j < kKTile; ++j) {
      if (k0 + j >= visible) continue;
      const std::size_t base =
          plane + cache_index<CacheT>(head_major, k0 + j, kvh, 0, max_ctx, kv_heads, head_dim);
      const float p = __expf(s[j] - mn);
      l += p;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const std::size_t d = lane + 64 * i;
        if (d < head_dim) acc[i] = fmaf(p, Elem<CacheT>::load(cache, base + d), acc[i]);
      }
    }
    m = mn;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const std::size_t d = lane + 64 * i;
    if (d < head_dim) {
      const std::size_t idx = qbase + d;
      Elem<ActT>::store(output, idx, (acc[i] / l) * sigmoid_gate(Elem<ActT>::load(gate, idx)));
    }
  }
}

// ---- materialized reference path (f32 token-major cache, logits workspace)
// cpp/kernels/qwen35_attention.cu:133-362: logits in a [T][Hq][ctx] fp32
// workspace, softmax with a double denominator, PV accumulated in double.

template <typename ActT>
__global__ __launch_bounds__(kBlockSize) void materialized_append_kernel(
    const ActT *__restrict__ key, const ActT *__restrict__ value, float *__restrict__ cache,
    std::size_t tokens, std::size_t kv_size, std::size_t max_ctx, std::size_t past) {
  const std::size_t e = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= tokens * kv_size) return;
  const std::size_t t = e / kv_size;
  const std::size_t idx = (past + t) * kv_size + (e - t * kv_size);
  cache[idx] = Elem<ActT>::load(key, e);
  cache[max_ctx * kv_size + idx] = Elem<ActT>::load(value, e);
}

// One workgroup per (token, query head): each wave computes dot products for
// a strided subset of the visible keys.
template <typename ActT>
__global__ __launch_bounds__(kBlockSize) void materialized_logits_kernel(
    const ActT *__restrict__ query, const float *__restrict__ cache, float *__restrict__ logits,
    std::size_t tokens, std::size_t query_heads, std::size_t kv_heads, std::size_t head_dim,
    std::size_t past) {
  const std::size_t pair = blockIdx.x;
  const std::size_t t = pair / query_heads;
  const std::size_t h = pair - t * query_heads;
  const std::size_t kvh = h / (query_heads / kv_heads);
  const std::size_t ctx = past + tokens;
  const std::size_t visible = past + t + 1;
  const float scale = rsqrtf(static_cast<float>(head_dim));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const std::size_t qbase = (t * query_heads + h) * head_dim;
  for (std::size_t key = wave; key < visible; key += kBlockSize / 64) {
    const std::size_t kbase = (key * kv_heads + kvh) * head_dim;
    float dot = 0.f;
    for (std::size_t d = lane; d < head_dim; d += 64)
      dot = fmaf(Elem<ActT>::load(query, qbase + d), cache[kbase + d], dot);
    dot = wave_sum(dot);
    if (lane == 0) logits[(t * query_heads + h) * ctx + key] = dot * scale;
  }
}

template <typename ActT>
__global__ __launch_bounds__(kBlockSize) void materialized_output_kernel(
    const float *__restrict__ cache, const ActT *__restrict__ gate, ActT *__restrict__ output,
    float *__restrict__ logits, std::size_t tokens, std::size_t query_heads,
    std::size_t kv_heads, std::size_t head_dim, std::size_t max_ctx, std::size_t past) {
  __shared__ float red_f[kBlockSize / 64];
  __shared__ double red_d[kBlockSize / 64];
  const std::size_t pair = blockIdx.x;
  const std::size_t t = pair / query_heads;
  const std::size_t h = pair - t * query_heads;
  const std::size_t kvh = h / (query_heads / kv_heads);
  const std::size_t ctx = past + tokens;
  const std::size_t visible = past + t + 1;
  float *row = logits + (t * query_heads + h) * ctx;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float mx = -INFINITY;
  for (std::size_t k = threadIdx.x; k < visible; k += kBlockSize) mx = fmaxf(mx, row[k]);
  mx = wave_max(mx);
  if (lane == 0) red_f[wave] = mx;
  __syncthreads();
  mx = red_f[0];
  for (int w = 1; w < kBlockSize / 64; ++w) mx = fmaxf(mx, red_f[w]);
  double den = 0.0;
  for (std::size_t k = threadIdx.x; k < visible; k += kBlockSize)
    den += exp(static_cast<double>(row[k]) - static_cast<double>(mx));
  for (int off = 32; off > 0; off >>= 1) den += __shfl_xor(den, off);
  if (lane == 0) red_d[wave] = den;
  __syncthreads();
  den = 0.0;
  for (int w = 0; w < kBlockSize / 64; ++w) den += red_d[w];
  const float denf = static_cast<float>(den);
  for (std::size_t k = threadIdx.x; k < visible; k += kBlockSize)
    row[k] = __expf(row[k] - mx) / denf;
  __syncthreads();
  const std::size_t kv_size = kv_heads * head_dim;
  const std::size_t plane = max_ctx * kv_size;
  for (std::size_t d = threadIdx.x; d < head_dim; d += kBlockSize) {
    double sum = 0.0;
    for (std::size_t k = 0; k < visible; ++k)
      sum += static_cast<double>(row[k]) *
             static_cast<double>(cache[plane + (k * kv_heads + kvh) * head_dim + d]);
    const std::size_t idx = (t * query_heads + h) * head_dim + d;
    Elem<ActT>::store(output, idx,
                      static_cast<float>(sum) * sigmoid_gate(Elem<ActT>::load(gate, idx)));
  }
}

template <typename ActT>
void launch_materialized(const void *q, const void *k, const void *v, const void *g, void *o,
                         float *cache, float *logits, Qwen35AttentionShape s, hipStream_t stream) {
  const std::size_t kv_size = s.kv_heads * s.head_dim;
  const std::size_t kv_elements = s.tokens * kv_size;
  const int append_grid = static_cast<int>(ceil_div_unchecked(kv_elements, kBlockSize));
  materialized_append_kernel<ActT><<<append_grid, kBlockSize, 0, stream>>>(
      static_cast<const ActT *>(k), static_cast<const ActT *>(v), cache, s.tokens, kv_size,
      s.max_context_tokens, s.past_tokens);
  check_launch<Err>("qwen35_attention_append_cache");
  const std::size_t pairs = s.tokens * s.query_heads;
  require<Err>(pairs <= static_cast<std::size_t>(std::numeric_limits<int>::max()),
               "attention grid dimension overflow");
  materialized_logits_kernel<ActT><<<static_cast<int>(pairs), kBlockSize, 0, stream>>>(
      static_cast<const ActT *>(q), cache, logits, s.tokens, s.query_heads, s.kv_heads,
      s.head_dim, s.past_tokens);
  check_launch<Err>("qwen35_attention_logits");
  materialized_output_kernel<ActT><<<static_cast<int>(pairs), kBlockSize, 0, stream>>>(
      cache, static_cast<const ActT *>(g), static_cast<ActT *>(o), logits, s.tokens,
      s.query_heads, s.kv_heads, s.head_dim, s.max_context_tokens, s.past_tokens);
  check_launch<Err>("qwen35_attention_output");
}

template <typename ActT, typename CacheT>
void launch_prefill(const void *q, const void *k, const void *v, const void *g, void *o,
                    void *cache, Qwen35AttentionShape s, Qwen35KvCacheLayout layout,
                    hipStream_t stream, bool kernel_only) {
  const bool head_major = layout == Qwen35KvCacheLayout::head_major;
  const std::size_t kv_elements = s.tokens * s.kv_heads * s.head_dim;
  const int append_grid = static_cast<int>(ceil_div_unchecked(kv_elements, kBlockSize));
  bool mfma = false, fused = false;
  if constexpr (std::is_same_v<ActT, bf16_bits> && std::is_same_v<CacheT, bf16_bits>) {
    const auto bits = [](const void *p) { return reinterpret_cast<std::uintptr_t>(p); };
    mfma = ((bits(q) | bits(cache)) & 15u) == 0 && ((bits(g) | bits(o)) & 7u) == 0 &&
           s.query_heads == kQueryHeads && s.kv_heads == kKvHeads && s.head_dim == kHeadDim;
    // A prompt with no past reads its keys straight from key/value and
    // appends them inside the attention kernel.
    fused = mfma && s.past_tokens == 0 && ((bits(k) | bits(v)) & 15u) == 0;
  }
  if (!kernel_only && !fused) {
    append_prefill_kernel<ActT, CacheT><<<append_grid, kBlockSize, 0, stream>>>(
        static_cast<const ActT *>(k), static_cast<const ActT *>(v), static_cast<CacheT *>(cache),
        s.tokens, s.kv_heads, s.head_dim, s.max_context_tokens, s.past_tokens, head_major);
    check_launch<Err>("qwen35_online_attention_append_cache");
  }
  if (mfma) {
    if constexpr (std::is_same_v<ActT, bf16_bits> && std::is_same_v<CacheT, bf16_bits>) {
      amd::launch_prefill_mfma(static_cast<const bf16_bits *>(q), static_cast<const bf16_bits *>(k),
                               static_cast<const bf16_bits *>(v), static_cast<const bf16_bits *>(g),
                               static_cast<bf16_bits *>(o), static_cast<bf16_bits *>(cache), s.tokens,
                               s.max_context_tokens, s.past_tokens, head_major, fused, stream);
      check_launch<Err>("qwen35_online_attention_prefill_gfx950_mfma_hd256");
      return;
    }
  }
  const dim3 grid{static_cast<unsigned>(s.query_heads),
                  static_cast<unsigned>(ceil_div_unchecked(s.tokens, kPrefillRowsPerBlock)), 1};
  prefill_generic_kernel<ActT, CacheT><<<grid, kBlockSize, 0, stream>>>(
      static_cast<const ActT *>(q), static_cast<const ActT *>(g), static_cast<ActT *>(o),
      static_cast<const CacheT *>(cache), s.tokens, s.query_heads, s.kv_heads, s.head_dim,
      s.max_context_tokens, s.past_tokens, head_major);
  check_launch<Err>("qwen35_online_attention_prefill_generic");
}

} // namespace

// ---------------------------------------------------------- sizing API

std::size_t qwen35_attention_workspace_floats(Qwen35AttentionShape shape) {
  validate_shape(shape);
  const std::size_t pairs =
      checked_mul<Err>(shape.tokens, shape.query_heads, "attention workspace shape overflow");
  return checked_mul<Err>(pairs, current_context_tokens(shape), "attention workspace shape overflow");
}

std::size_t qwen35_attention_workspace_bytes(Qwen35AttentionShape shape) {
  return checked_mul<Err>(qwen35_attention_workspace_floats(shape), sizeof(float),
                          "attention workspace byte size overflow");
}

std::size_t qwen35_attention_cache_bytes(Qwen35AttentionShape shape,
                                         Qwen35AttentionLaunchPolicy policy) {
  validate_shape(shape);
  validate_launch_policy(policy);
  const std::size_t elements =
      checked_mul<Err>(2,
                       checked_mul<Err>(shape.max_context_tokens, kv_vector_size(shape),
                                        "attention cache shape overflow"),
                       "attention cache shape overflow");
  return checked_mul<Err>(elements, kv_cache_element_bytes(policy.kv_cache_dtype),
                          "attention cache byte size overflow");
}

std::size_t qwen35_attention_workspace_bytes(Qwen35AttentionShape shape,
                                             Qwen35AttentionLaunchPolicy policy) {
  validate_launch_policy(policy);
  if (policy.implementation == Qwen35AttentionImplementation::materialized_reference)
    return qwen35_attention_workspace_bytes(shape);
  validate_shape(shape);
  return qwen35_online_attention_workspace_bytes(shape);
}

bool qwen35_online_attention_prefill_supported(Qwen35AttentionShape shape,
                                               RaftInferDataType act,
                                               Qwen35AttentionLaunchPolicy policy) noexcept {
  if (policy.implementation != Qwen35AttentionImplementation::online_tiled) return false;
  return online_prefill_signature_supported(shape, act, policy.kv_cache_dtype,
                                            policy.kv_cache_layout);
}

// ------------------------------------------------------------ prefill API
namespace {
// cpp/kernels/qwen35_online_attention.cu:1161-1218
void prefill_impl(const void *query, const void *key, const void *value, const void *gate,
                  void *output, void *kv_cache, std::size_t kv_cache_bytes,
                  Qwen35AttentionShape shape, RaftInferDataType act,
                  Qwen35KvCacheDType cache_dtype, Qwen35KvCacheLayout layout, hipStream_t stream,
                  bool kernel_only) {
  require<Err>(query != nullptr, "online attention query pointer is null");
  require<Err>(key != nullptr, "online attention key pointer is null");
  require<Err>(value != nullptr, "online attention value pointer is null");
  require<Err>(gate != nullptr, "online attention gate pointer is null");
  require<Err>(output != nullptr, "online attention output pointer is null");
  require<Err>(kv_cache != nullptr, "online attention KV cache pointer is null");
  require<Err>(stream != nullptr, "online attention HIP stream is null");
  require<Err>(online_prefill_signature_supported(shape, act, cache_dtype, layout),
               "unsupported online attention prefill signature; select the "
               "materialized implementation before allocation");
  const std::size_t eb = cache_dtype == Qwen35KvCacheDType::f32 ? 4 : 2;
  const std::size_t required = checked_mul<Err>(
      checked_mul<Err>(2,
                       checked_mul<Err>(shape.max_context_tokens,
                                        checked_mul<Err>(shape.kv_heads, shape.head_dim,
                                                         "online attention cache shape overflow"),
                                        "online attention cache shape overflow"),
                       "online attention cache shape overflow"),
      eb, "online attention cache byte size overflow");
  require<Err>(kv_cache_bytes >= required, "online attention KV cache is too small");
  const bool f32_act = act == RAFTINFER_DTYPE_F32;
  const bool f32_cache = cache_dtype == Qwen35KvCacheDType::f32;
  if (f32_act && f32_cache)
    launch_prefill<float, float>(query, key, value, gate, output, kv_cache, shape, layout, stream, kernel_only);
  else if (f32_act)
    launch_prefill<float, bf16_bits>(query, key, value, gate, output, kv_cache, shape, layout, stream,
                                     kernel_only);
  else if (f32_cache)
    launch_prefill<bf16_bits, float>(query, key, value, gate, output, kv_cache, shape, layout, stream,
                                     kernel_only);
  else
    launch_prefill<bf16_bits, bf16_bits>(query, key, value, gate, output, kv_cache, shape, layout,
                                         stream, kernel_only);
}
} // namespace

void qwen35_online_attention_prefill(const void *query, const void *key, const void *value,
                                     const void *gate, void *output, void *kv_cache,
                                     std::size_t kv_cache_bytes, Qwen35AttentionShape shape,
                                     RaftInferDataType act, Qwen35KvCacheDType cache_dtype,
                                     Qwen35KvCacheLayout layout, hipStream_t stream) {
  prefill_impl(query, key, value, gate, output, kv_cache, kv_cache_bytes, shape, act, cache_dtype,
               layout, stream, false);
}

void qwen35_online_attention_prefill_kernel_only(
    const void *query, const void *key, const void *value, const void *gate, void *output,
    void *kv_cache, std::size_t kv_cache_bytes, Qwen35AttentionShape shape, RaftInferDataType act,
    Qwen35KvCacheDType cache_dtype, Qwen35KvCacheLayout layout, hipStream_t stream) {
  prefill_impl(query, key, value, gate, output, kv_cache, kv_cache_bytes, shape, act, cache_dtype,
               layout, stream, true);
}

void qwen35_online_attention_prefill_fused(const void *query_gate, const void *key,
                                           const void *value, void *output, void *kv_cache,
                                           std::size_t kv_cache_bytes, Qwen35AttentionShape shape,
                                           Qwen35FusedNormRope norm, Qwen35KvCacheDType cache_dtype,
                                           Qwen35KvCacheLayout layout, hipStream_t stream) {
  require<Err>(query_gate != nullptr, "online attention query pointer is null");
  require<Err>(key != nullptr, "online attention key pointer is null");
  require<Err>(value != nullptr, "online attention value pointer is null");
  require<Err>(output != nullptr, "online attention output pointer is null");
  require<Err>(kv_cache != nullptr, "online attention KV cache pointer is null");
  require<Err>(stream != nullptr, "online attention HIP stream is null");
  require<Err>(online_prefill_signature_supported(shape, RAFTINFER_DTYPE_BF16, cache_dtype, layout),
               "unsupported online attention prefill signature; select the "
               "materialized implementation before allocation");
  require<Err>(cache_dtype == Qwen35KvCacheDType::bf16 && shape.query_heads == kQueryHeads &&
                   shape.kv_heads == kKvHeads && shape.head_dim == kHeadDim,
               "fused prefill requires the model signature with a bf16 KV cache");
  const std::size_t required = checked_mul<Err>(
      checked_mul<Err>(2, checked_mul<Err>(shape.max_context_tokens, kKvHeads * kHeadDim,
                                           "online attention cache shape overflow"),
                       "online attention cache shape overflow"),
      2, "online attention cache byte size overflow");
  require<Err>(kv_cache_bytes >= required, "online attention KV cache is too small");
  require<Err>(norm.query_norm_weight != nullptr && norm.key_norm_weight != nullptr,
               "fused prefill norm weight pointer is null");
  require<Err>(norm.weight_dtype == RAFTINFER_DTYPE_BF16 || norm.weight_dtype == RAFTINFER_DTYPE_F32,
               "fused prefill norm weights must be bf16 or f32");
  require<Err>(norm.rotary_dim > 0 && norm.rotary_dim <= kHeadDim && norm.rotary_dim % 8 == 0,
               "fused prefill rotary_dim must be a positive multiple of 8 up to 256");
  require<Err>(std::isfinite(norm.rope_base) && norm.rope_base > 0.0f,
               "qk_norm_rope rope_base must be finite and positive");
  require<Err>(std::isfinite(norm.epsilon) && norm.epsilon >= 0.0f,
               "qk_norm_rope epsilon must be finite and non-negative");
  const auto bits = [](const void *p) { return reinterpret_cast<std::uintptr_t>(p); };
  const std::size_t wa = norm.weight_dtype == RAFTINFER_DTYPE_F32 ? 16 : 8;
  require<Err>(((bits(norm.query_norm_weight) | bits(norm.key_norm_weight)) & (wa - 1)) == 0,
               "fused prefill norm weights are not vector-aligned");
  require<Err>(((bits(query_gate) | bits(kv_cache)) & 15u) == 0 &&
                   ((bits(key) | bits(value) | bits(output)) & 7u) == 0,
               "fused prefill needs 16-byte aligned q projection and cache, 8-byte aligned key, "
               "value and output");
  amd::launch_prefill_mfma_fused(
      static_cast<const bf16_bits *>(query_gate), static_cast<const bf16_bits *>(key),
      static_cast<const bf16_bits *>(value), static_cast<bf16_bits *>(output),
      static_cast<bf16_bits *>(kv_cache), shape.tokens, shape.max_context_tokens, shape.past_tokens,
      layout == Qwen35KvCacheLayout::head_major, norm.query_norm_weight, norm.key_norm_weight,
      norm.weight_dtype == RAFTINFER_DTYPE_F32, static_cast<int>(norm.rotary_dim / 2),
      std::pow(static_cast<double>(norm.rope_base), -2.0 / static_cast<double>(norm.rotary_dim)),
      norm.epsilon, stream);
  check_launch<Err>("qwen35_online_attention_prefill_fused");
}

// --------------------------------------------------------- dispatcher
// cpp/kernels/qwen35_attention.cu:463-613
void qwen35_causal_attention(const void *query, const void *key, const void *value,
                             const void *gate, void *output, void *kv_cache,
                             std::size_t kv_cache_bytes, void *workspace,
                             std::size_t workspace_bytes, Qwen35AttentionShape shape,
                             RaftInferDataType act, Qwen35AttentionLaunchPolicy policy,
                             hipStream_t stream) {
  const std::size_t required_workspace = qwen35_attention_workspace_bytes(shape, policy);
  validate_attention_pointers(query, key, value, gate, output, kv_cache, workspace,
                              required_workspace, stream);
  require<Err>(kv_cache_bytes >= qwen35_attention_cache_bytes(shape, policy),
               "attention KV cache is too small");
  require<Err>(workspace_bytes >= required_workspace, "attention workspace is too small");
  require_dtype(act);

  if (policy.implementation == Qwen35AttentionImplementation::materialized_reference) {
    require<Err>(policy.kv_cache_layout == Qwen35KvCacheLayout::token_major,
                 "materialized attention requires a token-major KV cache");
    require<Err>(policy.kv_cache_dtype == Qwen35KvCacheDType::f32,
                 "materialized attention requires an F32 KV cache");
    auto *cache = static_cast<float *>(kv_cache);
    auto *logits = static_cast<float *>(workspace);
    if (act == RAFTINFER_DTYPE_F32)
      launch_materialized<float>(query, key, value, gate, output, cache, logits, shape, stream);
    else if (act == RAFTINFER_DTYPE_F16)
      launch_materialized<_Float16>(query, key, value, gate, output, cache, logits, shape, stream);
    else
      launch_materialized<bf16_bits>(query, key, value, gate, output, cache, logits, shape, stream);
    return;
  }
  require<Err>(workspace == nullptr && workspace_bytes == 0,
               "online tiled attention forbids logits workspace");
  if (shape.tokens == 1) {
    qwen35_online_attention_decode(query, key, value, gate, output, kv_cache, kv_cache_bytes,
                                   shape, act, policy.kv_cache_dtype, policy.kv_cache_layout,
                                   nullptr, stream);
    return;
  }
  require<Err>(qwen35_online_attention_prefill_supported(shape, act, policy),
               "unsupported online tiled prefill signature; select the "
               "materialized implementation before allocation");
  qwen35_online_attention_prefill(query, key, value, gate, output, kv_cache, kv_cache_bytes, shape,
                                  act, policy.kv_cache_dtype, policy.kv_cache_layout, stream);
}

void qwen35_causal_attention(const void *query, const void *key, const void *value,
                             const void *gate, void *output, float *kv_cache,
                             float *logits_workspace, std::size_t logits_workspace_floats,
                             Qwen35AttentionShape shape, RaftInferDataType dtype,
                             hipStream_t stream) {
  const Qwen35AttentionLaunchPolicy policy{Qwen35AttentionImplementation::materialized_reference,
                                           Qwen35KvCacheDType::f32,
                                           Qwen35KvCacheLayout::token_major};
  qwen35_causal_attention(query, key, value, gate, output, kv_cache,
                          qwen35_attention_cache_bytes(shape, policy), logits_workspace,
                          checked_mul<Err>(logits_workspace_floats, sizeof(float),
                                           "attention workspace byte size overflow"),
                          shape, dtype, policy, stream);
}

} // namespace raftinfer::kernels
