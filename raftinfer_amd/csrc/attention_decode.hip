// Online decode attention for gfx950: KV append, zero-workspace single-block
// decode, split-K partitions with an fp32 log-sum-exp merge, the decode plan
// and workspace layout, and the batched ragged decode.
//
// Host semantics (validation order, messages, plan/layout arithmetic) follow
// cpp/kernels/qwen35_online_attention.cu:27-196 and :1071-1328.  Device work is
// this build's own: one workgroup per (KV head, partition) serves the four
// query heads of the GQA group, so each K/V byte is read from HBM once.
#include "decode_mfma.hpp"
#include "decode_scan.hpp"
#include "norm_rope.hpp"
#include "raftinfer_amd/qwen35_online_attention.hpp"

#include <algorithm>
#include <atomic>
#include <bit>
#include <type_traits>
#include <cmath>
#include <mutex>

namespace raftinfer::kernels {
namespace {

using namespace raftinfer::amd;
using Err = Qwen35PrimitiveError;

constexpr std::size_t kMinimumContextBucketTokens = 512;
constexpr Qwen35DecodeAttentionMode kDefaultOnlineDecodeMode = Qwen35DecodeAttentionMode::split_k_256;

__device__ unsigned int g_capacity_errors = 0;

bool multiplication_fits(std::size_t a, std::size_t b) noexcept {
  return a == 0 || b <= std::numeric_limits<std::size_t>::max() / a;
}

std::size_t cache_element_bytes_of(Qwen35KvCacheDType dtype) noexcept {
  switch (dtype) {
  case Qwen35KvCacheDType::f32: return sizeof(float);
  case Qwen35KvCacheDType::bf16: return sizeof(bf16_bits);
  }
  return 0;
}

bool layout_known(Qwen35KvCacheLayout layout) noexcept {
  return layout == Qwen35KvCacheLayout::token_major || layout == Qwen35KvCacheLayout::head_major;
}

// cpp/kernels/qwen35_online_attention.cu:96-139
bool online_decode_signature_supported(Qwen35AttentionShape shape, RaftInferDataType act,
                                       Qwen35KvCacheDType cache_dtype,
                                       Qwen35KvCacheLayout layout) noexcept {
  if (shape.tokens != 1 || shape.query_heads != 16 || shape.kv_heads != 4 ||
      shape.head_dim != 256 || shape.max_context_tokens == 0 ||
      shape.past_tokens >= shape.max_context_tokens)
    return false;
  if (act != RAFTINFER_DTYPE_F32 && act != RAFTINFER_DTYPE_BF16) return false;
  const std::size_t eb = cache_element_bytes_of(cache_dtype);
  if (eb == 0 || !layout_known(layout)) return false;
  const std::size_t kv_size = shape.kv_heads * shape.head_dim;
  if (!multiplication_fits(shape.max_context_tokens, kv_size)) return false;
  const std::size_t plane = shape.max_context_tokens * kv_size;
  return multiplication_fits(2, plane) && multiplication_fits(2 * plane, eb);
}

// cpp/kernels/qwen35_online_attention.cu:141-145
bool model_signature(Qwen35AttentionShape shape) noexcept {
  return shape.tokens == 1 && shape.query_heads == 16 && shape.kv_heads == 4 &&
         shape.head_dim == 256 && shape.max_context_tokens != 0;
}

std::size_t ceil_div(std::size_t n, std::size_t d, const char *message) {
  require<Err>(d != 0, message);
  return n / d + (n % d == 0 ? 0 : 1);
}

// Partition length of a resolved mode (cpp/kernels/qwen35_online_attention.cu:
// 171-183): the split modes name theirs, the others have none.
std::size_t partition_tokens_for_mode(Qwen35DecodeAttentionMode mode) {
  if (mode == Qwen35DecodeAttentionMode::split_k_256) return 256;
  if (mode == Qwen35DecodeAttentionMode::split_k_512) return 512;
  require<Err>(mode == Qwen35DecodeAttentionMode::single_block ||
                   mode == Qwen35DecodeAttentionMode::auto_select,
               "unsupported online decode attention mode");
  return 0;
}

// The context bucket (the plan's context_bucket_tokens, which fixes the
// partition capacity a captured decode graph is built for): the smallest
// power of two that is at least 512 and at least the context, capped at the
// maximum context.  A context beyond the largest power of two a size_t holds
// gets the maximum context.  The reference reaches the same value by doubling
// 512 in a loop (cpp/kernels/qwen35_online_attention.cu:185-196); the plan
// tests compare the two over every boundary.
std::size_t context_bucket_tokens(Qwen35AttentionShape shape, std::size_t context_tokens) {
  static_assert(std::has_single_bit(kMinimumContextBucketTokens));
  constexpr std::size_t kTopPower = std::size_t{1} << (std::numeric_limits<std::size_t>::digits - 1);
  std::size_t bucket = kMinimumContextBucketTokens;
  if (context_tokens > kTopPower)
    bucket = shape.max_context_tokens;
  else if (context_tokens > bucket)
    bucket = std::bit_ceil(context_tokens);
  return std::min(bucket, shape.max_context_tokens);
}

int grid_dim(std::size_t value, const char *message) {
  require<Err>(value <= static_cast<std::size_t>(std::numeric_limits<int>::max()), message);
  return static_cast<int>(value);
}

// ------------------------------------------------------------- kernels

__device__ __forceinline__ std::size_t read_position(const std::uint32_t *device_position,
                                                     std::size_t host_position) {
  return device_position == nullptr ? host_position : static_cast<std::size_t>(*device_position);
}

// Writes one token's K and V (4 x 256 each) at the position, RNE-cast to
// the cache dtype.  Grid: 4 x 256.
template <typename ActT, typename CacheT>
__global__ __launch_bounds__(256) void append_decode_kernel(
    const ActT *__restrict__ key, const ActT *__restrict__ value, CacheT *__restrict__ cache,
    std::size_t max_ctx, std::size_t host_position, bool head_major,
    const std::uint32_t *device_position) {
  const std::size_t position = read_position(device_position, host_position);
  if (position >= max_ctx) return;
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  const int kvh = e >> 8;
  const int d = e & 255;
  const std::size_t idx = cache_row(head_major, position, kvh, max_ctx) + d;
  const std::size_t plane = max_ctx * kKvHeads * kHeadDim;
  Elem<CacheT>::store(cache, idx, Elem<ActT>::load(key, e));
  Elem<CacheT>::store(cache, plane + idx, Elem<ActT>::load(value, e));
}

// Zero-workspace single-block decode: one workgroup per group of NH query
// heads scans the whole context and writes the gated output.  Exits when the
// plan's split threshold is reached (mirrors the device-side early exit of
// cpp/kernels/qwen35_online_attention.cu:427-430).
template <typename ActT, typename CacheT, int NH, int WAVES, int U>
__global__ __launch_bounds__(WAVES * 64) void decode_single_block_kernel(
    const ActT *__restrict__ query, const ActT *__restrict__ gate, ActT *__restrict__ output,
    const CacheT *__restrict__ cache, std::size_t max_ctx, std::size_t host_position,
    bool head_major, const std::uint32_t *device_position, std::size_t threshold) {
  __shared__ ScanShared<NH, WAVES> sh;
  const std::size_t position = read_position(device_position, host_position);
  if (position >= max_ctx) return;
  const std::size_t ctx = position + 1;
  if (threshold != 0 && ctx >= threshold) return;
  const std::size_t first_head = static_cast<std::size_t>(blockIdx.x) * NH;
  const std::size_t kv_head = first_head / kGroup;
  const CacheT *k_plane = cache;
  const CacheT *v_plane = cache + max_ctx * kKvHeads * kHeadDim;
  scan_range<ActT, CacheT, NH, WAVES, U>(query, first_head, k_plane, v_plane, head_major, max_ctx,
                                         kv_head, 0, ctx, sh);
  __syncthreads();
  for (int o = threadIdx.x; o < NH * kHeadDim; o += WAVES * 64) {
    const int h = o / kHeadDim, d = o % kHeadDim;
    float mm, l, a;
    combine_waves(sh, h, d, mm, l, a);
    const std::size_t out_idx = (first_head + h) * kHeadDim + d;
    const float gv = Elem<ActT>::load(gate, out_idx);
    Elem<ActT>::store(output, out_idx, (a / l) * sigmoid_gate(gv));
  }
}

// Split-K partition: workgroup (head group, partition p) scans tokens
// [p*P, min(ctx, (p+1)*P)) and writes fp32 (max, sum, value[256]) per query
// head at index qh*max_partitions + p, the reference workspace bookkeeping
// (cpp/kernels/qwen35_online_attention.cu:602-691).
template <typename ActT, typename CacheT, int NH, int WAVES, int U>
__global__ __launch_bounds__(WAVES * 64) void decode_partition_kernel(
    const ActT *__restrict__ query, const CacheT *__restrict__ cache, float *__restrict__ pmax,
    float *__restrict__ psum, float *__restrict__ pval, std::size_t max_ctx,
    std::size_t host_position, bool head_major, std::size_t capacity,
    std::size_t max_partitions, std::size_t partition_tokens, std::size_t threshold,
    const std::uint32_t *device_position) {
  __shared__ ScanShared<NH, WAVES> sh;
  const std::size_t position = read_position(device_position, host_position);
  if (position >= max_ctx) return;
  const std::size_t ctx = position + 1;
  if (ctx < threshold) return;
  const std::size_t unit = blockIdx.x / capacity;
  const std::size_t partition = blockIdx.x % capacity;
  const std::size_t begin = partition * partition_tokens;
  if (begin >= ctx) return;
  const std::size_t end = ctx < begin + partition_tokens ? ctx : begin + partition_tokens;
  const std::size_t first_head = unit * NH;
  const std::size_t kv_head = first_head / kGroup;
  const CacheT *k_plane = cache;
  const CacheT *v_plane = cache + max_ctx * kKvHeads * kHeadDim;
  scan_range<ActT, CacheT, NH, WAVES, U>(query, first_head, k_plane, v_plane, head_major, max_ctx,
                                         kv_head, begin, end, sh);
  __syncthreads();
  for (int o = threadIdx.x; o < NH * kHeadDim; o += WAVES * 64) {
    const int h = o / kHeadDim, d = o % kHeadDim;
    float mm, l, a;
    combine_waves(sh, h, d, mm, l, a);
    const std::size_t idx = (first_head + h) * max_partitions + partition;
    if (d == 0) {
      pmax[idx] = mm * kLn2;
      psum[idx] = l;
    }
    pval[idx * kHeadDim + d] = a;
  }
}

// Log-sum-exp merge over the active partitions of one query head plus the
// sigmoid gate (cpp/kernels/qwen35_online_attention.cu:693-756).  The value
// loads of a chunk do not wait for its max / sum, so they are all independent.
// A device position needing more partitions than
// the plan's capacity writes NaN and counts a capacity error instead of
// trapping.
constexpr int kMergeChunkShort = 16; // partitions per round trip (capacity at most 16)
constexpr int kMergeDims = 64;       // dims per merge workgroup (one thread each)

// Merges the partials of one head online over chunks of CH partitions;
// the calling thread owns output dim d.  Lane u of every wave reads the
// max and sum of partition base + u, the chunk max and the sum of weighted
// sums are lane reductions, and lane u's weight reaches the other lanes by
// v_readlane.  Every load of a chunk is issued before any is used, so a
// chunk costs one memory round trip.
template <int CH>
__device__ __forceinline__ void merge_head(int d, const float *__restrict__ pmax,
                                           const float *__restrict__ psum,
                                           const float *__restrict__ pval, std::size_t first,
                                           std::size_t active, float &l_out, float &a_out) {
  const int lane = threadIdx.x & 63;
  float m = -INFINITY, l = 0.f, a = 0.f;
  for (std::size_t base = 0; base < active; base += CH) {
    const std::size_t n = active - base < CH ? active - base : CH;
    const std::size_t pl = first + base + (static_cast<std::size_t>(lane) < n ? lane : n - 1);
    const float mraw = pmax[pl];
    const float sraw = psum[pl];
    float vx[CH];
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const std::size_t p = first + base + (static_cast<std::size_t>(u) < n ? u : n - 1);
      vx[u] = pval[p * kHeadDim + d];
    }
    const bool mine = static_cast<std::size_t>(lane) < n;
    const float ml = mine ? mraw : -INFINITY;
    const float cm = fmaxf(m, max_xor32(max_xor16(row16_max(ml))));
    const float r = __expf(m - cm); // m = -inf on the first chunk -> 0
    const float w = mine ? __expf(ml - cm) : 0.f;
    l = fmaf(l, r, sum_xor32(sum_xor16(row16_sum(sraw * w))));
    a *= r;
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      if (static_cast<std::size_t>(u) < n)
        a = fmaf(vx[u], __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), u)), a);
    }
    m = cm;
  }
  l_out = l;
  a_out = a;
}

template <typename ActT, int CH>
__global__ __launch_bounds__(kMergeDims) void decode_merge_kernel(
    const ActT *__restrict__ gate, std::size_t gate_stride, ActT *__restrict__ output,
    const float *__restrict__ pmax,
    const float *__restrict__ psum, const float *__restrict__ pval, std::size_t max_ctx,
    std::size_t host_position, std::size_t partition_tokens, std::size_t max_partitions,
    std::size_t capacity, std::size_t threshold, const std::uint32_t *device_position) {
  const std::size_t position = read_position(device_position, host_position);
  if (position >= max_ctx) return;
  const std::size_t ctx = position + 1;
  if (ctx < threshold) return;
  const std::size_t active = ctx / partition_tokens + (ctx % partition_tokens ? 1 : 0);
  // Workgroup = (head, block of kMergeDims dims); thread = dim.
  const std::size_t head = blockIdx.x / (kHeadDim / kMergeDims);
  const int d = static_cast<int>(blockIdx.x % (kHeadDim / kMergeDims)) * kMergeDims + threadIdx.x;
  const std::size_t out_idx = head * kHeadDim + d;
  if (active > capacity) {
    if (blockIdx.x == 0 && threadIdx.x == 0) atomicAdd(&g_capacity_errors, 1u);
    Elem<ActT>::store(output, out_idx, __builtin_nanf(""));
    return;
  }
  const float gv = Elem<ActT>::load(gate, head * gate_stride + d);
  float l, a;
  merge_head<CH>(d, pmax, psum, pval, head * max_partitions, active, l, a);
  Elem<ActT>::store(output, out_idx, (a / l) * sigmoid_gate(gv));
}

// Row merge for plans of more than 16 partitions and for the batched path:
// the same log-sum-exp merge, laid out for many partitions per head.  Workgroup = one head, W waves.  Wave w merges
// partitions w, w+W, w+2W, ... online, in chunks of kRowChunk; lane l owns
// dims 4l..4l+3, so every value load of a wave is one whole 1 KiB partial row
// (the quarter-row loads of merge_head took twice as long on the same bytes
// here).  The W waves' (max, sum, weighted row) then combine in LDS, thread d
// finishing dim d.  At 16 partitions (a 4096-token context) the 64-workgroup
// merge_head layout is faster: the call is latency-bound there.
constexpr int kRowChunk = 16;
constexpr int kBatchedMergeWaves = 8; // 128 partitions (32768 tokens) in one round trip
constexpr int kLongMergeWaves = 8;    // split-K merge of more than 16 partitions

template <int W> struct RowMergeShared {
  float a[W][kHeadDim];
  float m[W], l[W];
};

template <int W>
__device__ __forceinline__ void merge_rows(const float *__restrict__ pmax,
                                           const float *__restrict__ psum,
                                           const float *__restrict__ pval, std::size_t first,
                                           std::size_t active, RowMergeShared<W> &sh) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const std::size_t mine_total =
      active > static_cast<std::size_t>(wave) ? (active - wave + W - 1) / W : 0;
  const std::size_t own = first + wave;
  float m = -INFINITY, l = 0.f;
  float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
  for (std::size_t base = 0; base < mine_total; base += kRowChunk) {
    const std::size_t n = mine_total - base < kRowChunk ? mine_total - base : kRowChunk;
    const std::size_t pl = own + W * (base + (static_cast<std::size_t>(lane) < n ? lane : n - 1));
    const float mraw = pmax[pl];
    const float sraw = psum[pl];
    float4 vx[kRowChunk];
#pragma unroll
    for (int u = 0; u < kRowChunk; ++u) {
      const std::size_t p = own + W * (base + (static_cast<std::size_t>(u) < n ? u : n - 1));
      vx[u] = reinterpret_cast<const float4 *>(pval + p * kHeadDim)[lane];
    }
    const bool mine = static_cast<std::size_t>(lane) < n;
    const float ml = mine ? mraw : -INFINITY;
    const float cm = fmaxf(m, max_xor32(max_xor16(row16_max(ml))));
    const float r = __expf(m - cm); // m = -inf on the first chunk -> 0
    const float w = mine ? __expf(ml - cm) : 0.f;
    l = fmaf(l, r, sum_xor32(sum_xor16(row16_sum(sraw * w))));
    a.x *= r;
    a.y *= r;
    a.z *= r;
    a.w *= r;
#pragma unroll
    for (int u = 0; u < kRowChunk; ++u) {
      if (static_cast<std::size_t>(u) < n) {
        const float wu =
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), u));
        a.x = fmaf(vx[u].x, wu, a.x);
        a.y = fmaf(vx[u].y, wu, a.y);
        a.z = fmaf(vx[u].z, wu, a.z);
        a.w = fmaf(vx[u].w, wu, a.w);
      }
    }
    m = cm;
  }
  reinterpret_cast<float4 *>(sh.a[wave])[lane] = a;
  if (lane == 0) {
    sh.m[wave] = m;
    sh.l[wave] = l;
  }
}

// After merge_rows and a barrier: the merged, normalised value of dim d.  A
// wave without partitions left max -inf, sum 0 and a zero row; it weighs 0.
template <int W>
__device__ __forceinline__ float combine_rows(const RowMergeShared<W> &sh, int d) {
  float mm = sh.m[0];
#pragma unroll
  for (int v = 1; v < W; ++v) mm = fmaxf(mm, sh.m[v]);
  float lt = 0.f, at = 0.f;
#pragma unroll
  for (int v = 0; v < W; ++v) {
    const float e = sh.m[v] == -INFINITY ? 0.f : __expf(sh.m[v] - mm);
    lt = fmaf(sh.l[v], e, lt);
    at = fmaf(sh.a[v][d], e, at);
  }
  return at / lt;
}

template <typename ActT, int W>
__global__ __launch_bounds__(W * 64) void decode_merge_rows_kernel(
    const ActT *__restrict__ gate, std::size_t gate_stride, ActT *__restrict__ output,
    const float *__restrict__ pmax,
    const float *__restrict__ psum, const float *__restrict__ pval, std::size_t max_ctx,
    std::size_t host_position, std::size_t partition_tokens, std::size_t max_partitions,
    std::size_t capacity, std::size_t threshold, const std::uint32_t *device_position) {
  __shared__ RowMergeShared<W> sh;
  const std::size_t position = read_position(device_position, host_position);
  if (position >= max_ctx) return;
  const std::size_t ctx = position + 1;
  if (ctx < threshold) return;
  const std::size_t active = ctx / partition_tokens + (ctx % partition_tokens ? 1 : 0);
  const std::size_t head = blockIdx.x;
  const int d = threadIdx.x & (kHeadDim - 1);
  const std::size_t out_idx = head * kHeadDim + d;
  const bool finisher = threadIdx.x < kHeadDim;
  if (active > capacity) {
    if (blockIdx.x == 0 && threadIdx.x == 0) atomicAdd(&g_capacity_errors, 1u);
    if (finisher) Elem<ActT>::store(output, out_idx, __builtin_nanf(""));
    return;
  }
  const float gv = finisher ? Elem<ActT>::load(gate, head * gate_stride + d) : 0.f;
  merge_rows<W>(pmax, psum, pval, head * max_partitions, active, sh);
  __syncthreads();
  if (finisher) Elem<ActT>::store(output, out_idx, combine_rows<W>(sh, d) * sigmoid_gate(gv));
}

// ---- bf16 activations + bf16 cache: MFMA scores, dims-sliced workgroups.
constexpr int kSplitDs = 4, kSplitWaves = 8;
// Tokens per wave step of the split-K partition scan.  With all 256 dims in
// one workgroup (DS = 1, long contexts) 16-token steps halve the K/V
// registers of a step, which measured faster (ctx 16384 cold 19.5 -> 18.1 us
// per call); with sliced dims 32-token steps are as fast or faster.
constexpr int split_chunk(int ds) { return ds == 1 ? 16 : 32; }
constexpr int kSingleDs = 16, kSingleMfmaWaves = 8;
// Tokens per wave step of the register-fed single-block scan: 16 rather than
// 32 halves the registers a step holds (ctx 512 cold 8.5 -> 8.15 us, hot
// 7.25 -> 6.95 us; 16 waves per workgroup measured slower).  The LDS-staged
// scan keeps 32-token chunks.
constexpr int kSingleChunk = 16;

// Copies the new token's K and V rows of kv_head into the cache (bf16 to
// bf16, so the stored bits equal the RNE cast of the reference's append).
__device__ __forceinline__ void append_rows(const DecodeMfmaArgs &a, std::size_t kv_head,
                                            std::size_t pos) {
  const int t = threadIdx.x;
  if (t < kHeadDim / 8) {
    const std::size_t row = cache_row(a.head_major, pos, kv_head, a.max_ctx) + 8 * t;
    const std::size_t plane = a.max_ctx * kKvHeads * kHeadDim;
    *reinterpret_cast<u32x4 *>(a.cache_rw + row) =
        *reinterpret_cast<const u32x4 *>(a.key_new + kv_head * kHeadDim + 8 * t);
    *reinterpret_cast<u32x4 *>(a.cache_rw + plane + row) =
        *reinterpret_cast<const u32x4 *>(a.value_new + kv_head * kHeadDim + 8 * t);
  }
}

// The producers fused into a decode step (qwen35_split_query_gate_norm_rope of
// q and qwen35_qk_norm_rope of k, cpp/kernels/qwen35_primitives.cu:158-210):
// the raw q projection rows [16][2][256] (the query half is normalised and
// rotated in the kernel, the gate half read by the output stage), the raw key
// row [4][256], the norm weights and the RoPE parameters.
struct FusedNormRope {
  const bf16_bits *query_gate;
  const bf16_bits *key;
  const void *q_weight;
  const void *k_weight;
  bool weight_f32;
  int pairs;    // rotary_dim / 2
  double ratio; // rope_base^(-2 / rotary_dim)
  float epsilon;
};

// RMSNorm + RoPE of the group's four q heads and of its key row at
// `position`, into LDS (waves 0..3: q heads, wave 4: k; the workgroup has at
// least 5 waves), with exactly the arithmetic of the producer kernels.
// Its loads and its arithmetic are split so that a caller can issue other
// loads in between (fused_qk_load, then fused_qk_finish).
struct FusedQKRows { // raw bits: converting them at the load would wait for it there
  u32x2 x;
  u32x2 w0, w1; // f32 weights (w0, w1), or bf16 weights (w0; w1 re-reads them)
};
__device__ __forceinline__ FusedQKRows fused_qk_load(const FusedNormRope &f, std::size_t kv_head) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // Waves past the group read the first row; their values are not used.
  const int row = wave <= kGroup ? wave : 0;
  const bf16_bits *src = row < kGroup ? f.query_gate + (kv_head * kGroup + row) * 2 * kHeadDim
                                      : f.key + kv_head * kHeadDim;
  const auto *wp = static_cast<const unsigned char *>(row < kGroup ? f.q_weight : f.k_weight);
  // Unconditional loads (the address, not the load, depends on the weight
  // type), so no value is merged across branches.
  const std::size_t w0 = f.weight_f32 ? 16u * lane : 8u * lane;
  const std::size_t w1 = f.weight_f32 ? 16u * lane + 8u : 8u * lane;
  return FusedQKRows{*reinterpret_cast<const u32x2 *>(src + 4 * lane), *reinterpret_cast<const u32x2 *>(wp + w0),
                     *reinterpret_cast<const u32x2 *>(wp + w1)};
}
// The rotation table of `position` (read after the next barrier).  It runs
// before the loads are issued: with the loaded raw values live across its
// per-lane branches, the compiler reused one of their registers inside them.
__device__ __forceinline__ void fused_qk_rot(const FusedNormRope &f, std::size_t position, DecodeFusedQK &fq) {
  const int tid = threadIdx.x;
  if (tid < f.pairs) {
    float cs, sn;
    rope_cos_sin(tid, position, f.ratio, cs, sn);
    fq.rot[tid] = cs;
    fq.rot[f.pairs + tid] = sn;
  }
}
__device__ __forceinline__ void fused_qk_finish(const FusedNormRope &f, const FusedQKRows &r, DecodeFusedQK &fq) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  __syncthreads();
  if (wave <= kGroup) {
    const float x[4] = {bf16_lo(r.x[0]), bf16_hi(r.x[0]), bf16_lo(r.x[1]), bf16_hi(r.x[1])};
    float w[4];
    if (f.weight_f32) {
      // (Element by element through a scalar: this compiler's
      // __builtin_bit_cast of a vector element reads element 0.)
      const std::uint32_t b[4] = {r.w0[0], r.w0[1], r.w1[0], r.w1[1]};
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = __builtin_bit_cast(float, b[e]);
    } else {
      w[0] = bf16_lo(r.w0[0]); w[1] = bf16_hi(r.w0[0]); w[2] = bf16_lo(r.w0[1]); w[3] = bf16_hi(r.w0[1]);
    }
    float v[4];
    norm_rope_256_lane(x, w, lane, f.pairs, fq.rot, f.epsilon, v);
    bf16_bits *dst = wave < kGroup ? fq.q[wave] : fq.k;
    *reinterpret_cast<u32x2 *>(dst + 4 * lane) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  }
  __syncthreads();
}
__device__ __forceinline__ void fused_qk_prologue(const FusedNormRope &f, std::size_t kv_head,
                                                  std::size_t position, DecodeFusedQK &fq) {
  fused_qk_rot(f, position, fq);
  fused_qk_finish(f, fused_qk_load(f, kv_head), fq);
}

// The fused form of append_rows: the key row comes from LDS (normalised and
// rotated by fused_qk_prologue), the value row from the input.
__device__ __forceinline__ void append_rows_fused(const DecodeMfmaArgs &a, const DecodeFusedQK &fq,
                                                  std::size_t kv_head, std::size_t pos) {
  const int t = threadIdx.x;
  if (t < kHeadDim / 8) {
    const std::size_t row = cache_row(a.head_major, pos, kv_head, a.max_ctx) + 8 * t;
    const std::size_t plane = a.max_ctx * kKvHeads * kHeadDim;
    *reinterpret_cast<u32x4 *>(a.cache_rw + row) = *reinterpret_cast<const u32x4 *>(&fq.k[8 * t]);
    *reinterpret_cast<u32x4 *>(a.cache_rw + plane + row) =
        *reinterpret_cast<const u32x4 *>(a.value_new + kv_head * kHeadDim + 8 * t);
  }
}

// gate: element (head h, dim d) at gate[h * gate_stride + d] (gate_stride 256
// for a split gate, 512 for the gate half of a q projection row).
// Single-block workgroup `block` at `position` (ctx = position + 1).
template <int DS, int WAVES, bool kFused, bool kDma = false, int CT = 32>
__device__ __forceinline__ void single_block_body(unsigned block, const DecodeMfmaArgs &a,
                                                  const bf16_bits *__restrict__ gate,
                                                  std::size_t gate_stride,
                                                  bf16_bits *__restrict__ output,
                                                  std::size_t position, const FusedNormRope &f,
                                                  DecodeMfmaShared<DS, WAVES, CT> &sh, DecodeFusedQK &fq,
                                                  DecodeStage<DS, WAVES, CT> *stage = nullptr) {
  constexpr int DIMS = kHeadDim / DS;
  const std::size_t ctx = position + 1;
  std::size_t kv_head;
  int dq;
  xcd_unit<DS>(block, kv_head, dq);
  if (kv_head >= kKvHeads) return;
  __shared__ unsigned prefetch_sink[64];
  prefetch_head_rows<DS, WAVES>(a, kv_head, dq, ctx, lds_address(&prefetch_sink[0]));
  // The gate values of this thread's outputs are loaded before the scan, so
  // the epilogue does not wait for a load round trip of its own.
  // kDma: unconditional (index clamped) with the raw bits kept until the
  // epilogue, since a conditional load converted on the spot is waited for
  // right here, before the stage loads go out.
  constexpr int kOut = (kGroup * DIMS + WAVES * 64 - 1) / (WAVES * 64);
  float gv[kOut];
  [[maybe_unused]] bf16_bits graw[kOut];
#pragma unroll
  for (int n = 0; n < kOut; ++n) {
    const int o = threadIdx.x + n * WAVES * 64;
    if constexpr (kDma) {
      const int oc = o < kGroup * DIMS ? o : kGroup * DIMS - 1;
      graw[n] = gate[(kv_head * kGroup + oc / DIMS) * gate_stride + dq * DIMS + oc % DIMS];
    } else {
      gv[n] = 0.f;
      if (o < kGroup * DIMS)
        gv[n] = bf16_to_f32(gate[(kv_head * kGroup + o / DIMS) * gate_stride + dq * DIMS + o % DIMS]);
    }
  }
  if constexpr (kFused) fused_qk_prologue(f, kv_head, position, fq);
  decode_mfma_scan<DS, WAVES, CT, kFused, kDma>(a, kv_head, dq, 0, ctx, position, sh, &fq, stage);
  __syncthreads();
  // The scan read the new row from key/value; the cache copy goes last so its
  // load latency is not on the critical path.
  if (dq == 0) {
    if constexpr (kFused)
      append_rows_fused(a, fq, kv_head, position);
    else
      append_rows(a, kv_head, position);
  }
#pragma unroll
  for (int n = 0; n < kOut; ++n) {
    const int o = threadIdx.x + n * WAVES * 64;
    if (o >= kGroup * DIMS) break;
    const int h = o / DIMS, d = o % DIMS;
    float mm, l, acc;
    decode_mfma_combine(sh, h, d, mm, l, acc);
    const std::size_t idx = (kv_head * kGroup + h) * kHeadDim + dq * DIMS + d;
    if constexpr (kDma) gv[n] = bf16_to_f32(graw[n]);
    output[idx] = f32_to_bf16((acc / l) * sigmoid_gate(gv[n]));
  }
}

// kDma: K and V reach the scan through an LDS stage (DecodeStage, 146 KiB).
template <int DS, int WAVES, bool kFused = false, bool kDma = false>
__global__ __launch_bounds__(WAVES * 64) void decode_single_mfma_kernel(
    DecodeMfmaArgs a, const bf16_bits *__restrict__ gate, std::size_t gate_stride,
    bf16_bits *__restrict__ output, std::size_t host_position, const std::uint32_t *device_position,
    std::size_t threshold, FusedNormRope f) {
  constexpr int CT = kDma ? 32 : kSingleChunk;
  __shared__ DecodeMfmaShared<DS, WAVES, CT> sh;
  __shared__ DecodeFusedQK fq;
  using Stage = std::conditional_t<kDma, DecodeStage<DS, WAVES>, char>;
  __shared__ Stage stage;
  const std::size_t position = read_position(device_position, host_position);
  if (position >= a.max_ctx) return;
  if (threshold != 0 && position + 1 >= threshold) return;
  if constexpr (kDma)
    single_block_body<DS, WAVES, kFused, true>(blockIdx.x, a, gate, gate_stride, output, position, f, sh, fq,
                                               &stage);
  else
    single_block_body<DS, WAVES, kFused, false, CT>(blockIdx.x, a, gate, gate_stride, output, position, f, sh, fq);
}

// Split-K partition workgroup `block` at `position`.
template <int DS, int WAVES, int CT, bool kFused>
__device__ __forceinline__ void split_body(unsigned block, const DecodeMfmaArgs &a,
                                           float *__restrict__ pmax, float *__restrict__ psum,
                                           float *__restrict__ pval, std::size_t position,
                                           std::size_t capacity, std::size_t max_partitions,
                                           std::size_t partition_tokens, const FusedNormRope &f,
                                           DecodeMfmaShared<DS, WAVES, CT> &sh, DecodeFusedQK &fq) {
  constexpr int DIMS = kHeadDim / DS;
  const std::size_t ctx = position + 1;
  std::size_t unit;
  int dq;
  xcd_unit<DS>(block, unit, dq);
  if (unit >= kKvHeads * capacity) return;
  // All dims per workgroup (long contexts): the four KV heads of a partition
  // run side by side, which streams the cache faster than consecutive
  // partitions of one head (ctx 16384: 18.3 -> 18.1 us cold, 16.7 -> 16.0
  // hot); with dims-slice siblings the head-major order is kept.
  const std::size_t kv_head = DS == 1 ? unit % kKvHeads : unit / capacity;
  const std::size_t partition = DS == 1 ? unit / kKvHeads : unit % capacity;
  const std::size_t begin = partition * partition_tokens;
  if (begin >= ctx) return;
  const std::size_t end = ctx < begin + partition_tokens ? ctx : begin + partition_tokens;
  if constexpr (kFused) {
    // The q / k rows are loaded first; the prologue's arithmetic runs inside
    // the scan, once the first chunk's loads have gone out behind them.
    fused_qk_rot(f, position, fq);
    const FusedQKRows rows = fused_qk_load(f, kv_head);
    __builtin_amdgcn_sched_barrier(0);
    auto pro = [&] { fused_qk_finish(f, rows, fq); };
    decode_mfma_scan<DS, WAVES, CT, true, false, decltype(pro)>(a, kv_head, dq, begin, end, position, sh, &fq,
                                                                nullptr, pro);
  } else {
    decode_mfma_scan<DS, WAVES, CT, false>(a, kv_head, dq, begin, end, position, sh, &fq);
  }
  __syncthreads();
  // The workgroup whose range holds the position appends the new row.  When a
  // device position lies beyond the plan's capacity no workgroup holds it (the
  // merge then reports the capacity error); the last partition appends it so
  // the cache still receives the row, as the reference's separate append
  // kernel guarantees (cpp/kernels/qwen35_online_attention.cu:936-945).
  const bool owns_position = position >= begin && position < end;
  const bool past_capacity = partition + 1 == capacity && position >= begin + partition_tokens;
  if (dq == 0 && (owns_position || past_capacity)) {
    if constexpr (kFused)
      append_rows_fused(a, fq, kv_head, position);
    else
      append_rows(a, kv_head, position);
  }
  for (int o = threadIdx.x; o < kGroup * DIMS; o += WAVES * 64) {
    const int h = o / DIMS, d = o % DIMS;
    float mm, l, acc;
    decode_mfma_combine(sh, h, d, mm, l, acc);
    const std::size_t idx = (kv_head * kGroup + h) * max_partitions + partition;
    if (dq == 0 && d == 0) {
      pmax[idx] = mm * kLn2;
      psum[idx] = l;
    }
    pval[idx * kHeadDim + dq * DIMS + d] = acc;
  }
}

template <int DS, int WAVES, int CT = 32, bool kFused = false>
__global__ __launch_bounds__(WAVES * 64) void decode_split_mfma_kernel(
    DecodeMfmaArgs a, float *__restrict__ pmax, float *__restrict__ psum,
    float *__restrict__ pval, std::size_t host_position, const std::uint32_t *device_position,
    std::size_t capacity, std::size_t max_partitions, std::size_t partition_tokens,
    std::size_t threshold, FusedNormRope f) {
  __shared__ DecodeMfmaShared<DS, WAVES, CT> sh;
  __shared__ DecodeFusedQK fq;
  const std::size_t position = read_position(device_position, host_position);
  if (position >= a.max_ctx) return;
  if (position + 1 < threshold) return;
  split_body<DS, WAVES, CT, kFused>(blockIdx.x, a, pmax, psum, pval, position, capacity,
                                    max_partitions, partition_tokens, f, sh, fq);
}

// Device-position decode of a split-K plan in one launch instead of two: the
// position is read on the device, and below the split threshold the first
// blocks run the single-block scan (writing the gated output) while the rest
// exit; from the threshold on the grid runs the split-K partitions.  The
// merge kernel that follows exits below the threshold, as before.
template <int DS, int WAVES, bool kFused>
__global__ __launch_bounds__(WAVES * 64) void decode_dynamic_mfma_kernel(
    DecodeMfmaArgs a, const bf16_bits *__restrict__ gate, std::size_t gate_stride,
    bf16_bits *__restrict__ output, float *__restrict__ pmax, float *__restrict__ psum,
    float *__restrict__ pval, const std::uint32_t *device_position, std::size_t capacity,
    std::size_t max_partitions, std::size_t partition_tokens, std::size_t threshold,
    FusedNormRope f) {
  __shared__ DecodeMfmaShared<kSingleDs, WAVES, kSingleChunk> ssh;
  __shared__ DecodeMfmaShared<DS, WAVES, split_chunk(DS)> psh;
  __shared__ DecodeFusedQK fq;
  const std::size_t position = *device_position;
  if (position >= a.max_ctx) return;
  if (position + 1 < threshold)
    single_block_body<kSingleDs, WAVES, kFused, false, kSingleChunk>(blockIdx.x, a, gate, gate_stride, output,
                                                                      position, f, ssh, fq);
  else
    split_body<DS, WAVES, split_chunk(DS), kFused>(blockIdx.x, a, pmax, psum, pval, position, capacity,
                                      max_partitions, partition_tokens, f, psh, fq);
}

// ------------------------------------------------------------ launchers

// Plans of at most 16 partitions (ctx 4096 at P=256) use the 64-workgroup
// quarter-row merge, which is latency-bound there; longer plans use the
// 8-wave row merge, which reads whole partial rows and holds 128 partitions
// in one round trip (ctx 16384: 20.9 -> 19.8 us per call).
template <typename ActT>
void launch_merge(const ActT *g, std::size_t gate_stride, ActT *out, const float *pmax,
                  const float *psum, const float *pval, Qwen35AttentionShape shape,
                  Qwen35OnlineDecodePlan plan, std::size_t max_partitions,
                  const std::uint32_t *device_position, hipStream_t stream) {
  constexpr unsigned grid = kQueryHeads * (kHeadDim / kMergeDims);
  if (plan.active_partition_capacity <= static_cast<std::size_t>(kMergeChunkShort))
    decode_merge_kernel<ActT, kMergeChunkShort><<<grid, kMergeDims, 0, stream>>>(
        g, gate_stride, out, pmax, psum, pval, shape.max_context_tokens, shape.past_tokens, plan.partition_tokens,
        max_partitions, plan.active_partition_capacity, plan.split_k_threshold_tokens, device_position);
  else
    decode_merge_rows_kernel<ActT, kLongMergeWaves><<<kQueryHeads, kLongMergeWaves * 64, 0, stream>>>(
        g, gate_stride, out, pmax, psum, pval, shape.max_context_tokens, shape.past_tokens, plan.partition_tokens,
        max_partitions, plan.active_partition_capacity, plan.split_k_threshold_tokens, device_position);
}

// Device-position decode of a split-K plan: decode_dynamic_mfma_kernel (the
// single-block or the partition work, chosen on the device), then the merge.
template <bool kFused>
void launch_dynamic_decode(const DecodeMfmaArgs &args, const bf16_bits *g, std::size_t gate_stride,
                           bf16_bits *out, void *workspace, Qwen35AttentionShape shape,
                           Qwen35OnlineDecodePlan plan, Qwen35OnlineDecodeWorkspaceLayout ws,
                           const std::uint32_t *device_position, hipStream_t stream,
                           FusedNormRope f) {
  const std::size_t max_partitions = ceil_div(shape.max_context_tokens, plan.partition_tokens,
                                              "online decode maximum partition capacity overflow");
  const std::size_t units = checked_mul<Err>(kKvHeads, plan.active_partition_capacity,
                                             "online decode partition grid dimension overflow");
  (void)grid_dim(checked_mul<Err>(units + 8, kSplitDs, "online decode partition grid dimension overflow"),
                 "online decode partition grid dimension overflow");
  auto *bytes = static_cast<std::byte *>(workspace);
  auto *pmax = reinterpret_cast<float *>(bytes + ws.max_offset_bytes);
  auto *psum = reinterpret_cast<float *>(bytes + ws.sum_offset_bytes);
  auto *pval = reinterpret_cast<float *>(bytes + ws.value_offset_bytes);
  const unsigned single_grid = xcd_grid<kSingleDs>(kKvHeads);
  auto grid_for = [&](unsigned split_grid) { return split_grid > single_grid ? split_grid : single_grid; };
  if (units >= 192)
    decode_dynamic_mfma_kernel<1, kSplitWaves, kFused><<<grid_for(xcd_grid<1>(units)), kSplitWaves * 64, 0, stream>>>(
        args, g, gate_stride, out, pmax, psum, pval, device_position, plan.active_partition_capacity,
        max_partitions, plan.partition_tokens, plan.split_k_threshold_tokens, f);
  else if (units >= 96)
    decode_dynamic_mfma_kernel<2, kSplitWaves, kFused><<<grid_for(xcd_grid<2>(units)), kSplitWaves * 64, 0, stream>>>(
        args, g, gate_stride, out, pmax, psum, pval, device_position, plan.active_partition_capacity,
        max_partitions, plan.partition_tokens, plan.split_k_threshold_tokens, f);
  else
    decode_dynamic_mfma_kernel<kSplitDs, kSplitWaves, kFused>
        <<<grid_for(xcd_grid<kSplitDs>(units)), kSplitWaves * 64, 0, stream>>>(
            args, g, gate_stride, out, pmax, psum, pval, device_position, plan.active_partition_capacity,
            max_partitions, plan.partition_tokens, plan.split_k_threshold_tokens, f);
  check_launch<Err>(plan.partition_tokens == 256
                        ? "qwen35_online_attention_decode_split_k_256_partition"
                        : "qwen35_online_attention_decode_split_k_512_partition");
  launch_merge<bf16_bits>(g, gate_stride, out, pmax, psum, pval, shape, plan, max_partitions,
                          device_position, stream);
  check_launch<Err>("qwen35_online_attention_decode_split_k_merge");
}

// bf16 activations and cache: single-block and / or split-K MFMA kernels of
// the plan, then the merge.  kFused: q and k are normalised and rotated in
// the kernels (fused producers) and the gate is the q projection's second half.
template <bool kFused>
void launch_decode_mfma(const DecodeMfmaArgs &args, const bf16_bits *g, std::size_t gate_stride,
                        bf16_bits *out, void *workspace, Qwen35AttentionShape shape,
                        Qwen35OnlineDecodePlan plan, Qwen35OnlineDecodeWorkspaceLayout ws,
                        const std::uint32_t *device_position, hipStream_t stream,
                        bool partition_only, FusedNormRope f) {
  const std::size_t host_ctx = shape.past_tokens + 1;
  const bool dynamic = device_position != nullptr;
  const bool single = plan.resolved_mode == Qwen35DecodeAttentionMode::single_block;
  if (partition_only) require<Err>(!single, "partition-only decode needs a split-K plan");
  if (dynamic && !single && !partition_only) {
    // one launch selects single-block or split-K on the device, then the merge
    launch_dynamic_decode<kFused>(args, g, gate_stride, out, workspace, shape, plan, ws,
                                  device_position, stream, f);
    return;
  }
  if (!partition_only && (dynamic || single || host_ctx < plan.split_k_threshold_tokens)) {
    // Above 1.5 chunks per wave the LDS-staged scan streams the next chunk
    // under the current one (ctx 1024: 11.2 -> 10.3 us hot; with the
    // cold-cache prefetch, ctx 512 cold 8.23 -> 8.06 us, hot 6.93 -> 6.86);
    // at ctx 320 the register-fed scan is faster (6.65 against 6.75 us cold).
    // (The stage's LDS-direct loads of the new row need 16-byte aligned
    // key / value rows; other pointers take the register-fed scan.)
    const std::size_t ctx_bound = dynamic ? shape.max_context_tokens : host_ctx;
    const bool rows_aligned =
        ((reinterpret_cast<std::uintptr_t>(args.key_new) | reinterpret_cast<std::uintptr_t>(args.value_new)) &
         15u) == 0;
    if (2 * ctx_bound > 3 * kSingleMfmaWaves * 32 && rows_aligned)
      decode_single_mfma_kernel<kSingleDs, kSingleMfmaWaves, kFused, true>
          <<<xcd_grid<kSingleDs>(kKvHeads), kSingleMfmaWaves * 64, 0, stream>>>(
              args, g, gate_stride, out, shape.past_tokens, device_position,
              plan.split_k_threshold_tokens, f);
    else
      decode_single_mfma_kernel<kSingleDs, kSingleMfmaWaves, kFused, false>
          <<<xcd_grid<kSingleDs>(kKvHeads), kSingleMfmaWaves * 64, 0, stream>>>(
              args, g, gate_stride, out, shape.past_tokens, device_position,
              plan.split_k_threshold_tokens, f);
    check_launch<Err>("qwen35_online_attention_decode_gfx950_hd256");
  }
  if (single || (!dynamic && host_ctx < plan.split_k_threshold_tokens)) return;
  const std::size_t max_partitions = ceil_div(shape.max_context_tokens, plan.partition_tokens,
                                              "online decode maximum partition capacity overflow");
  const std::size_t units = checked_mul<Err>(kKvHeads, plan.active_partition_capacity,
                                             "online decode partition grid dimension overflow");
  (void)grid_dim(checked_mul<Err>(units + 8, kSplitDs, "online decode partition grid dimension overflow"),
                 "online decode partition grid dimension overflow");
  auto *bytes = static_cast<std::byte *>(workspace);
  auto *pmax = reinterpret_cast<float *>(bytes + ws.max_offset_bytes);
  auto *psum = reinterpret_cast<float *>(bytes + ws.sum_offset_bytes);
  auto *pval = reinterpret_cast<float *>(bytes + ws.value_offset_bytes);
  // Slice the dims only while the partitions alone leave the 256 CUs idle.
  if (units >= 192)
    decode_split_mfma_kernel<1, kSplitWaves, split_chunk(1), kFused>
        <<<xcd_grid<1>(units), kSplitWaves * 64, 0, stream>>>(
        args, pmax, psum, pval, shape.past_tokens, device_position, plan.active_partition_capacity,
        max_partitions, plan.partition_tokens, plan.split_k_threshold_tokens, f);
  else if (units >= 96)
    decode_split_mfma_kernel<2, kSplitWaves, split_chunk(2), kFused>
        <<<xcd_grid<2>(units), kSplitWaves * 64, 0, stream>>>(
        args, pmax, psum, pval, shape.past_tokens, device_position, plan.active_partition_capacity,
        max_partitions, plan.partition_tokens, plan.split_k_threshold_tokens, f);
  else
    decode_split_mfma_kernel<kSplitDs, kSplitWaves, split_chunk(kSplitDs), kFused>
        <<<xcd_grid<kSplitDs>(units), kSplitWaves * 64, 0, stream>>>(
            args, pmax, psum, pval, shape.past_tokens, device_position, plan.active_partition_capacity,
            max_partitions, plan.partition_tokens, plan.split_k_threshold_tokens, f);
  check_launch<Err>(plan.partition_tokens == 256
                        ? "qwen35_online_attention_decode_split_k_256_partition"
                        : "qwen35_online_attention_decode_split_k_512_partition");
  if (partition_only) return;
  launch_merge<bf16_bits>(g, gate_stride, out, pmax, psum, pval, shape, plan, max_partitions,
                          device_position, stream);
  check_launch<Err>("qwen35_online_attention_decode_split_k_merge");
}

constexpr int kSingleHeads = 1, kSingleWaves = 16, kSingleUnroll = 2;
constexpr int kPartHeads = 4, kPartWaves = 8, kPartUnroll = 2;

template <typename ActT, typename CacheT>
void launch_decode(const void *query, const void *key, const void *value, const void *gate,
                   void *output, void *kv_cache, void *workspace, Qwen35AttentionShape shape,
                   Qwen35KvCacheLayout layout, Qwen35OnlineDecodePlan plan,
                   Qwen35OnlineDecodeWorkspaceLayout ws, const std::uint32_t *device_position,
                   hipStream_t stream, bool partition_only) {
  const bool head_major = layout == Qwen35KvCacheLayout::head_major;
  const auto *q = static_cast<const ActT *>(query);
  const auto *g = static_cast<const ActT *>(gate);
  auto *out = static_cast<ActT *>(output);
  auto *cache = static_cast<CacheT *>(kv_cache);
  if constexpr (std::is_same_v<ActT, bf16_bits> && std::is_same_v<CacheT, bf16_bits>) {
    const DecodeMfmaArgs args{q, static_cast<const bf16_bits *>(key),
                              static_cast<const bf16_bits *>(value), cache, cache,
                              shape.max_context_tokens, head_major};
    launch_decode_mfma<false>(args, g, kHeadDim, out, workspace, shape, plan, ws, device_position,
                              stream, partition_only, FusedNormRope{});
    return;
  }
  if (partition_only) {
    require<Err>(plan.partition_tokens != 0, "partition-only decode needs a split-K plan");
  } else {
  append_decode_kernel<ActT, CacheT><<<4, 256, 0, stream>>>(
      static_cast<const ActT *>(key), static_cast<const ActT *>(value), cache,
      shape.max_context_tokens, shape.past_tokens, head_major, device_position);
  check_launch<Err>("qwen35_online_attention_decode_append_cache");
  }

  // With a host position the path is known here, so kernels that would only
  // early-exit are not enqueued.  With a device position every kernel of the
  // plan is enqueued and selects itself on-device (graph-capture safe).
  const std::size_t host_ctx = shape.past_tokens + 1;
  const bool dynamic = device_position != nullptr;
  const bool single = plan.resolved_mode == Qwen35DecodeAttentionMode::single_block;
  if (!partition_only && (dynamic || single || host_ctx < plan.split_k_threshold_tokens)) {
    decode_single_block_kernel<ActT, CacheT, kSingleHeads, kSingleWaves, kSingleUnroll>
        <<<kQueryHeads / kSingleHeads, kSingleWaves * 64, 0, stream>>>(
            q, g, out, cache, shape.max_context_tokens, shape.past_tokens, head_major,
            device_position, plan.split_k_threshold_tokens);
    check_launch<Err>("qwen35_online_attention_decode_gfx950_hd256");
  }
  if (single) return;
  if (!dynamic && host_ctx < plan.split_k_threshold_tokens) return;

  const std::size_t max_partitions = ceil_div(shape.max_context_tokens, plan.partition_tokens,
                                              "online decode maximum partition capacity overflow");
  const std::size_t units = kQueryHeads / kPartHeads;
  const int grid = grid_dim(checked_mul<Err>(units, plan.active_partition_capacity,
                                             "online decode partition grid dimension overflow"),
                            "online decode partition grid dimension overflow");
  auto *bytes = static_cast<std::byte *>(workspace);
  auto *pmax = reinterpret_cast<float *>(bytes + ws.max_offset_bytes);
  auto *psum = reinterpret_cast<float *>(bytes + ws.sum_offset_bytes);
  auto *pval = reinterpret_cast<float *>(bytes + ws.value_offset_bytes);
  decode_partition_kernel<ActT, CacheT, kPartHeads, kPartWaves, kPartUnroll>
      <<<grid, kPartWaves * 64, 0, stream>>>(
          q, cache, pmax, psum, pval, shape.max_context_tokens, shape.past_tokens, head_major,
          plan.active_partition_capacity, max_partitions, plan.partition_tokens,
          plan.split_k_threshold_tokens, device_position);
  check_launch<Err>(plan.partition_tokens == 256
                        ? "qwen35_online_attention_decode_split_k_256_partition"
                        : "qwen35_online_attention_decode_split_k_512_partition");
  launch_merge<ActT>(g, kHeadDim, out, pmax, psum, pval, shape, plan, max_partitions, device_position,
                     stream);
  check_launch<Err>("qwen35_online_attention_decode_split_k_merge");
}

void require_aligned16(const void *p, const char *message) {
  require<Err>((reinterpret_cast<std::uintptr_t>(p) & 15u) == 0, message);
}

} // namespace

// ------------------------------------------------------------- plan API

Qwen35OnlineDecodePlan qwen35_online_decode_plan(Qwen35AttentionShape shape,
                                                 Qwen35DecodeAttentionMode requested,
                                                 std::size_t context_tokens) {
  require<Err>(shape.max_context_tokens != 0, "online decode plan maximum context tokens is zero");
  require<Err>(context_tokens != 0, "online decode plan context tokens is zero");
  require<Err>(context_tokens <= shape.max_context_tokens,
               "online decode plan context tokens exceed maximum context");
  const Qwen35DecodeAttentionMode resolved =
      requested == Qwen35DecodeAttentionMode::auto_select ? kDefaultOnlineDecodeMode : requested;
  const std::size_t partition = partition_tokens_for_mode(resolved);
  if (partition != 0)
    require<Err>(model_signature(shape), "split-K online decode requires the Qwen3.5 model signature");
  const std::size_t bucket = context_bucket_tokens(shape, context_tokens);
  if (partition == 0) return {resolved, 0, 0, bucket, 1};
  return {resolved, partition, partition, bucket,
          ceil_div(bucket, partition, "online decode active partition capacity overflow")};
}

Qwen35OnlineDecodeWorkspaceLayout
qwen35_online_decode_workspace_layout(Qwen35AttentionShape shape,
                                      Qwen35DecodeAttentionMode resolved_mode) {
  require<Err>(resolved_mode != Qwen35DecodeAttentionMode::auto_select,
               "online decode workspace mode must be resolved");
  const std::size_t partition = partition_tokens_for_mode(resolved_mode);
  if (partition == 0) return {};
  require<Err>(model_signature(shape), "split-K online decode requires the Qwen3.5 model signature");
  const std::size_t max_partitions = ceil_div(shape.max_context_tokens, partition,
                                              "online decode maximum partition capacity overflow");
  const std::size_t pc = checked_mul<Err>(shape.query_heads, max_partitions,
                                          "online decode partial count overflow");
  const std::size_t partial_bytes =
      checked_mul<Err>(pc, sizeof(float), "online decode partial bytes overflow");
  const std::size_t value_offset =
      checked_mul<Err>(2, partial_bytes, "online decode value offset overflow");
  const std::size_t value_bytes = checked_mul<Err>(
      checked_mul<Err>(pc, shape.head_dim, "online decode partial value count overflow"),
      sizeof(float), "online decode partial value bytes overflow");
  return {pc, 0, partial_bytes, value_offset,
          checked_add<Err>(value_offset, value_bytes, "online decode workspace bytes overflow")};
}

std::size_t qwen35_online_attention_workspace_bytes(Qwen35AttentionShape) noexcept { return 0; }

// ------------------------------------------------------------ decode API
namespace {
// Validation order and messages: cpp/kernels/qwen35_online_attention.cu:1220-1314.
void decode_impl(const void *query, const void *key, const void *value, const void *gate,
                 void *output, void *kv_cache, std::size_t kv_cache_bytes, void *workspace,
                 std::size_t workspace_bytes, Qwen35AttentionShape shape, RaftInferDataType act,
                 Qwen35KvCacheDType cache_dtype, Qwen35KvCacheLayout layout,
                 Qwen35OnlineDecodePlan plan, const std::uint32_t *device_position,
                 hipStream_t stream, bool partition_only, const FusedNormRope *fused = nullptr) {
  require<Err>(query != nullptr, "online decode query pointer is null");
  require<Err>(key != nullptr, "online decode key pointer is null");
  require<Err>(value != nullptr, "online decode value pointer is null");
  require<Err>(gate != nullptr, "online decode gate pointer is null");
  require<Err>(output != nullptr, "online decode output pointer is null");
  require<Err>(kv_cache != nullptr, "online decode KV cache pointer is null");
  require<Err>(stream != nullptr, "online decode HIP stream is null");
  require<Err>(online_decode_signature_supported(shape, act, cache_dtype, layout),
               "unsupported online attention decode signature; select the "
               "materialized implementation before allocation");
  require<Err>(plan.resolved_mode != Qwen35DecodeAttentionMode::auto_select,
               "online decode plan mode must be resolved");
  const std::size_t expected_partition = partition_tokens_for_mode(plan.resolved_mode);
  require<Err>(plan.partition_tokens == expected_partition,
               "online decode plan partition size is inconsistent");
  if (expected_partition == 0) {
    require<Err>(plan.split_k_threshold_tokens == 0 && plan.active_partition_capacity == 1,
                 "single-block online decode plan is inconsistent");
    require<Err>(workspace_bytes == 0, "single-block online decode does not use split-K workspace");
  } else {
    require<Err>(plan.split_k_threshold_tokens == expected_partition,
                 "split-K online decode threshold is inconsistent");
    require<Err>(plan.context_bucket_tokens != 0 &&
                     plan.context_bucket_tokens <= shape.max_context_tokens,
                 "split-K online decode context bucket is invalid");
    require<Err>(plan.active_partition_capacity ==
                     ceil_div(plan.context_bucket_tokens, expected_partition,
                              "online decode active partition capacity overflow"),
                 "split-K online decode partition capacity is inconsistent");
    require<Err>(device_position != nullptr || shape.past_tokens + 1 <= plan.context_bucket_tokens,
                 "split-K online decode context exceeds the planned bucket");
  }
  const auto ws = qwen35_online_decode_workspace_layout(shape, plan.resolved_mode);
  if (ws.bytes != 0) {
    require<Err>(workspace != nullptr, "split-K online decode workspace is null");
    require<Err>(workspace_bytes >= ws.bytes, "split-K online decode workspace is too small");
    require_aligned16(workspace, "split-K online decode workspace must be 16-byte aligned");
  }
  const std::size_t eb = cache_element_bytes_of(cache_dtype);
  require<Err>(eb != 0, "unsupported online attention KV cache dtype");
  require<Err>(layout_known(layout), "unsupported online attention KV cache layout");
  const std::size_t required = checked_mul<Err>(
      checked_mul<Err>(2,
                       checked_mul<Err>(shape.max_context_tokens,
                                        checked_mul<Err>(shape.kv_heads, shape.head_dim,
                                                         "online decode cache shape overflow"),
                                        "online decode cache shape overflow"),
                       "online decode cache shape overflow"),
      eb, "online decode cache byte size overflow");
  require<Err>(kv_cache_bytes >= required, "online decode KV cache is too small");
  // gfx950 kernels use 16-byte vector loads (an addition to the reference's
  // checks; device allocations are 256-byte aligned).
  require_aligned16(query, "online decode query must be 16-byte aligned");
  require_aligned16(kv_cache, "online decode KV cache must be 16-byte aligned");

  if (fused != nullptr) {
    // query = the q projection rows [16][2][256]; the gate is their second half
    require<Err>(act == RAFTINFER_DTYPE_BF16 && cache_dtype == Qwen35KvCacheDType::bf16,
                 "fused decode requires bf16 activations and a bf16 KV cache");
    const DecodeMfmaArgs args{nullptr, nullptr, static_cast<const bf16_bits *>(value),
                              static_cast<bf16_bits *>(kv_cache), static_cast<bf16_bits *>(kv_cache),
                              shape.max_context_tokens, layout == Qwen35KvCacheLayout::head_major};
    launch_decode_mfma<true>(args, static_cast<const bf16_bits *>(query) + kHeadDim, 2 * kHeadDim,
                             static_cast<bf16_bits *>(output), workspace, shape, plan, ws,
                             device_position, stream, false, *fused);
    return;
  }
  const bool f32_act = act == RAFTINFER_DTYPE_F32;
  const bool f32_cache = cache_dtype == Qwen35KvCacheDType::f32;
  if (f32_act && f32_cache)
    launch_decode<float, float>(query, key, value, gate, output, kv_cache, workspace, shape,
                                layout, plan, ws, device_position, stream, partition_only);
  else if (f32_act)
    launch_decode<float, bf16_bits>(query, key, value, gate, output, kv_cache, workspace, shape,
                                    layout, plan, ws, device_position, stream, partition_only);
  else if (f32_cache)
    launch_decode<bf16_bits, float>(query, key, value, gate, output, kv_cache, workspace, shape,
                                    layout, plan, ws, device_position, stream, partition_only);
  else
    launch_decode<bf16_bits, bf16_bits>(query, key, value, gate, output, kv_cache, workspace,
                                        shape, layout, plan, ws, device_position, stream, partition_only);
}

} // namespace

void qwen35_online_attention_decode(const void *query, const void *key, const void *value,
                                    const void *gate, void *output, void *kv_cache,
                                    std::size_t kv_cache_bytes, void *workspace,
                                    std::size_t workspace_bytes, Qwen35AttentionShape shape,
                                    RaftInferDataType act, Qwen35KvCacheDType cache_dtype,
                                    Qwen35KvCacheLayout layout, Qwen35OnlineDecodePlan plan,
                                    const std::uint32_t *device_position, hipStream_t stream) {
  decode_impl(query, key, value, gate, output, kv_cache, kv_cache_bytes, workspace,
              workspace_bytes, shape, act, cache_dtype, layout, plan, device_position, stream,
              false);
}

void qwen35_online_attention_decode_partition_only(
    const void *query, const void *key, const void *value, const void *gate, void *output,
    void *kv_cache, std::size_t kv_cache_bytes, void *workspace, std::size_t workspace_bytes,
    Qwen35AttentionShape shape, RaftInferDataType act, Qwen35KvCacheDType cache_dtype,
    Qwen35KvCacheLayout layout, Qwen35OnlineDecodePlan plan, const std::uint32_t *device_position,
    hipStream_t stream) {
  decode_impl(query, key, value, gate, output, kv_cache, kv_cache_bytes, workspace,
              workspace_bytes, shape, act, cache_dtype, layout, plan, device_position, stream,
              true);
}

void qwen35_online_attention_decode(const void *query, const void *key, const void *value,
                                    const void *gate, void *output, void *kv_cache,
                                    std::size_t kv_cache_bytes, Qwen35AttentionShape shape,
                                    RaftInferDataType act, Qwen35KvCacheDType cache_dtype,
                                    Qwen35KvCacheLayout layout,
                                    const std::uint32_t *device_position, hipStream_t stream) {
  const auto plan = qwen35_online_decode_plan(shape, Qwen35DecodeAttentionMode::single_block,
                                              shape.past_tokens + 1);
  qwen35_online_attention_decode(query, key, value, gate, output, kv_cache, kv_cache_bytes,
                                 nullptr, 0, shape, act, cache_dtype, layout, plan,
                                 device_position, stream);
}

// ------------------------------------------- allocation-free decode
// The split-K partials of the static-workspace entry point live in this
// file-scope array: 16 query heads x 512 partitions x (max + sum + 256
// values) fp32, i.e. a 131,072-token maximum context at P=256 (262,144 at
// P=512).  Each GPU holds its own copy for the life of the process.  Host
// code never uses the array's name as an address: the per-device address
// comes from hipGetSymbolAddress.
constexpr std::size_t kStaticWorkspaceBytes =
    std::size_t{16} * 512 * (2 + 256) * sizeof(float); // 8,454,144
static __device__ __align__(256) unsigned char scratch[kStaticWorkspaceBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`, looked up once per device with
// that device current.
void *scratch_for_current_device(hipStream_t stream) {
  int device = -1;
  require<Err>(hipGetDevice(&device) == hipSuccess, "static decode workspace: hipGetDevice failed");
  require<Err>(device >= 0 && device < kMaxDevices, "static decode workspace: device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[device] == nullptr) {
    // The lookup is not a stream operation, but it may load the code object;
    // it is done outside any capture so that a captured call never depends on it.
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    require<Err>(hipStreamIsCapturing(stream, &capture) == hipSuccess &&
                     capture == hipStreamCaptureStatusNone,
                 "static decode workspace: the first call on a device must not be captured "
                 "(call it once eagerly on this device before capturing it)");
    void *ptr = nullptr;
    const hipError_t rc = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    require<Err>(rc == hipSuccess && ptr != nullptr,
                 "static decode workspace: hipGetSymbolAddress failed");
    g_scratch_ptr[device] = ptr;
  }
  return g_scratch_ptr[device];
}
} // namespace

std::size_t qwen35_online_attention_static_workspace_bytes() noexcept {
  return kStaticWorkspaceBytes;
}

void qwen35_online_attention_decode_static_workspace(
    const void *query, const void *key, const void *value, const void *gate, void *output,
    void *kv_cache, std::size_t kv_cache_bytes, Qwen35AttentionShape shape,
    RaftInferDataType activation_dtype, Qwen35KvCacheDType cache_dtype,
    Qwen35KvCacheLayout cache_layout, Qwen35OnlineDecodePlan plan,
    const std::uint32_t *device_position, hipStream_t stream) {
  require<Err>(plan.resolved_mode != Qwen35DecodeAttentionMode::auto_select,
               "online decode plan mode must be resolved");
  std::size_t bytes = 0;
  if (partition_tokens_for_mode(plan.resolved_mode) != 0) {
    require<Err>(model_signature(shape),
                 "split-K online decode requires the Qwen3.5 model signature");
    bytes = qwen35_online_decode_workspace_layout(shape, plan.resolved_mode).bytes;
    require<Err>(bytes <= kStaticWorkspaceBytes,
                 "static decode workspace is too small for this maximum context (at most "
                 "131072 tokens at split_k_256, 262144 at split_k_512); pass a workspace to "
                 "qwen35_online_attention_decode instead");
  }
  void *workspace = bytes != 0 ? scratch_for_current_device(stream) : nullptr;
  decode_impl(query, key, value, gate, output, kv_cache, kv_cache_bytes, workspace, bytes, shape,
              activation_dtype, cache_dtype, cache_layout, plan, device_position, stream, false);
}

void qwen35_online_attention_decode_fused(const void *query_gate, const void *key,
                                          const void *value, void *output, void *kv_cache,
                                          std::size_t kv_cache_bytes, void *workspace,
                                          std::size_t workspace_bytes, Qwen35AttentionShape shape,
                                          Qwen35FusedNormRope norm, Qwen35KvCacheDType cache_dtype,
                                          Qwen35KvCacheLayout layout, Qwen35OnlineDecodePlan plan,
                                          const std::uint32_t *device_position, hipStream_t stream) {
  // The producer's checks (cpp/kernels/qwen35_primitives.cu:580-601) for the
  // parameters it adds, then the decode's own validation.
  require<Err>(norm.query_norm_weight != nullptr && norm.key_norm_weight != nullptr,
               "fused decode norm weight pointer is null");
  require<Err>(norm.weight_dtype == RAFTINFER_DTYPE_BF16 || norm.weight_dtype == RAFTINFER_DTYPE_F32,
               "fused decode norm weights must be bf16 or f32");
  require<Err>(norm.rotary_dim > 0 && norm.rotary_dim <= kHeadDim && norm.rotary_dim % 8 == 0,
               "fused decode rotary_dim must be a positive multiple of 8 up to 256");
  require<Err>(std::isfinite(norm.rope_base) && norm.rope_base > 0.0f,
               "qk_norm_rope rope_base must be finite and positive");
  require<Err>(std::isfinite(norm.epsilon) && norm.epsilon >= 0.0f,
               "qk_norm_rope epsilon must be finite and non-negative");
  const std::size_t wa = norm.weight_dtype == RAFTINFER_DTYPE_F32 ? 16 : 8;
  require<Err>(((reinterpret_cast<std::uintptr_t>(norm.query_norm_weight) |
                 reinterpret_cast<std::uintptr_t>(norm.key_norm_weight)) & (wa - 1)) == 0,
               "fused decode norm weights are not vector-aligned");
  require<Err>(((reinterpret_cast<std::uintptr_t>(key) | reinterpret_cast<std::uintptr_t>(value)) & 15u) == 0,
               "fused decode key and value must be 16-byte aligned");
  const FusedNormRope f{static_cast<const bf16_bits *>(query_gate), static_cast<const bf16_bits *>(key),
                        norm.query_norm_weight, norm.key_norm_weight,
                        norm.weight_dtype == RAFTINFER_DTYPE_F32, static_cast<int>(norm.rotary_dim / 2),
                        std::pow(static_cast<double>(norm.rope_base), -2.0 / static_cast<double>(norm.rotary_dim)),
                        norm.epsilon};
  const void *gate = query_gate == nullptr ? nullptr : static_cast<const bf16_bits *>(query_gate) + kHeadDim;
  decode_impl(query_gate, key, value, gate, output, kv_cache, kv_cache_bytes, workspace,
              workspace_bytes, shape, RAFTINFER_DTYPE_BF16, cache_dtype, layout, plan, device_position,
              stream, false, &f);
}

std::uint32_t qwen35_online_attention_consume_capacity_errors() {
  unsigned int value = 0;
  const unsigned int zero = 0;
  require<Err>(hipDeviceSynchronize() == hipSuccess, "device synchronize failed");
  require<Err>(hipMemcpyFromSymbol(&value, HIP_SYMBOL(g_capacity_errors), sizeof value) == hipSuccess,
               "reading the capacity error counter failed");
  require<Err>(hipMemcpyToSymbol(HIP_SYMBOL(g_capacity_errors), &zero, sizeof zero) == hipSuccess,
               "clearing the capacity error counter failed");
  return value;
}

// ------------------------------------------------------ batched decode
namespace {

constexpr std::size_t kBatchedPartition = 256;

// Workgroup (sequence, head group, partition).  Sequences whose context is at
// most single_max run single-block in partition 0 and write the gated output;
// longer ones write partials for the merge.
template <typename ActT, int NH, int WAVES, int U>
__global__ __launch_bounds__(WAVES * 64) void batched_partition_kernel(
    const ActT *__restrict__ query, const ActT *__restrict__ key, const ActT *__restrict__ value,
    const ActT *__restrict__ gate, ActT *__restrict__ output, const std::byte *cache_base,
    std::size_t cache_stride, std::size_t max_ctx, const std::uint32_t *__restrict__ lengths,
    std::size_t max_partitions, std::size_t single_max, float *__restrict__ pmax,
    float *__restrict__ psum, float *__restrict__ pval) {
  __shared__ ScanShared<NH, WAVES> sh;
  constexpr std::size_t units = kQueryHeads / NH;
  const std::size_t seq = blockIdx.y;
  const std::size_t unit = blockIdx.x / max_partitions;
  const std::size_t partition = blockIdx.x % max_partitions;
  const std::size_t ctx = lengths[seq];
  if (ctx == 0 || ctx > max_ctx) return;
  const bool single = ctx <= single_max;
  const std::size_t begin = partition * kBatchedPartition;
  if (single ? partition != 0 : begin >= ctx) return;
  const std::size_t end = single ? ctx : (ctx < begin + kBatchedPartition ? ctx : begin + kBatchedPartition);
  const auto *cache = reinterpret_cast<const bf16_bits *>(cache_base + seq * cache_stride);
  const std::size_t first_head = unit * NH;
  const std::size_t kv_head = first_head / kGroup;
  const bf16_bits *k_plane = cache;
  const bf16_bits *v_plane = cache + max_ctx * kKvHeads * kHeadDim;
  const ActT *q = query + seq * kQueryHeads * kHeadDim;
  scan_range<ActT, bf16_bits, NH, WAVES, U>(q, first_head, k_plane, v_plane, true, max_ctx,
                                            kv_head, begin, end, sh);
  __syncthreads();
  for (int o = threadIdx.x; o < NH * kHeadDim; o += WAVES * 64) {
    const int h = o / kHeadDim, d = o % kHeadDim;
    float mm, l, a;
    combine_waves(sh, h, d, mm, l, a);
    const std::size_t head = first_head + h;
    if (single) {
      const std::size_t out_idx = (seq * kQueryHeads + head) * kHeadDim + d;
      Elem<ActT>::store(output, out_idx, (a / l) * sigmoid_gate(Elem<ActT>::load(gate, out_idx)));
    } else {
      const std::size_t idx = (seq * kQueryHeads + head) * max_partitions + partition;
      if (d == 0) {
        pmax[idx] = mm * kLn2;
        psum[idx] = l;
      }
      pval[idx * kHeadDim + d] = a;
    }
  }
  (void)units;
  (void)key;
  (void)value;
}

template <typename ActT>
__global__ __launch_bounds__(256) void batched_append_kernel(const ActT *__restrict__ key,
                                                             const ActT *__restrict__ value,
                                                             std::byte *cache_base,
                                                             std::size_t cache_stride,
                                                             std::size_t max_ctx,
                                                             const std::uint32_t *lengths) {
  const std::size_t seq = blockIdx.y;
  const std::size_t ctx = lengths[seq];
  if (ctx == 0 || ctx > max_ctx) return;
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  auto *cache = reinterpret_cast<bf16_bits *>(cache_base + seq * cache_stride);
  const std::size_t idx = cache_row(true, ctx - 1, e >> 8, max_ctx) + (e & 255);
  const std::size_t plane = max_ctx * kKvHeads * kHeadDim;
  const std::size_t src = seq * kKvHeads * kHeadDim + e;
  cache[idx] = f32_to_bf16(Elem<ActT>::load(key, src));
  cache[plane + idx] = f32_to_bf16(Elem<ActT>::load(value, src));
}

// Workgroup = (sequence, head), kBatchedMergeWaves waves, so a 32768-token
// context (128 partitions) takes one round trip.
template <typename ActT>
__global__ __launch_bounds__(kBatchedMergeWaves * 64) void batched_merge_kernel(
    const ActT *__restrict__ gate, ActT *__restrict__ output, const float *__restrict__ pmax,
    const float *__restrict__ psum, const float *__restrict__ pval,
    const std::uint32_t *__restrict__ lengths, std::size_t max_ctx, std::size_t max_partitions,
    std::size_t single_max) {
  __shared__ RowMergeShared<kBatchedMergeWaves> sh;
  const std::size_t seq = blockIdx.y;
  const std::size_t head = blockIdx.x;
  const std::size_t ctx = lengths[seq];
  const int d = threadIdx.x & (kHeadDim - 1);
  const bool finisher = threadIdx.x < kHeadDim;
  const std::size_t out_idx = (seq * kQueryHeads + head) * kHeadDim + d;
  // A length of 0 or above max_ctx (a negative int32 reads as a huge uint32)
  // has no valid context: every other kernel skips the sequence, and here its
  // output rows become NaN and the guard counter counts it once.
  if (ctx == 0 || ctx > max_ctx) {
    if (head == 0 && threadIdx.x == 0) atomicAdd(&g_capacity_errors, 1u);
    if (finisher) Elem<ActT>::store(output, out_idx, __builtin_nanf(""));
    return;
  }
  if (ctx <= single_max) return;
  const std::size_t active = ctx / kBatchedPartition + (ctx % kBatchedPartition ? 1 : 0);
  const float gv = finisher ? Elem<ActT>::load(gate, out_idx) : 0.f;
  merge_rows<kBatchedMergeWaves>(pmax, psum, pval, (seq * kQueryHeads + head) * max_partitions,
                                 active, sh);
  __syncthreads();
  if (finisher)
    Elem<ActT>::store(output, out_idx, combine_rows<kBatchedMergeWaves>(sh, d) * sigmoid_gate(gv));
}

// bf16 batched path: MFMA scores, dims-sliced workgroups, fused append.
template <int DS, int WAVES, int CT>
__global__ __launch_bounds__(WAVES * 64) void batched_mfma_kernel(
    const bf16_bits *__restrict__ query, const bf16_bits *__restrict__ key,
    const bf16_bits *__restrict__ value, const bf16_bits *__restrict__ gate,
    bf16_bits *__restrict__ output, std::byte *cache_base, std::size_t cache_stride,
    std::size_t max_ctx, const std::uint32_t *__restrict__ lengths, std::size_t max_partitions,
    std::size_t single_max, float *__restrict__ pmax, float *__restrict__ psum,
    float *__restrict__ pval) {
  __shared__ DecodeMfmaShared<DS, WAVES, CT> sh;
  constexpr int DIMS = kHeadDim / DS;
  const std::size_t seq = blockIdx.y;
  const std::size_t ctx = lengths[seq];
  if (ctx == 0 || ctx > max_ctx) return;
  std::size_t unit;
  int dq;
  xcd_unit<DS>(blockIdx.x, unit, dq);
  const bool single = ctx <= single_max;
  std::size_t kv_head, partition = 0, begin = 0, end = ctx;
  if (single) {
    if (unit >= kKvHeads) return;
    kv_head = unit;
  } else {
    if (unit >= kKvHeads * max_partitions) return;
    kv_head = unit / max_partitions;
    partition = unit % max_partitions;
    begin = partition * kBatchedPartition;
    if (begin >= ctx) return;
    end = ctx < begin + kBatchedPartition ? ctx : begin + kBatchedPartition;
  }
  auto *cache = reinterpret_cast<bf16_bits *>(cache_base + seq * cache_stride);
  const DecodeMfmaArgs a{query + seq * kQueryHeads * kHeadDim, key + seq * kKvHeads * kHeadDim,
                         value + seq * kKvHeads * kHeadDim, cache, cache, max_ctx, true};
  const std::size_t pos = ctx - 1;
  // Single-block sequences: the gate values of this thread's outputs are
  // loaded before the scan (no load round trip in the epilogue).
  constexpr int kOut = (kGroup * DIMS + WAVES * 64 - 1) / (WAVES * 64);
  float gv[kOut];
#pragma unroll
  for (int n = 0; n < kOut; ++n) {
    const int o = threadIdx.x + n * WAVES * 64;
    gv[n] = 0.f;
    if (single && o < kGroup * DIMS)
      gv[n] = bf16_to_f32(gate[(seq * kQueryHeads + kv_head * kGroup + o / DIMS) * kHeadDim + dq * DIMS +
                               o % DIMS]);
  }
  decode_mfma_scan<DS, WAVES, CT>(a, kv_head, dq, begin, end, pos, sh);
  __syncthreads();
  if (dq == 0 && pos >= begin && pos < end) append_rows(a, kv_head, pos);
#pragma unroll
  for (int n = 0; n < kOut; ++n) {
    const int o = threadIdx.x + n * WAVES * 64;
    if (o >= kGroup * DIMS) break;
    const int h = o / DIMS, d = o % DIMS;
    float mm, l, acc;
    decode_mfma_combine(sh, h, d, mm, l, acc);
    const std::size_t head = seq * kQueryHeads + kv_head * kGroup + h;
    if (single) {
      const std::size_t idx = head * kHeadDim + dq * DIMS + d;
      output[idx] = f32_to_bf16((acc / l) * sigmoid_gate(gv[n]));
    } else {
      const std::size_t idx = head * max_partitions + partition;
      if (dq == 0 && d == 0) {
        pmax[idx] = mm * kLn2;
        psum[idx] = l;
      }
      pval[idx * kHeadDim + dq * DIMS + d] = acc;
    }
  }
}

template <typename ActT>
void launch_batched(const void *query, const void *key, const void *value, const void *gate,
                    void *output, void *kv_cache, const std::uint32_t *lengths, void *workspace,
                    Qwen35BatchedDecodeShape shape, hipStream_t stream) {
  const std::size_t max_partitions = ceil_div_unchecked(shape.max_context_tokens, kBatchedPartition);
  const std::size_t partials = shape.sequences * kQueryHeads * max_partitions;
  auto *pmax = static_cast<float *>(workspace);
  auto *psum = pmax + partials;
  auto *pval = psum + partials;
  auto *base = static_cast<std::byte *>(kv_cache);
  const auto *q = static_cast<const ActT *>(query);
  const auto *k = static_cast<const ActT *>(key);
  const auto *v = static_cast<const ActT *>(value);
  const auto *g = static_cast<const ActT *>(gate);
  auto *out = static_cast<ActT *>(output);
  const unsigned int seqs = static_cast<unsigned int>(shape.sequences);
  if constexpr (std::is_same_v<ActT, bf16_bits>) {
    // 4-wave workgroups with 16-token chunks: 148 VGPRs, so three fit a CU
    // (three waves per SIMD) and one workgroup's loads overlap the others'
    // reductions and stores (32-token chunks: 218 VGPRs, two per CU, 3%
    // slower on the x32 batch).
    constexpr int DS = 1, WAVES = 4, CT = 16;
    batched_mfma_kernel<DS, WAVES, CT>
        <<<dim3(xcd_grid<DS>(kKvHeads * max_partitions), seqs), WAVES * 64, 0, stream>>>(
            q, k, v, g, out, base, shape.cache_stride_bytes, shape.max_context_tokens, lengths,
            max_partitions, shape.single_block_max_tokens, pmax, psum, pval);
    check_launch<Err>("qwen35_batched_decode_partition");
    batched_merge_kernel<ActT><<<dim3(kQueryHeads, seqs), kBatchedMergeWaves * 64, 0, stream>>>(
        g, out, pmax, psum, pval, lengths, shape.max_context_tokens, max_partitions,
        shape.single_block_max_tokens);
    check_launch<Err>("qwen35_batched_decode_merge");
    return;
  }
  batched_append_kernel<ActT><<<dim3(4, seqs), 256, 0, stream>>>(
      k, v, base, shape.cache_stride_bytes, shape.max_context_tokens, lengths);
  check_launch<Err>("qwen35_batched_decode_append_cache");
  constexpr int NH = 4, WAVES = 8, U = 2;
  const unsigned int gx = static_cast<unsigned int>((kQueryHeads / NH) * max_partitions);
  batched_partition_kernel<ActT, NH, WAVES, U><<<dim3(gx, seqs), WAVES * 64, 0, stream>>>(
      q, k, v, g, out, base, shape.cache_stride_bytes, shape.max_context_tokens, lengths,
      max_partitions, shape.single_block_max_tokens, pmax, psum, pval);
  check_launch<Err>("qwen35_batched_decode_partition");
  batched_merge_kernel<ActT><<<dim3(kQueryHeads, seqs), kBatchedMergeWaves * 64, 0, stream>>>(
      g, out, pmax, psum, pval, lengths, shape.max_context_tokens, max_partitions,
      shape.single_block_max_tokens);
  check_launch<Err>("qwen35_batched_decode_merge");
}

} // namespace

std::size_t qwen35_batched_decode_workspace_bytes(Qwen35BatchedDecodeShape shape) {
  require<Err>(shape.sequences != 0, "batched decode needs at least one sequence");
  require<Err>(shape.max_context_tokens != 0, "batched decode maximum context is zero");
  const std::size_t max_partitions = ceil_div_unchecked(shape.max_context_tokens, kBatchedPartition);
  const std::size_t partials = checked_mul<Err>(
      checked_mul<Err>(shape.sequences, kQueryHeads, "batched decode workspace overflow"),
      max_partitions, "batched decode workspace overflow");
  return checked_mul<Err>(checked_mul<Err>(partials, 2 + kHeadDim, "batched decode workspace overflow"),
                          sizeof(float), "batched decode workspace overflow");
}

void qwen35_online_attention_decode_batched(const void *query, const void *key,
                                            const void *value, const void *gate, void *output,
                                            void *kv_cache, std::size_t kv_cache_bytes,
                                            const std::uint32_t *context_lengths,
                                            void *workspace, std::size_t workspace_bytes,
                                            Qwen35BatchedDecodeShape shape, RaftInferDataType act,
                                            hipStream_t stream) {
  require<Err>(query && key && value && gate && output && kv_cache && context_lengths && workspace,
               "batched decode pointer is null");
  require<Err>(stream != nullptr, "batched decode HIP stream is null");
  require<Err>(act == RAFTINFER_DTYPE_F32 || act == RAFTINFER_DTYPE_BF16,
               "batched decode activation dtype must be f32 or bf16");
  require<Err>(shape.sequences <= 65535, "batched decode supports at most 65535 sequences");
  const std::size_t need_ws = qwen35_batched_decode_workspace_bytes(shape);
  require<Err>(workspace_bytes >= need_ws, "batched decode workspace is too small");
  const std::size_t per_seq = checked_mul<Err>(
      checked_mul<Err>(2 * kKvHeads * kHeadDim, shape.max_context_tokens,
                       "batched decode cache overflow"),
      sizeof(bf16_bits), "batched decode cache overflow");
  require<Err>(shape.cache_stride_bytes >= per_seq && shape.cache_stride_bytes % 16 == 0,
               "batched decode cache stride is too small or not 16-byte aligned");
  require<Err>(kv_cache_bytes >= checked_add<Err>(checked_mul<Err>(shape.sequences - 1,
                                                                   shape.cache_stride_bytes,
                                                                   "batched decode cache overflow"),
                                                  per_seq, "batched decode cache overflow"),
               "batched decode KV cache is too small");
  require<Err>(ceil_div_unchecked(shape.max_context_tokens, kBatchedPartition) * 4 <= 0x7FFFFFFF,
               "batched decode grid overflow");
  require_aligned16(query, "batched decode query must be 16-byte aligned");
  require_aligned16(kv_cache, "batched decode KV cache must be 16-byte aligned");
  require_aligned16(workspace, "batched decode workspace must be 16-byte aligned");
  if (act == RAFTINFER_DTYPE_F32)
    launch_batched<float>(query, key, value, gate, output, kv_cache, context_lengths, workspace,
                          shape, stream);
  else
    launch_batched<bf16_bits>(query, key, value, gate, output, kv_cache, context_lengths,
                              workspace, shape, stream);
}

} // namespace raftinfer::kernels
