// Gated DeltaNet (linear attention) for gfx950.
//
// Stages of qwen35_gated_delta (the reference's cpp/kernels/qwen35_delta.cu:
// 675-755 runs the same four):
//   1. conv_norm_kernel   causal depthwise conv (width W) + SiLU for every
//                         q/k/v channel of a token, L2-norm of q/k heads
//                         (q also x 1/sqrt(dk)), beta = sigmoid(b) and the log
//                         decay g = A * softplus(a + dt_bias) per value head.
//                         Fully parallel over (token, head vector).
//      conv_state_kernel  shifts the W-1 token convolution history.
//   2. recurrence, one of
//      recurrent_kernel   lane = state column, rows split across 8 waves, the
//                         fp32 state held in VGPRs over the token loop
//                         (decode and short prefill);
//      chunk_prep_kernel  per (value head, 64-token chunk), in parallel:
//      + chunk_scan_kernel  UT/WY form of the chunk (fp32 MFMA 16x16x4):
//                         A = beta_i e^{G_i-G_j} k_i.k_j (j<i), T = (I+A)^-1,
//                         W = T diag(beta e^G) K, U = T diag(beta) V,
//                         M = e^{G_i-G_j} q_i.k_j (j<=i); then per (value head,
//                         16-column block) sequentially over chunks:
//                         D = U - W S, O = e^G (Q S) + M D,
//                         S' = e^{G_last} S + (e^{G_last-G} K)^T D.
//                         Only differences G_i - G_j <= 0 are exponentiated.
//      chunk_tb_kernel    the same recurrence for bf16 q / k / v (the
//      + chunk_tscan_kernel core entry): the record holds only T diag(beta)
//                         and M, and the scan forms D = T diag(beta) (V -
//                         e^G K S) from the inputs.
//   3. out_norm_kernel    RMSNorm(raw) * w * SiLU(z) -> activation dtype.
// Host validation mirrors cpp/kernels/qwen35_delta.cu:26-135, :761-897.
#include "common.hpp"
#include "decode_scan.hpp"
#include "raftinfer_amd/qwen35_delta.hpp"

#include <cmath>
#include <type_traits>

namespace raftinfer::kernels {
namespace {

using namespace raftinfer::amd;
using Err = Qwen35DeltaError;

constexpr float kQkNormEpsilon = 1.0e-6f;
constexpr int kChunk = 64;
constexpr int kColBlock = 16;
constexpr int kChunkDim = 128;
constexpr int kRecWaves = 8;
constexpr std::size_t kChunkThreshold = 64;

// Chunk records: one per (value head, 64-token chunk), written by the prep
// kernel and streamed by the scan.  Rows past the chunk's last token are
// padded (W, U, M rows are 0 there).  bf16 pairs are the (hi, lo) split of an
// fp32 value: x = hi + lo with hi = bf16(x), lo = bf16(x - hi).
namespace rec {
constexpr std::size_t kW = 0;                                        // bf16 [2][64][128]  W
constexpr std::size_t kQ = kW + 2 * kChunk * kChunkDim * 2;          // bf16 [2][64][128]  Q * q_scale
constexpr std::size_t kKt = kQ + 2 * kChunk * kChunkDim * 2;         // bf16 [2][128][64]  (K * k_scale)^T
constexpr std::size_t kM = kKt + 2 * kChunkDim * kChunk * 2;         // bf16 [2][64][64]   M
constexpr std::size_t kU = kM + 2 * kChunk * kChunk * 2;             // f32  [64][128]     U
constexpr std::size_t kG = kU + kChunk * kChunkDim * 4;              // f32  [64]          G (padded with G[L-1])
constexpr std::size_t kBytes = kG + kChunk * 4;                      // 147,712
} // namespace rec

// Records of the bf16-input path (q, k, v exact in bf16): the scan reads Q,
// K and V from the inputs; the record holds the chunk's two 64 x 64 factors.
namespace rec2 {
constexpr std::size_t kTb = 0;                            // bf16 [2][64][64]  T diag(beta) (hi, lo)
constexpr std::size_t kM = kTb + 2 * kChunk * kChunk * 2; // bf16 [2][64][64]  M (hi, lo)
constexpr std::size_t kG = kM + 2 * kChunk * kChunk * 2;  // f32  [64]        G (padded with G[L-1])
constexpr std::size_t kBytes = kG + kChunk * 4;           // 33,024
} // namespace rec2

struct ChunkScratch {
  unsigned char *rec; // [hv][chunks] records of `bytes` (rec::kBytes or rec2::kBytes)
  std::size_t chunks;
  std::size_t bytes;
  __device__ __forceinline__ unsigned char *at(std::size_t h, std::size_t c) const {
    return rec + (h * chunks + c) * bytes;
  }
};

// Chunk records start on a 256-byte boundary after the per-token buffers.
std::size_t record_offset(std::size_t per_token_bytes) {
  return checked_add<Err>(per_token_bytes, 255, "gated-delta workspace byte size overflow") & ~std::size_t{255};
}

std::size_t chunk_record_bytes(std::size_t tokens, std::size_t hv, std::size_t dk, std::size_t dv,
                               std::size_t record = rec::kBytes) {
  if (dk != kChunkDim || dv != kChunkDim) return 0;
  return checked_mul<Err>(checked_mul<Err>(hv, ceil_div_unchecked(tokens, kChunk),
                                           "gated-delta workspace shape overflow"),
                          record, "gated-delta workspace shape overflow");
}

// The model shapes whose convolution runs channel-spread (conv_norm_wide_kernel):
// their chunked prefill uses the 33,024-byte T-records, so the workspace is
// sized for those; other dk = dv = 128 shapes take the 147,712-byte W/U records.
bool channel_spread_shape(const GatedDeltaShape &s, std::size_t conv_dim) {
  return s.key_dim == kChunkDim && s.value_dim == kChunkDim && s.conv_width == 4 && conv_dim % 2048 == 0 &&
         s.hidden_size % 2048 == 0;
}

struct CheckedShape {
  std::size_t key_size, value_size, conv_dim, token_stride, convolution_elements,
      recurrent_elements, workspace_bytes;
};

// cpp/kernels/qwen35_delta.cu:67-135.  The workspace additionally holds
// per-token beta / log-decay and the chunk scratch (still linear in tokens).
CheckedShape validate_shape(const GatedDeltaShape &s) {
  require<Err>(s.tokens > 0, "gated-delta tokens must be positive");
  require<Err>(s.hidden_size > 0, "gated-delta hidden_size must be positive");
  require<Err>(s.key_heads > 0, "gated-delta key_heads must be positive");
  require<Err>(s.value_heads > 0, "gated-delta value_heads must be positive");
  require<Err>(s.key_dim > 0, "gated-delta key_dim must be positive");
  require<Err>(s.value_dim > 0, "gated-delta value_dim must be positive");
  require<Err>(s.conv_width > 0, "gated-delta conv_width must be positive");
  require<Err>(std::isfinite(s.epsilon) && s.epsilon >= 0.0f,
               "gated-delta epsilon must be finite and non-negative");
  require<Err>(s.value_heads % s.key_heads == 0,
               "gated-delta value_heads must be divisible by key_heads");
  const std::size_t key_size = checked_mul<Err>(s.key_heads, s.key_dim, "gated-delta key shape overflow");
  const std::size_t value_size =
      checked_mul<Err>(s.value_heads, s.value_dim, "gated-delta value shape overflow");
  require<Err>(value_size == s.hidden_size,
               "gated-delta value_heads * value_dim must equal hidden_size");
  const std::size_t conv_dim =
      checked_add<Err>(checked_mul<Err>(key_size, 2, "gated-delta convolution shape overflow"),
                       value_size, "gated-delta convolution shape overflow");
  const std::size_t token_stride = checked_add<Err>(
      checked_add<Err>(conv_dim, checked_mul<Err>(s.value_heads, 2, "gated-delta input shape overflow"),
                       "gated-delta input shape overflow"),
      s.hidden_size, "gated-delta input shape overflow");
  (void)checked_mul<Err>(s.tokens, token_stride, "gated-delta input shape overflow");
  (void)checked_mul<Err>(s.tokens, s.hidden_size, "gated-delta output shape overflow");
  (void)checked_mul<Err>(conv_dim, s.conv_width, "gated-delta convolution weight shape overflow");
  const std::size_t conv_elems = checked_mul<Err>(conv_dim, s.conv_width - 1,
                                                  "gated-delta convolution state shape overflow");
  const std::size_t rec_elems =
      checked_mul<Err>(value_size, s.key_dim, "gated-delta recurrent state shape overflow");
  require<Err>(s.value_dim <= std::numeric_limits<std::size_t>::max() / 4 &&
                   s.key_dim <= std::numeric_limits<std::size_t>::max() / 4,
               "gated-delta workspace shape overflow");
  const std::size_t per_token = checked_add<Err>(
      checked_add<Err>(conv_dim, s.hidden_size, "gated-delta workspace shape overflow"),
      checked_mul<Err>(2, s.value_heads, "gated-delta workspace shape overflow"),
      "gated-delta workspace shape overflow");
  std::size_t ws_bytes = checked_mul<Err>(
      checked_mul<Err>(s.tokens, per_token, "gated-delta workspace shape overflow"), sizeof(float),
      "gated-delta workspace byte size overflow");
  const std::size_t records =
      chunk_record_bytes(s.tokens, s.value_heads, s.key_dim, s.value_dim,
                         channel_spread_shape(s, conv_dim) ? rec2::kBytes : rec::kBytes);
  if (records != 0)
    ws_bytes = checked_add<Err>(record_offset(ws_bytes), records,
                                "gated-delta workspace byte size overflow");
  const auto int_max = static_cast<std::size_t>(std::numeric_limits<int>::max());
  require<Err>(s.tokens <= int_max, "gated-delta token count exceeds launch limit");
  require<Err>(conv_dim <= int_max, "gated-delta convolution grid overflow");
  require<Err>(s.key_heads * 2 <= int_max, "gated-delta Q/K normalization grid overflow");
  require<Err>(s.value_heads <= 65535, "gated-delta recurrent grid overflow");
  return {key_size, value_size, conv_dim, token_stride, conv_elems, rec_elems, ws_bytes};
}

void require_dtype(RaftInferDataType d) {
  require<Err>(d == RAFTINFER_DTYPE_F32 || d == RAFTINFER_DTYPE_F16 || d == RAFTINFER_DTYPE_BF16,
               "unsupported Qwen3.5 gated-delta dtype");
}

void require_weight_dtype(RaftInferDataType d, RaftInferDataType w) {
  require<Err>(w == RAFTINFER_DTYPE_F32 || w == d ||
                   (d == RAFTINFER_DTYPE_F32 && (w == RAFTINFER_DTYPE_F16 || w == RAFTINFER_DTYPE_BF16)),
               "Qwen3.5 gated-delta weight dtype is incompatible with activations");
}

void require_aligned(const void *p, std::size_t a, const char *m) {
  require<Err>(reinterpret_cast<std::uintptr_t>(p) % a == 0, m);
}

// cpp/kernels/qwen35_delta.cu:188-217
void validate_policy(const GatedDeltaLaunchPolicy &p, const GatedDeltaShape &s) {
  require<Err>(p.warps_per_block == 4, "gated-delta schedule requires four warps per block");
  require<Err>(!p.transposed_boundary_state, "gated-delta transposed boundary state is not initialized");
  switch (p.schedule) {
  case GatedDeltaSchedule::register_resident_current: break;
  case GatedDeltaSchedule::register_resident_prefill_sm120:
    require<Err>(s.key_dim == 64 || s.key_dim == 128,
                 "gated-delta sm120 schedule requires key dimension 64 or 128");
    require<Err>(s.value_dim == s.key_dim,
                 "gated-delta sm120 schedule requires matching value dimension");
    break;
  case GatedDeltaSchedule::register_resident_decode_sm120:
    require<Err>(s.key_dim == 64 || s.key_dim == 128,
                 "gated-delta sm120 schedule requires key dimension 64 or 128");
    require<Err>(s.value_dim == s.key_dim,
                 "gated-delta sm120 schedule requires matching value dimension");
    require<Err>(s.tokens == 1, "gated-delta decode schedule requires exactly one token");
    break;
  default: throw Err("unknown gated-delta schedule");
  }
}

// ---------------------------------------------------------- device math
// Split of a float pair into packed (hi, lo) bf16 pairs.
__device__ __forceinline__ void split2(float a, float b, std::uint32_t &h, std::uint32_t &l) {
  h = pack_bf16x2(a, b);
  l = pack_bf16x2(a - bf16_lo(h), b - bf16_hi(h));
}
// The hardware reciprocal (1 ulp) instead of an IEEE division, whose
// scale / FMA / fix-up sequence per element made SiLU the costliest part of
// the convolution and output norm (T = 512 entry 45.5 -> 44.4 us).
__device__ __forceinline__ float silu(float v) { return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v)); }
__device__ __forceinline__ float sigmoid(float v) { return __builtin_amdgcn_rcpf(1.0f + __expf(-v)); }
__device__ __forceinline__ float softplus(float v) {
  if (v > 20.0f) return v;
  if (v < -20.0f) return __expf(v);
  return log1pf(__expf(v));
}

// Strided row source for q / k / v: element (t, head, i) at
// base[t*row + head*head_stride + i] * scale.
template <typename T> struct Src {
  const T *base;
  std::size_t row, head_stride;
  float scale;
  __device__ __forceinline__ float at(std::size_t t, std::size_t head, std::size_t i) const {
    return Elem<T>::load(base, t * row + head * head_stride + i) * scale;
  }
};

template <typename T> struct OutRows {
  T *base; // [t][head][dv]
  __device__ __forceinline__ void put(std::size_t idx, float v) const { Elem<T>::store(base, idx, v); }
};

// Where a token's input rows come from: the packed [q k v | b | a | z] row of
// qwen35_gated_delta (cpp/kernels/qwen35_delta.cuh:77-86; every stride is the
// packed width), or the four projection outputs that
// qwen35_pack_linear_delta_input would pack (cpp/kernels/qwen35_primitives.cu:
// 388-420), read in place by qwen35_gated_delta_unpacked.
template <typename T> struct DeltaRows {
  const T *qkv; // conv channel c of token t at qkv[t * qkv_stride + c]
  std::size_t qkv_stride;
  const T *b; // beta logit of value head h at b[t * b_stride + h]
  std::size_t b_stride;
  const T *a; // decay logit
  std::size_t a_stride;
  const T *z; // output gate, value channel c at z[t * z_stride + c]
  std::size_t z_stride;
  __device__ __forceinline__ float x(std::size_t t, std::size_t c) const {
    return Elem<T>::load(qkv, t * qkv_stride + c);
  }
  __device__ __forceinline__ float gate(std::size_t t, std::size_t c) const {
    return Elem<T>::load(z, t * z_stride + c);
  }
};

// -------------------------------------------------------- stage 1 kernels

// Block (token, vector): vector < Hk -> q head, < 2Hk -> k head, else v head.
template <typename T, typename Wt>
__global__ __launch_bounds__(256) void conv_norm_kernel(
    DeltaRows<T> in, const Wt *__restrict__ conv_w, const float *__restrict__ conv_state,
    const Wt *__restrict__ recurrent_a, const Wt *__restrict__ dt_bias, float *__restrict__ convolved,
    float *__restrict__ beta, float *__restrict__ gdecay, std::size_t tokens,
    std::size_t conv_dim, std::size_t hk, std::size_t hv, std::size_t dk, std::size_t dv,
    std::size_t width) {
  __shared__ float red[4];
  const std::size_t t = blockIdx.x;
  const std::size_t vec = blockIdx.y;
  const bool is_q = vec < hk, is_k = !is_q && vec < 2 * hk;
  const std::size_t base = is_q ? vec * dk : is_k ? hk * dk + (vec - hk) * dk : 2 * hk * dk + (vec - 2 * hk) * dv;
  const std::size_t len = (is_q || is_k) ? dk : dv;
  const std::size_t hist = width - 1;
  float ss = 0.f;
  float vals[4];
  int n = 0;
  for (std::size_t i = threadIdx.x; i < len; i += 256, ++n) {
    const std::size_t ch = base + i;
    const std::size_t wb = ch * width;
    float sum = in.x(t, ch) * Elem<Wt>::load(conv_w, wb + hist);
    for (std::size_t h = 0; h < hist; ++h) {
      const std::size_t src = t + h;
      const float prev = src < hist ? conv_state[ch * hist + src]
                                    : in.x(src - hist, ch);
      sum += prev * Elem<Wt>::load(conv_w, wb + h);
    }
    const float y = silu(sum);
    if (n < 4) vals[n] = y;
    ss += y * y;
    if (!(is_q || is_k)) convolved[t * conv_dim + ch] = y;
  }
  if (is_q || is_k) {
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float total = red[0] + red[1] + red[2] + red[3];
    float scale = 1.0f / sqrtf(total + kQkNormEpsilon);
    if (is_q) scale *= 1.0f / sqrtf(static_cast<float>(dk));
    n = 0;
    for (std::size_t i = threadIdx.x; i < len; i += 256, ++n) {
      float y = vals[n < 4 ? n : 3];
      if (n >= 4) { // dims > 1024: recompute (never hit for Qwen3.5 shapes)
        const std::size_t ch = base + i;
        const std::size_t wb = ch * width;
        float sum = in.x(t, ch) * Elem<Wt>::load(conv_w, wb + hist);
        for (std::size_t h = 0; h < hist; ++h) {
          const std::size_t src = t + h;
          const float prev = src < hist ? conv_state[ch * hist + src]
                                        : in.x(src - hist, ch);
          sum += prev * Elem<Wt>::load(conv_w, wb + h);
        }
        y = silu(sum);
      }
      convolved[t * conv_dim + base + i] = y * scale;
    }
  }
  if (vec == 0) {
    for (std::size_t h = threadIdx.x; h < hv; h += 256) {
      const float b = Elem<T>::load(in.b, t * in.b_stride + h);
      const float a = Elem<T>::load(in.a, t * in.a_stride + h);
      beta[t * hv + h] = sigmoid(b);
      gdecay[t * hv + h] = Elem<Wt>::load(recurrent_a, h) * softplus(a + Elem<Wt>::load(dt_bias, h));
    }
  }
}

// Vector loads of 8 consecutive activation / weight values.
template <typename T> __device__ __forceinline__ void load8(const T *p, float (&x)[8]) {
  if constexpr (std::is_same_v<T, float>) {
    const float4 a = *reinterpret_cast<const float4 *>(p), b = *reinterpret_cast<const float4 *>(p + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  } else {
    const u32x4 w = *reinterpret_cast<const u32x4 *>(p);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const std::uint16_t bits = static_cast<std::uint16_t>(w[e >> 1] >> ((e & 1) * 16));
      if constexpr (std::is_same_v<T, bf16_bits>)
        x[e] = bf16_to_f32(bits);
      else
        x[e] = static_cast<float>(__builtin_bit_cast(_Float16, bits));
    }
  }
}

// Qwen3.5 head dims (dk = dv = 128): one block per token, 8 channels per
// thread; a 128-channel head is one 16-lane DPP row, so the q/k L2 norms
// reduce in-row.  Same math as conv_norm_kernel.
template <typename T, typename Wt, int W>
__global__ __launch_bounds__(256) void conv_norm_fast_kernel(
    DeltaRows<T> in, const Wt *__restrict__ conv_w, const float *__restrict__ conv_state,
    const Wt *__restrict__ recurrent_a, const Wt *__restrict__ dt_bias, float *__restrict__ convolved,
    float *__restrict__ beta, float *__restrict__ gdecay, std::size_t conv_dim,
    std::size_t qk_channels, std::size_t hv) {
  constexpr int H = W - 1;
  const std::size_t t = blockIdx.x;
  const float qscale = 1.0f / sqrtf(static_cast<float>(kChunkDim));
  for (std::size_t base = 0; base < conv_dim; base += 2048) {
    const std::size_t c = base + 8 * threadIdx.x;
    float cur[8], prev[H > 0 ? H : 1][8], w[8][W];
    load8(in.qkv + t * in.qkv_stride + c, cur);
#pragma unroll
    for (int h = 0; h < H; ++h) {
      const std::size_t src = t + h;
      if (src < static_cast<std::size_t>(H)) {
#pragma unroll
        for (int e = 0; e < 8; ++e) prev[h][e] = conv_state[(c + e) * H + src];
      } else {
        load8(in.qkv + (src - H) * in.qkv_stride + c, prev[h]);
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int k = 0; k < W; ++k) w[e][k] = Elem<Wt>::load(conv_w, (c + e) * W + k);
    float y[8], ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float sum = cur[e] * w[e][H];
#pragma unroll
      for (int h = 0; h < H; ++h) sum += prev[h][e] * w[e][h];
      y[e] = silu(sum);
      ss += y[e] * y[e];
    }
    if (c < qk_channels) { // q or k head: L2 norm over its 128 channels
      ss = row16_sum(ss);
      float scale = 1.0f / sqrtf(ss + kQkNormEpsilon);
      if (c < qk_channels / 2) scale *= qscale;
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] *= scale;
    }
    float *dst = convolved + t * conv_dim + c;
    *reinterpret_cast<float4 *>(dst) = make_float4(y[0], y[1], y[2], y[3]);
    *reinterpret_cast<float4 *>(dst + 4) = make_float4(y[4], y[5], y[6], y[7]);
  }
  for (std::size_t h = threadIdx.x; h < hv; h += 256) {
    const float b = Elem<T>::load(in.b, t * in.b_stride + h);
    const float a = Elem<T>::load(in.a, t * in.a_stride + h);
    beta[t * hv + h] = sigmoid(b);
    gdecay[t * hv + h] = Elem<Wt>::load(recurrent_a, h) * softplus(a + Elem<Wt>::load(dt_bias, h));
  }
}

// Qwen3.5 shapes, spread over channels: workgroup (TT consecutive tokens,
// 512-channel block), one wave, 8 channels per lane (a 128-channel head is one
// 16-lane DPP row), so a one-token call still spans conv_dim / 512 CUs.
// Input, weights and history are read as 16-byte vectors, every load of the
// workgroup is issued before the first use, and the TT tokens slide one
// window over their inputs (TT + 3 rows read for TT outputs).  With
// kUpdateState (one token) the lane that reads a channel's history also writes
// its shifted history, so no separate state update runs.  Same math as
// conv_norm_kernel.
constexpr int kConvWideChannels = 512;
// kSplitOut: the convolved rows go out as two bf16 planes, x = hi + lo with
// hi = bf16(x), lo = bf16(x - hi) (hi at element t * conv_dim + c of the
// buffer, lo tokens * conv_dim elements further), the form the chunked scan
// reads; otherwise as fp32 rows.
template <typename T, typename Wt, int W, int TT, bool kUpdateState, bool kSplitOut = false>
__global__ __launch_bounds__(64) void conv_norm_wide_kernel(
    DeltaRows<T> in, const Wt *__restrict__ conv_w, float *__restrict__ conv_state,
    const Wt *__restrict__ recurrent_a, const Wt *__restrict__ dt_bias, float *__restrict__ convolved,
    float *__restrict__ beta, float *__restrict__ gdecay, std::size_t tokens,
    std::size_t conv_dim, std::size_t qk_channels, std::size_t hv) {
  constexpr int H = W - 1;
  static_assert(H == 3, "history vectors assume a width-4 convolution");
  static_assert(!kUpdateState || TT == 1, "the fused state update is for one-token calls");
  const std::size_t t0 = static_cast<std::size_t>(blockIdx.x) * TT;
  const std::size_t c = static_cast<std::size_t>(blockIdx.y) * kConvWideChannels + 8 * threadIdx.x;
  // beta and the decay of the block's tokens: from an extra row of blocks
  // past the channels when the grid has one (it then costs no other block a
  // further round trip), else from the first block of channels.
  auto beta_decay = [&]() {
    for (int i = threadIdx.x; i < TT * static_cast<int>(hv); i += 64) {
      const std::size_t t = t0 + i / hv, h = i % hv;
      if (t >= tokens) break;
      const float b = Elem<T>::load(in.b, t * in.b_stride + h);
      const float a = Elem<T>::load(in.a, t * in.a_stride + h);
      beta[t * hv + h] = sigmoid(b);
      gdecay[t * hv + h] = Elem<Wt>::load(recurrent_a, h) * softplus(a + Elem<Wt>::load(dt_bias, h));
    }
  };
  if (c >= conv_dim) {
    beta_decay();
    return;
  }
  // win[j]: the input row of extended index t0 + j, where extended indices
  // 0..H-1 are the stored history and H + t is token t.
  float win[H + TT][8], w[8 * W];
#pragma unroll
  for (int u = 0; u < TT; ++u) {
    const std::size_t t = t0 + u < tokens ? t0 + u : tokens - 1;
    load8(in.qkv + t * in.qkv_stride + c, win[H + u]);
  }
#pragma unroll
  for (int j = 0; j < W; ++j) {
    float x[8];
    load8(conv_w + c * W + 8 * j, x);
#pragma unroll
    for (int e = 0; e < 8; ++e) w[8 * j + e] = x[e];
  }
  float hist[8 * H]; // history of channel c + e, slot s: conv_state[(c + e) * H + s]
  if (t0 < static_cast<std::size_t>(H)) {
    const float4 *hp = reinterpret_cast<const float4 *>(conv_state + c * H);
#pragma unroll
    for (int j = 0; j < 2 * H; ++j) {
      const float4 v = hp[j];
      hist[4 * j] = v.x; hist[4 * j + 1] = v.y; hist[4 * j + 2] = v.z; hist[4 * j + 3] = v.w;
    }
  }
#pragma unroll
  for (int h = 0; h < H; ++h) {
    const std::size_t src = t0 + h;
    if (src < static_cast<std::size_t>(H)) {
#pragma unroll
      for (int e = 0; e < 8; ++e) win[h][e] = hist[e * H + static_cast<int>(src)];
    } else {
      load8(in.qkv + (src - H) * in.qkv_stride + c, win[h]);
    }
  }
  const bool qk = c < qk_channels;
  const float qscale = c < qk_channels / 2 ? 1.0f / sqrtf(static_cast<float>(kChunkDim)) : 1.0f;
#pragma unroll
  for (int u = 0; u < TT; ++u) {
    if (t0 + u >= tokens) break;
    float y[8], ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float sum = win[H + u][e] * w[e * W + H];
#pragma unroll
      for (int h = 0; h < H; ++h) sum += win[u + h][e] * w[e * W + h];
      y[e] = silu(sum);
      ss += y[e] * y[e];
    }
    if (qk) { // q or k head: L2 norm over its 128 channels
      ss = row16_sum(ss);
      const float scale = qscale / sqrtf(ss + kQkNormEpsilon);
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] *= scale;
    }
    if constexpr (kSplitOut) {
      u32x4 hi, lo;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        std::uint32_t hw, lw;
        split2(y[2 * e], y[2 * e + 1], hw, lw);
        hi[e] = hw;
        lo[e] = lw;
      }
      bf16_bits *dst = reinterpret_cast<bf16_bits *>(convolved) + (t0 + u) * conv_dim + c;
      // Streaming stores (the planes are read by the next kernels from the
      // MALL): 9.1 -> 7.8 us at T=512, 8192 channels.
      __builtin_nontemporal_store(hi, reinterpret_cast<u32x4 *>(dst));
      __builtin_nontemporal_store(lo, reinterpret_cast<u32x4 *>(dst + tokens * conv_dim));
    } else {
      float *dst = convolved + (t0 + u) * conv_dim + c;
      *reinterpret_cast<float4 *>(dst) = make_float4(y[0], y[1], y[2], y[3]);
      *reinterpret_cast<float4 *>(dst + 4) = make_float4(y[4], y[5], y[6], y[7]);
    }
  }
  if constexpr (kUpdateState) {
    // one token: the new history of channel c + e is (slot 1, slot 2, cur)
    float nh[8 * H];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      nh[e * H] = hist[e * H + 1];
      nh[e * H + 1] = hist[e * H + 2];
      nh[e * H + 2] = win[H][e];
    }
    float4 *hp = reinterpret_cast<float4 *>(conv_state + c * H);
#pragma unroll
    for (int j = 0; j < 2 * H; ++j) hp[j] = make_float4(nh[4 * j], nh[4 * j + 1], nh[4 * j + 2], nh[4 * j + 3]);
  }
  if (blockIdx.y == 0 && gridDim.y * static_cast<std::size_t>(kConvWideChannels) == conv_dim) beta_decay();
}

// Shifts the convolution history of the channels this thread owns (channel
// ch = first, first + step, ...): slot s becomes the input row of token
// tokens - H + s, or the old slot s + tokens when that token precedes the call.
// Runs in a kernel that starts after every read of the old history has
// finished (a later launch on the same stream), and each channel has one
// owner, so the update is race-free.
template <int H, typename T>
__device__ __forceinline__ void shift_conv_history(const DeltaRows<T> &in,
                                                   float *__restrict__ conv_state,
                                                   std::size_t tokens, std::size_t conv_dim,
                                                   std::size_t first, std::size_t step) {
  for (std::size_t ch = first; ch < conv_dim; ch += step) {
    float nh[H];
#pragma unroll
    for (int s = 0; s < H; ++s) {
      const std::size_t src = tokens + s; // extended index
      nh[s] = src < static_cast<std::size_t>(H) ? conv_state[ch * H + src]
                                                : in.x(src - H, ch);
    }
#pragma unroll
    for (int s = 0; s < H; ++s) conv_state[ch * H + s] = nh[s];
  }
}

// One block per token; a 128-wide value head is one 16-lane DPP row.
template <typename T, typename Wt>
__global__ __launch_bounds__(256) void out_norm_fast_kernel(DeltaRows<T> in,
                                                            const Wt *__restrict__ norm_w,
                                                            const float *__restrict__ raw,
                                                            T *__restrict__ output,
                                                            std::size_t conv_dim, std::size_t hv,
                                                            float eps,
                                                            float *__restrict__ conv_state,
                                                            std::size_t tokens) {
  const std::size_t t = blockIdx.x;
  const std::size_t hidden = hv * kChunkDim;
  // the convolution history update of the whole call, spread over the grid
  if (conv_state != nullptr)
    shift_conv_history<3>(in, conv_state, tokens, conv_dim, t * 256 + threadIdx.x, tokens * 256);
  for (std::size_t base = 0; base < hidden; base += 2048) {
    const std::size_t c = base + 8 * threadIdx.x;
    const float4 r0 = *reinterpret_cast<const float4 *>(raw + t * hidden + c);
    const float4 r1 = *reinterpret_cast<const float4 *>(raw + t * hidden + c + 4);
    const float x[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
    ss = row16_sum(ss);
    const float scale = rsqrtf(ss / static_cast<float>(kChunkDim) + eps);
    float z[8];
    load8(in.z + t * in.z_stride + c, z);
    const std::size_t wc = c % kChunkDim;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      Elem<T>::store(output, t * hidden + c + e,
                     x[e] * scale * Elem<Wt>::load(norm_w, wc + e) * silu(z[e]));
  }
}

template <typename T>
__global__ __launch_bounds__(256) void conv_state_kernel(DeltaRows<T> in,
                                                         float *__restrict__ conv_state,
                                                         std::size_t tokens, std::size_t conv_dim,
                                                         std::size_t width) {
  const std::size_t ch = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (ch >= conv_dim) return;
  const std::size_t hist = width - 1;
  for (std::size_t h = 0; h < hist; ++h) {
    const std::size_t src = tokens + h;
    conv_state[ch * hist + h] = src < hist ? conv_state[ch * hist + src]
                                           : in.x(src - hist, ch);
  }
}

// ------------------------------------------------ stage 2a: recurrent
// Block (value head, 64-column block).  Lane = column; wave w owns rows
// [w*MAXR, (w+1)*MAXR).  Per token: S *= decay; kv = S^T k (cross-wave sum
// in LDS); delta = beta (v - kv); S += k delta; o = S^T q (cross-wave sum).
template <typename InT, typename OutT, int MAXR>
__global__ __launch_bounds__(kRecWaves * 64) void recurrent_kernel(
    Src<InT> qs, Src<InT> ks, Src<InT> vs, const float *__restrict__ beta,
    const float *__restrict__ gdecay, float *__restrict__ state, OutT *__restrict__ out,
    std::size_t tokens, std::size_t hk, std::size_t hv, std::size_t dk, std::size_t dv) {
  __shared__ float red_kv[kRecWaves][64];
  __shared__ float red_o[kRecWaves][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const std::size_t h = blockIdx.x;
  const std::size_t kh = h % hk;
  const std::size_t c = static_cast<std::size_t>(blockIdx.y) * 64 + lane;
  const bool cvalid = c < dv;
  float s[MAXR];
  float *sh = state + h * dk * dv;
#pragma unroll
  for (int i = 0; i < MAXR; ++i) {
    const std::size_t r = static_cast<std::size_t>(wave) * MAXR + i;
    s[i] = (r < dk && cvalid) ? sh[r * dv + c] : 0.f;
  }
  for (std::size_t t = 0; t < tokens; ++t) {
    const float b = beta[t * hv + h];
    const float decay = __expf(gdecay[t * hv + h]);
    float kr[MAXR];
    float part = 0.f;
#pragma unroll
    for (int i = 0; i < MAXR; ++i) {
      const std::size_t r = static_cast<std::size_t>(wave) * MAXR + i;
      kr[i] = r < dk ? ks.at(t, kh, r) : 0.f;
      s[i] *= decay;
      part = fmaf(s[i], kr[i], part);
    }
    red_kv[wave][lane] = part;
    __syncthreads();
    float kv = 0.f;
#pragma unroll
    for (int w = 0; w < kRecWaves; ++w) kv += red_kv[w][lane];
    const float delta = ((cvalid ? vs.at(t, h, c) : 0.f) - kv) * b;
    float po = 0.f;
#pragma unroll
    for (int i = 0; i < MAXR; ++i) {
      const std::size_t r = static_cast<std::size_t>(wave) * MAXR + i;
      s[i] = fmaf(kr[i], delta, s[i]);
      po = fmaf(s[i], r < dk ? qs.at(t, kh, r) : 0.f, po);
    }
    red_o[wave][lane] = po;
    __syncthreads();
    if (wave == 0 && cvalid) {
      float o = 0.f;
#pragma unroll
      for (int w = 0; w < kRecWaves; ++w) o += red_o[w][lane];
      Elem<OutT>::store(out, (t * hv + h) * dv + c, o);
    }
  }
#pragma unroll
  for (int i = 0; i < MAXR; ++i) {
    const std::size_t r = static_cast<std::size_t>(wave) * MAXR + i;
    if (r < dk && cvalid) sh[r * dv + c] = s[i];
  }
}

// Model-shape recurrence (dk = dv = 128), block (value head, 32-column
// block), 256 threads: thread (row group rg = tid / 8, column quad cq =
// tid % 8) holds S[4 rg .. 4 rg + 3][c0 + 4 cq .. + 3] as four float4 rows, so
// every state load or store instruction of a wave covers 8 whole 128-byte
// rows.  The sums over the 128 rows run as a butterfly over the 8 row groups
// of a wave (lanes ^ 8, ^ 16, ^ 32) and an LDS sum over the 4 waves; every
// thread then holds kv (and o) of its 4 columns.  Same update order as the
// generic kernel: S *= decay; kv = S^T k; delta = beta (v - kv); S += k delta;
// o = S^T q.
constexpr int kRec128Cols = 32;
template <typename InT, typename OutT>
__global__ __launch_bounds__(256) void recurrent_128_kernel(
    Src<InT> qs, Src<InT> ks, Src<InT> vs, const float *__restrict__ beta,
    const float *__restrict__ gdecay, float *__restrict__ state, OutT *__restrict__ out,
    std::size_t tokens, std::size_t hk, std::size_t hv) {
  constexpr int kDim = 128;
  __shared__ float4 red[2][4][kRec128Cols / 4]; // [kv / o][wave][column quad]
  const int tid = threadIdx.x, wave = tid >> 6;
  const int cq = tid & 7, rg = tid >> 3;
  const std::size_t h = blockIdx.x;
  const std::size_t kh = h % hk;
  const int c0 = blockIdx.y * kRec128Cols + 4 * cq;
  float *sh = state + h * kDim * kDim;
  float4 s[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) s[i] = *reinterpret_cast<const float4 *>(sh + (4 * rg + i) * kDim + c0);
  auto row_sum = [&](float4 x, int which) {
    // lanes ^ 8 (DPP row_ror:8), ^ 16, ^ 32 hold the other row groups of
    // this wave for the same column quad.
    x.x = sum_xor32(sum_xor16(sum_xor8(x.x)));
    x.y = sum_xor32(sum_xor16(sum_xor8(x.y)));
    x.z = sum_xor32(sum_xor16(sum_xor8(x.z)));
    x.w = sum_xor32(sum_xor16(sum_xor8(x.w)));
    if ((tid & 63) < 8) red[which][wave][cq] = x;
    __syncthreads();
    float4 t = red[which][0][cq];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      const float4 u = red[which][w][cq];
      t.x += u.x; t.y += u.y; t.z += u.z; t.w += u.w;
    }
    return t;
  };
  for (std::size_t t = 0; t < tokens; ++t) {
    const float b = beta[t * hv + h];
    const float decay = __expf(gdecay[t * hv + h]);
    float kr[4], qr[4], vv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kr[i] = ks.at(t, kh, 4 * rg + i);
      qr[i] = qs.at(t, kh, 4 * rg + i);
      vv[i] = vs.at(t, h, c0 + i);
    }
    float4 part = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s[i].x *= decay; s[i].y *= decay; s[i].z *= decay; s[i].w *= decay;
      part.x = fmaf(s[i].x, kr[i], part.x);
      part.y = fmaf(s[i].y, kr[i], part.y);
      part.z = fmaf(s[i].z, kr[i], part.z);
      part.w = fmaf(s[i].w, kr[i], part.w);
    }
    const float4 kv = row_sum(part, 0);
    const float4 d = make_float4((vv[0] - kv.x) * b, (vv[1] - kv.y) * b, (vv[2] - kv.z) * b,
                                 (vv[3] - kv.w) * b);
    float4 po = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s[i].x = fmaf(kr[i], d.x, s[i].x);
      s[i].y = fmaf(kr[i], d.y, s[i].y);
      s[i].z = fmaf(kr[i], d.z, s[i].z);
      s[i].w = fmaf(kr[i], d.w, s[i].w);
      po.x = fmaf(s[i].x, qr[i], po.x);
      po.y = fmaf(s[i].y, qr[i], po.y);
      po.z = fmaf(s[i].z, qr[i], po.z);
      po.w = fmaf(s[i].w, qr[i], po.w);
    }
    const float4 o = row_sum(po, 1);
    if (rg == 0) {
      const std::size_t base = (t * hv + h) * kDim + c0;
      Elem<OutT>::store(out, base, o.x);
      Elem<OutT>::store(out, base + 1, o.y);
      Elem<OutT>::store(out, base + 2, o.z);
      Elem<OutT>::store(out, base + 3, o.w);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) *reinterpret_cast<float4 *>(sh + (4 * rg + i) * kDim + c0) = s[i];
}

// Recurrence + output norm for the Qwen3.5 shape (dk = dv = 128) when the
// whole call is recurrent (decode, short prefill): one workgroup of 8 waves
// per value head holds the head's full fp32 state, thread (row group rg =
// tid / 32, column quad cq = tid % 32) rows 8 rg .. 8 rg + 7 of columns
// 4 cq .. 4 cq + 3, so each state load or store instruction of a wave covers
// two whole 512-byte rows.  Owning all 128 columns lets the workgroup finish
// RMSNorm(o) * w * SiLU(z) itself (cpp/kernels/qwen35_delta.cu:578-621), so
// no separate norm kernel runs.  Same update order as recurrent_128_kernel.
template <typename T, typename Wt>
__global__ __launch_bounds__(512) void recurrent_head_norm_kernel(
    Src<float> qs, Src<float> ks, Src<float> vs, const float *__restrict__ beta,
    const float *__restrict__ gdecay, float *__restrict__ state, DeltaRows<T> in,
    const Wt *__restrict__ norm_w, T *__restrict__ output, std::size_t tokens, std::size_t hk,
    std::size_t hv, std::size_t conv_dim, float eps,
    float *__restrict__ conv_state) {
  constexpr int kDim = 128, kRows = 8;
  // the convolution history update of the whole call (multi-token calls),
  // spread over the grid
  if (conv_state != nullptr)
    shift_conv_history<3>(in, conv_state, tokens, conv_dim, blockIdx.x * 512 + threadIdx.x, hv * 512);
  __shared__ float4 red[2][8][32]; // [kv / o][wave][column quad]
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int cq = tid & 31, rg = tid >> 5;
  const std::size_t h = blockIdx.x;
  const std::size_t kh = h % hk;
  const int c0 = 4 * cq, r0 = kRows * rg;
  float *sh = state + h * kDim * kDim;
  float4 s[kRows];
#pragma unroll
  for (int i = 0; i < kRows; ++i) s[i] = *reinterpret_cast<const float4 *>(sh + (r0 + i) * kDim + c0);
  // norm weight and, per token, the z gate of this lane's four columns
  float nw[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) nw[i] = Elem<Wt>::load(norm_w, c0 + i);
  auto row_sum = [&](float4 x, int which) {
    // lane ^ 32 holds the other row group of this wave for the same quad
    x.x = sum_xor32(x.x);
    x.y = sum_xor32(x.y);
    x.z = sum_xor32(x.z);
    x.w = sum_xor32(x.w);
    if (lane < 32) red[which][wave][cq] = x;
    __syncthreads();
    float4 t = red[which][0][cq];
#pragma unroll
    for (int w = 1; w < 8; ++w) {
      const float4 u = red[which][w][cq];
      t.x += u.x; t.y += u.y; t.z += u.z; t.w += u.w;
    }
    return t;
  };
  const std::size_t hidden = hv * kDim;
  for (std::size_t t = 0; t < tokens; ++t) {
    const float b = beta[t * hv + h];
    const float decay = __expf(gdecay[t * hv + h]);
    float kr[kRows], qr[kRows], vv[4], z[4];
    const float4 *kp = reinterpret_cast<const float4 *>(ks.base + t * ks.row + kh * ks.head_stride + r0);
    const float4 *qp = reinterpret_cast<const float4 *>(qs.base + t * qs.row + kh * qs.head_stride + r0);
#pragma unroll
    for (int j = 0; j < kRows / 4; ++j) {
      const float4 a = kp[j], q4 = qp[j];
      kr[4 * j] = a.x; kr[4 * j + 1] = a.y; kr[4 * j + 2] = a.z; kr[4 * j + 3] = a.w;
      qr[4 * j] = q4.x; qr[4 * j + 1] = q4.y; qr[4 * j + 2] = q4.z; qr[4 * j + 3] = q4.w;
    }
    const float4 v4 = *reinterpret_cast<const float4 *>(vs.base + t * vs.row + h * vs.head_stride + c0);
    vv[0] = v4.x; vv[1] = v4.y; vv[2] = v4.z; vv[3] = v4.w;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      z[i] = in.gate(t, h * kDim + c0 + i);
    float4 part = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      s[i].x *= decay; s[i].y *= decay; s[i].z *= decay; s[i].w *= decay;
      part.x = fmaf(s[i].x, kr[i], part.x);
      part.y = fmaf(s[i].y, kr[i], part.y);
      part.z = fmaf(s[i].z, kr[i], part.z);
      part.w = fmaf(s[i].w, kr[i], part.w);
    }
    const float4 kv = row_sum(part, 0);
    const float4 d = make_float4((vv[0] - kv.x) * b, (vv[1] - kv.y) * b, (vv[2] - kv.z) * b,
                                 (vv[3] - kv.w) * b);
    float4 po = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      s[i].x = fmaf(kr[i], d.x, s[i].x);
      s[i].y = fmaf(kr[i], d.y, s[i].y);
      s[i].z = fmaf(kr[i], d.z, s[i].z);
      s[i].w = fmaf(kr[i], d.w, s[i].w);
      po.x = fmaf(s[i].x, qr[i], po.x);
      po.y = fmaf(s[i].y, qr[i], po.y);
      po.z = fmaf(s[i].z, qr[i], po.z);
      po.w = fmaf(s[i].w, qr[i], po.w);
    }
    const float4 o = row_sum(po, 1);
    if (wave == 0) {
      // lanes 0..31 cover the 32 column quads (lanes 32..63 repeat them)
      float ss = o.x * o.x + o.y * o.y + o.z * o.z + o.w * o.w;
      ss = sum_xor16(row16_sum(ss));
      const float scale = rsqrtf(ss / static_cast<float>(kDim) + eps);
      if (lane < 32) {
        const std::size_t base = t * hidden + h * kDim + c0;
        const float ov[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) Elem<T>::store(output, base + i, ov[i] * scale * nw[i] * silu(z[i]));
      }
    }
  }
#pragma unroll
  for (int i = 0; i < kRows; ++i) *reinterpret_cast<float4 *>(sh + (r0 + i) * kDim + c0) = s[i];
}

// ------------------------------------------------- stage 2b: chunked
// fp32 MFMA 16x16x4: lane l supplies A[l%16][l/16] and B[l/16][l%16] and
// holds D[(l/16)*4 + r][l%16], r = 0..3.
__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

constexpr int kLd = kChunkDim + 4; // LDS row stride for 128-wide rows
constexpr int kLdC = kChunk + 4;   // LDS row stride for 64-wide rows

// Batched staging of a 64 x 128 block of rows (rows >= L repeat row L-1): thread owns
// rows (tid + 256 r) / 16, dims 8 * ((tid + 256 r) % 16), r = 0..3, so every
// global load of the block is issued before any of them is consumed.
template <typename T> struct RowBlock {
  Chunk8<T> c[4];
  template <typename Addr>
  __device__ __forceinline__ void load(int L, Addr addr) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int p = threadIdx.x + 256 * r;
      const int i = p >> 4, d = 8 * (p & 15);
      // Rows past L load row L-1 (in bounds, finite); every consumer gives
      // them zero weight, and no branch splits the batch of loads.
      c[r].load(addr(i < L ? i : L - 1, d));
    }
  }
  __device__ __forceinline__ void store(float (*dst)[kLd], float scale) const {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int p = threadIdx.x + 256 * r;
      const int i = p >> 4, d = 8 * (p & 15);
      float4 lo, hi;
      lo.x = c[r].get(0) * scale; lo.y = c[r].get(1) * scale; lo.z = c[r].get(2) * scale; lo.w = c[r].get(3) * scale;
      hi.x = c[r].get(4) * scale; hi.y = c[r].get(5) * scale; hi.z = c[r].get(6) * scale; hi.w = c[r].get(7) * scale;
      *reinterpret_cast<float4 *>(&dst[i][d]) = lo;
      *reinterpret_cast<float4 *>(&dst[i][d + 4]) = hi;
    }
  }
};

template <> struct RowBlock<float> {
  float4 c[4][2];
  template <typename Addr>
  __device__ __forceinline__ void load(int L, Addr addr) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int p = threadIdx.x + 256 * r;
      const int i = p >> 4, d = 8 * (p & 15);
      const float *src = addr(i < L ? i : L - 1, d);
      c[r][0] = *reinterpret_cast<const float4 *>(src);
      c[r][1] = *reinterpret_cast<const float4 *>(src + 4);
    }
  }
  __device__ __forceinline__ void store(float (*dst)[kLd], float scale) const {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int p = threadIdx.x + 256 * r;
      const int i = p >> 4, d = 8 * (p & 15);
#pragma unroll
      for (int hpart = 0; hpart < 2; ++hpart) {
        float4 v = c[r][hpart];
        v.x *= scale; v.y *= scale; v.z *= scale; v.w *= scale;
        *reinterpret_cast<float4 *>(&dst[i][d + 4 * hpart]) = v;
      }
    }
  }
};

template <typename T>
__device__ __forceinline__ const T *src_row(const Src<T> &s, std::size_t t, std::size_t head, int d) {
  return s.base + t * s.row + head * s.head_stride + d;
}

// T = (I + A)^-1 for a strictly lower-triangular 64 x 64 A (fp32, LDS), by
// blocks: [[P, 0], [C, Q]]^-1 = [[P^-1, 0], [-Q^-1 C P^-1, Q^-1]].
//   1. wave w inverts the unit lower-triangular diagonal block w (16 x 16) by
//      substitution, lane = column (all four blocks at once);
//   2. waves 0 and 1 form the two 16 x 16 off-diagonal blocks of the 32 x 32
//      diagonal blocks;
//   3. waves 0-3 form the 32 x 32 lower-left block, one 16 x 16 tile each, in
//      two products (3a, 3b).
// Products run on fp32 MFMA 16x16x4; `y` is 32 x 36 fp32 scratch.  Each step
// reads what the previous ones wrote, so a barrier separates them.  T's
// strictly upper part is written as 0.

// Step 1 for diagonal block w, by wave w: zeros rows 16w .. 16w+15 right of
// the block, then lanes 0..15 (lane = column) substitute.  entry(r, j) gives
// A[16w + r][16w + j] for j < r (the same value in every lane).
template <typename Entry>
__device__ __forceinline__ void invert_step1(float (*tm)[kLdC], int w, Entry entry) {
  const int lane = threadIdx.x & 63;
  const int b = 16 * w;
  for (int j = 16 * (w + 1) + lane; j < kChunk; j += 64)
#pragma unroll
    for (int r = 0; r < 16; ++r) tm[b + r][j] = 0.f;
  float x[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) x[r] = r == lane ? 1.f : 0.f;
  // Right-looking: once x[j] is final, the updates of rows j+1.. are
  // independent, so the dependent chain is 15 FMAs long, not 120.
#pragma unroll
  for (int j = 0; j < 15; ++j)
#pragma unroll
    for (int r = j + 1; r < 16; ++r) x[r] = fmaf(-entry(r, j), x[j], x[r]);
  if (lane < 16) {
#pragma unroll
    for (int r = 0; r < 16; ++r) tm[b + r][b + lane] = x[r];
  }
}

// Step 2, block (2p+1, 2p) = -T_qq A_qp T_pp for p = w (waves 0, 1).
__device__ __forceinline__ void invert_step2(const float (*a)[kLdC], float (*tm)[kLdC], float (*y)[36],
                                             int w) {
  const int lane = threadIdx.x & 63, lr = lane & 15, lk = lane >> 4;
  const int P = 32 * w, Q = P + 16;
  floatx4 acc = floatx4{};
#pragma unroll
  for (int k0 = 0; k0 < 16; k0 += 4) acc = mfma4(a[Q + lr][P + k0 + lk], tm[P + k0 + lk][P + lr], acc);
  float(*yw)[36] = y + 16 * w;
#pragma unroll
  for (int r = 0; r < 4; ++r) yw[4 * lk + r][lr] = acc[r];
  wave_lds_order();
  acc = floatx4{};
#pragma unroll
  for (int k0 = 0; k0 < 16; k0 += 4) acc = mfma4(tm[Q + lr][Q + k0 + lk], yw[k0 + lk][lr], acc);
#pragma unroll
  for (int r = 0; r < 4; ++r) tm[Q + 4 * lk + r][P + lr] = -acc[r];
}

// Step 3a (waves 0-3): y tile (ti - 2, tj) = A_BL T_TL, ti = 2 + w / 2, tj = w % 2.
__device__ __forceinline__ void invert_step3a(const float (*a)[kLdC], const float (*tm)[kLdC],
                                              float (*y)[36], int w) {
  const int lane = threadIdx.x & 63, lr = lane & 15, lk = lane >> 4;
  const int ti = 2 + (w >> 1), tj = w & 1;
  // T_TL is lower triangular and its upper right block is stored as 0, so the
  // full k range gives the same sums; the operands are read up front.
  float av[8], bv[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    av[n] = a[16 * ti + lr][4 * n + lk];
    bv[n] = tm[4 * n + lk][16 * tj + lr];
  }
  floatx4 acc = floatx4{};
#pragma unroll
  for (int n = 0; n < 8; ++n) acc = mfma4(av[n], bv[n], acc);
#pragma unroll
  for (int r = 0; r < 4; ++r) y[16 * (ti - 2) + 4 * lk + r][16 * tj + lr] = acc[r];
}

// Step 3b (waves 0-3): T tile (ti, tj) = -T_BR y.
__device__ __forceinline__ void invert_step3b(float (*tm)[kLdC], const float (*y)[36], int w) {
  const int lane = threadIdx.x & 63, lr = lane & 15, lk = lane >> 4;
  const int ti = 2 + (w >> 1), tj = w & 1;
  // T_BR is lower triangular with its upper right block stored as 0.
  float av[8], bv[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    av[n] = tm[16 * ti + lr][32 + 4 * n + lk];
    bv[n] = y[4 * n + lk][16 * tj + lr];
  }
  floatx4 acc = floatx4{};
#pragma unroll
  for (int n = 0; n < 8; ++n) acc = mfma4(av[n], bv[n], acc);
#pragma unroll
  for (int r = 0; r < 4; ++r) tm[16 * ti + 4 * lk + r][16 * tj + lr] = -acc[r];
}

// Steps 2 and 3 with their barriers (every wave of the workgroup takes them;
// waves 0-3 do the work), after step 1 and a barrier.  Ends with a barrier.
__device__ __forceinline__ void invert_steps23(const float (*a)[kLdC], float (*tm)[kLdC], float (*y)[36]) {
  const int wave = threadIdx.x >> 6;
  if (wave < 2) invert_step2(a, tm, y, wave);
  __syncthreads();
  if (wave < 4) invert_step3a(a, tm, y, wave);
  __syncthreads();
  if (wave < 4) invert_step3b(tm, y, wave);
  __syncthreads();
}

// All four steps, A read from LDS.  Ends with a barrier.
__device__ __forceinline__ void invert_unit_lower_64(const float (*a)[kLdC], float (*tm)[kLdC],
                                                     float (*y)[36]) {
  const int wave = threadIdx.x >> 6;
  if (wave < 4) {
    const int b = 16 * wave;
    invert_step1(tm, wave, [&](int r, int j) { return a[b + r][b + j]; });
  }
  __syncthreads();
  invert_steps23(a, tm, y);
}

struct PrepShared {
  float k[kChunk][kLd];   // K * k_scale; later W
  float qv[kChunk][kLd];  // Q * q_scale, then V; later U
  float a[kChunk][kLdC];  // A
  float tm[kChunk][kLdC]; // T = (I + A)^-1
  float mm[kChunk][kLdC]; // M
  float y[32][36];        // inverse scratch
  float g[kChunk];
  float beta[kChunk];
};

// Inclusive prefix sum over the 64 lanes of a wave: shifts within 16-lane
// rows, then the row totals carried across rows, all on DPP (no LDS trip).
__device__ __forceinline__ float wave_prefix_sum(float x) {
  auto shr = [](float v, auto ctrl_tag) {
    constexpr int kCtrl = decltype(ctrl_tag)::value;
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xf, 0xf, false));
  };
  x += shr(x, std::integral_constant<int, 0x111>{}); // row_shr:1
  x += shr(x, std::integral_constant<int, 0x112>{}); // row_shr:2
  x += shr(x, std::integral_constant<int, 0x114>{}); // row_shr:4
  x += shr(x, std::integral_constant<int, 0x118>{}); // row_shr:8
  // row_bcast:15 adds lane 15 of row r to every lane of row r + 1 (rows 1, 3);
  // row_bcast:31 adds lane 31 to every lane of rows 2 and 3.
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x142, 0xa, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x143, 0xc, 0xf, false));
  return x;
}


// Writes a [rows][cols] fp32 LDS tile (row stride LD) to a record as split
// bf16 [2][rows][cols], 8 elements (two 16-byte stores) per item.
template <int LD, int NT = 256>
__device__ __forceinline__ void write_split_rows(const float (*src)[LD], int rows, int cols,
                                                 bf16_bits *dst) {
  const int per_row = cols / 8;
  for (int item = threadIdx.x; item < rows * per_row; item += NT) {
    const int r = item / per_row, c = 8 * (item % per_row);
    u32x4 hi, lo;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      std::uint32_t h, l;
      split2(src[r][c + 2 * e], src[r][c + 2 * e + 1], h, l);
      hi[e] = h;
      lo[e] = l;
    }
    *reinterpret_cast<u32x4 *>(dst + r * cols + c) = hi;
    *reinterpret_cast<u32x4 *>(dst + rows * cols + r * cols + c) = lo;
  }
}

// Per (value head, chunk), in parallel over chunks: the UT/WY quantities of
// the chunk, written as one record (see rec::).
template <typename InT>
__global__ __launch_bounds__(256) void chunk_prep_kernel(Src<InT> qs, Src<InT> ks, Src<InT> vs,
                                                         const float *__restrict__ beta,
                                                         const float *__restrict__ gdecay,
                                                         ChunkScratch scratch, std::size_t tokens,
                                                         std::size_t hk, std::size_t hv) {
  __shared__ PrepShared sh;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, lk = lane >> 4;
  const std::size_t h = blockIdx.x;
  const std::size_t kh = h % hk;
  const std::size_t t0 = static_cast<std::size_t>(blockIdx.y) * kChunk;
  const int L = static_cast<int>(tokens - t0 < kChunk ? tokens - t0 : kChunk);
  unsigned char *record = scratch.at(h, blockIdx.y);

  RowBlock<InT> kb, qb;
  kb.load(L, [&](int i, int d) { return src_row(ks, t0 + i, kh, d); });
  qb.load(L, [&](int i, int d) { return src_row(qs, t0 + i, kh, d); });
  float bt = 0.f, gt = 0.f;
  if (tid < L) {
    bt = beta[(t0 + tid) * hv + h];
    gt = gdecay[(t0 + tid) * hv + h];
  }
  kb.store(sh.k, ks.scale);
  qb.store(sh.qv, qs.scale);
  RowBlock<InT> vb; // issued now, consumed after the Q-dependent products
  vb.load(L, [&](int i, int d) { return src_row(vs, t0 + i, h, d); });
  if (tid < kChunk) {
    sh.beta[tid] = bt;
    sh.g[tid] = gt;
  }
  __syncthreads();
  if (wave == 0) sh.g[lane] = wave_prefix_sum(sh.g[lane]); // rows past L repeat G[L-1] (g = 0)
  __syncthreads();

  // M = e^{G_i-G_j} (q_i . k_j), j <= i, and A = beta_i e^{G_i-G_j} (k_i . k_j),
  // j < i, on fp32 MFMA 16x16x4; wave w = row tile w.  The per-row G and
  // beta are read once, before the products, and every entry is formed
  // unconditionally and masked by a multiply (a select would put its LDS
  // reads behind a branch each).
  float gi[4], bi[4], mi[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = wave * 16 + lk * 4 + r;
    gi[r] = sh.g[i];
    bi[r] = sh.beta[i];
    mi[r] = i < L ? 1.f : 0.f;
  }
  for (int tj = 0; tj < 4; ++tj) {
    floatx4 am = floatx4{}, aa = floatx4{};
    if (tj <= wave) {
#pragma unroll 8
      for (int k0 = 0; k0 < kChunkDim; k0 += 4) {
        const float kj = sh.k[tj * 16 + lr][k0 + lk];
        am = mfma4(sh.qv[wave * 16 + lr][k0 + lk], kj, am);
        aa = mfma4(sh.k[wave * 16 + lr][k0 + lk], kj, aa);
      }
    }
    const int j = tj * 16 + lr;
    const float gj = sh.g[j];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = wave * 16 + lk * 4 + r;
      // Only j <= i is kept; clamping keeps e^{G_i-G_j} finite above the
      // diagonal (G_i > G_j there) so the masking multiply gives 0, not NaN.
      const float e = __expf(fminf(gi[r] - gj, 0.f)) * mi[r];
      sh.mm[i][j] = (j <= i ? 1.f : 0.f) * (am[r] * e);
      sh.a[i][j] = (j < i ? 1.f : 0.f) * (bi[r] * e * aa[r]);
    }
  }
  // Q and K^T go to the record before Q's LDS is reused, as
  // (Q * q_scale, (K * k_scale)^T) split pairs.
  write_split_rows<kLd>(sh.qv, kChunk, kChunkDim, reinterpret_cast<bf16_bits *>(record + rec::kQ));
  {
    bf16_bits *kt = reinterpret_cast<bf16_bits *>(record + rec::kKt);
    for (int item = tid; item < kChunkDim * (kChunk / 2); item += 256) {
      const int d = item / (kChunk / 2), j = 2 * (item % (kChunk / 2));
      std::uint32_t hi, lo;
      split2(sh.k[j][d], sh.k[j + 1][d], hi, lo);
      *reinterpret_cast<std::uint32_t *>(kt + d * kChunk + j) = hi;
      *reinterpret_cast<std::uint32_t *>(kt + kChunkDim * kChunk + d * kChunk + j) = lo;
    }
  }
  __syncthreads();
  vb.store(sh.qv, vs.scale); // Q no longer needed: stage V.
  invert_unit_lower_64(sh.a, sh.tm, sh.y);
  // W = T diag(beta e^G) K, U = T diag(beta) V: 4 x 8 output tiles, wave w
  // takes tiles w, w+4, ...; staged through LDS (over K and V) for the
  // row-contiguous record writes.
  floatx4 aw[8], au[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    const int tile = wave + 4 * n;
    const int ti = tile >> 3, tn = tile & 7;
    aw[n] = floatx4{};
    au[n] = floatx4{};
#pragma unroll 4
    for (int j0 = 0; j0 < kChunk; j0 += 4) {
      const int j = j0 + lk;
      const float tmv = sh.tm[ti * 16 + lr][j];
      const float bj = sh.beta[j];
      aw[n] = mfma4(tmv * bj * __expf(sh.g[j]), sh.k[j][tn * 16 + lr], aw[n]);
      au[n] = mfma4(tmv * bj, sh.qv[j][tn * 16 + lr], au[n]);
    }
  }
  __syncthreads(); // K and V reads done
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    const int tile = wave + 4 * n;
    const int ti = tile >> 3, tn = tile & 7;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sh.k[ti * 16 + lk * 4 + r][tn * 16 + lr] = aw[n][r];
      sh.qv[ti * 16 + lk * 4 + r][tn * 16 + lr] = au[n][r];
    }
  }
  __syncthreads();
  write_split_rows<kLd>(sh.k, kChunk, kChunkDim, reinterpret_cast<bf16_bits *>(record + rec::kW));
  write_split_rows<kLdC>(sh.mm, kChunk, kChunk, reinterpret_cast<bf16_bits *>(record + rec::kM));
  {
    float *u = reinterpret_cast<float *>(record + rec::kU);
    for (int item = tid; item < kChunk * (kChunkDim / 4); item += 256) {
      const int r = item / (kChunkDim / 4), c = 4 * (item % (kChunkDim / 4));
      *reinterpret_cast<float4 *>(u + r * kChunkDim + c) =
          make_float4(sh.qv[r][c], sh.qv[r][c + 1], sh.qv[r][c + 2], sh.qv[r][c + 3]);
    }
  }
  if (tid < kChunk) reinterpret_cast<float *>(record + rec::kG)[tid] = sh.g[tid];
}

__device__ __forceinline__ bf16x8 lds8(const bf16_bits *p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(p));
}

// Chunk scan on bf16 MFMA with fp32-accurate products.  The records hold
// every fp32 operand x split as x = xh + xl, and a product of two split
// operands is taken as ah*bh + ah*bl + al*bh (the dropped al*bl is below
// 2^-16 of it), each term one v_mfma_f32_16x16x32_bf16 with fp32
// accumulation.  The fp32 state of the block's 16 columns stays in VGPRs
// across chunks; LDS holds its split transpose as the B operand.
//
// MFMA 16x16x32 bf16: lane l supplies A[l%16][8*(l/16) .. +7] and
// B[8*(l/16) .. +7][l%16], and holds C[4*(l/16) + r][l%16], r = 0..3, so A is
// read from a row-major [m][k] tile and B from a transposed [n][k] tile, one
// 16-byte LDS read each.
constexpr int kLdK = kChunkDim + 8; // bf16 row stride for 128-long k
constexpr int kLdJ = kChunk + 8;    // bf16 row stride for 64-long k

// Chunk operands W, Q, M (rows i) and K^T (rows d) are loaded from the chunk
// record straight into LDS (global_load_lds_dwordx4) in unpadded rows whose
// 16-byte chunks are XOR-swizzled by row, so the MFMA operand reads (16
// rows x one chunk per lane group) hit distinct banks: 128-wide rows (16
// chunks) use chunk ^ (row & 15), 64-wide rows (8 chunks, two rows per bank
// window) chunk ^ ((row >> 1) & 7).  Every wave reads only its own rows of
// these four blocks (W, Q, M rows 16w.., K^T rows 32w..), so each wave loads
// its own rows and waits for them alone.
struct Scan3Shared {
  bf16_bits w[2][kChunk][kChunkDim];   // W (hi, lo), [i][d]
  bf16_bits q[2][kChunk][kChunkDim];   // Q (hi, lo), [i][d]
  bf16_bits kt[2][kChunkDim][kChunk];  // K^T (hi, lo), [d][j]
  bf16_bits m[2][kChunk][kChunk];      // M (hi, lo), [i][j]
  bf16_bits st[2][kColBlock][kLdK];    // S^T (hi, lo), [c][d]
  bf16_bits dt[2][kColBlock][kLdJ];    // D^T (hi, lo), [c][i]
  bf16_bits ft[2][kColBlock][kLdJ];    // (e^{G_last-G} D)^T (hi, lo), [c][j]
  float u[kChunk][kColBlock];          // U[i][c0 ..], this block's columns
  float g[2][kChunk];                  // cumulative log decay G, by chunk parity
};
// Element offset of logical 16-byte chunk c in row r of a swizzled block.
__device__ __forceinline__ int swz128(int r, int c) { return r * kChunkDim + ((c ^ (r & 15)) << 3); }
__device__ __forceinline__ int swz64(int r, int c) { return r * kChunk + ((c ^ ((r >> 1) & 7)) << 3); }

// LDS-direct load of rows row0 .. row0+ROWS-1 of halves 0 .. HALVES-1 of a
// bf16 [2][R][C] record block at byte offset `off` into its swizzled LDS copy
// `dst` (same shape).  One instruction moves 1 KiB = 1024 / (2 C) rows; lane
// i fills physical chunk i % (C / 8) of its row with the logical chunk that
// the swizzle puts there.  row0 is wave-uniform.
template <int R, int C, int ROWS, int HALVES>
__device__ __forceinline__ void load_rows_lds(const unsigned char *record, std::uint32_t off,
                                              bf16_bits (*dst)[R][C], int row0) {
  constexpr int kCpr = C / 8, kRpi = 64 / kCpr;
  const int lane = threadIdx.x & 63;
  const int rr = lane / kCpr, p = lane % kCpr;
#pragma unroll
  for (int hl = 0; hl < HALVES; ++hl)
#pragma unroll
    for (int j = 0; j < ROWS / kRpi; ++j) {
      const int row = row0 + j * kRpi + rr;
      const int logical = C == kChunkDim ? p ^ (row & 15) : p ^ ((row >> 1) & 7);
      load_lds_b128(record, off + static_cast<std::uint32_t>(((hl * R + row) * C + logical * 8) * 2),
                    lds_address(&dst[hl][row0 + j * kRpi][0]));
    }
}

// Writes a C-layout 16x16 fp32 tile transposed and split: lane holds rows
// 4*(lane/16) + r of column lane%16, stored at dst[col][row0 + 4*(lane/16) ..].
template <int LD>
__device__ __forceinline__ void store_split_t(bf16_bits (*hi)[LD], bf16_bits (*lo)[LD], int row0,
                                              floatx4 v) {
  const int lane = threadIdx.x & 63;
  std::uint32_t h0, l0, h1, l1;
  split2(v[0], v[1], h0, l0);
  split2(v[2], v[3], h1, l1);
  const int c = lane & 15, rr = row0 + 4 * (lane >> 4);
  *reinterpret_cast<u32x2 *>(&hi[c][rr]) = u32x2{h0, h1};
  *reinterpret_cast<u32x2 *>(&lo[c][rr]) = u32x2{l0, l1};
}

// Loads of chunk record `record`, in the order the scan consumes them, each
// wave fetching only the rows it reads.  The first part (W, U, G) has
// kFirstLoads instructions per wave, K^T kKtLoads, Q and M kQmLoads.
struct ScanLoads {
  static constexpr int kQkHalves = 2;
  static constexpr int kFirstLoads = 8 + 1 + 1;
  static constexpr int kKtLoads = 4 * kQkHalves;
  static constexpr int kQmLoads = 4 * kQkHalves + 4;
  __device__ static void first(Scan3Shared &sh, const unsigned char *record, int wave, int c0,
                               int parity) {
    load_rows_lds<kChunk, kChunkDim, 16, 2>(record, rec::kW, sh.w, 16 * wave);
    const int lane = threadIdx.x & 63;
    // U rows 16 wave + lane / 4, 16-byte piece lane % 4 of columns c0 ..
    load_lds_b128(record,
                  static_cast<std::uint32_t>(rec::kU + ((16 * wave + (lane >> 2)) * kChunkDim + c0) * 4 +
                                             (lane & 3) * 16),
                  lds_address(&sh.u[16 * wave][0]));
    // G[16 wave .. +15]: lanes 0..3 only (every wave issues the instruction).
    if (lane < 4)
      load_lds_b128(record, static_cast<std::uint32_t>(rec::kG + (16 * wave + 4 * lane) * 4),
                    lds_address(&sh.g[parity][16 * wave]));
  }
  __device__ static void kt(Scan3Shared &sh, const unsigned char *record, int wave) {
    load_rows_lds<kChunkDim, kChunk, 32, kQkHalves>(record, rec::kKt, sh.kt, 32 * wave);
  }
  __device__ static void qm(Scan3Shared &sh, const unsigned char *record, int wave) {
    load_rows_lds<kChunk, kChunkDim, 16, kQkHalves>(record, rec::kQ, sh.q, 16 * wave);
    load_rows_lds<kChunk, kChunk, 16, 2>(record, rec::kM, sh.m, 16 * wave);
  }
};

// Block (value head, 16-column block), sequential over chunks.  Wave w owns
// rows 16w.. of D and O and state rows 32w.. (two 16-row tiles) of S.  The
// next chunk's record streams into LDS behind the current chunk's work: each
// part is reissued as soon as its wave has finished reading the current one
// (W, U, G after D; K^T after the S update; Q, M after O).
template <typename OutT>
__global__ __launch_bounds__(256) void chunk_scan_kernel(ChunkScratch scratch,
                                                         float *__restrict__ state,
                                                         OutT *__restrict__ out, std::size_t tokens,
                                                         std::size_t hv) {
  using Loads = ScanLoads;
  __shared__ Scan3Shared sh;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lk = lane >> 4;
  const std::size_t h = blockIdx.x;
  const int c0 = blockIdx.y * kColBlock;
  float *sg = state + h * kChunkDim * kChunkDim;
  {
    const unsigned char *first = scratch.at(h, 0);
    Loads::first(sh, first, wave, c0, 0);
    Loads::kt(sh, first, wave);
    Loads::qm(sh, first, wave);
  }
  // fp32 state tiles: s[tt] holds S[32 wave + 16 tt + 4 lk + r][c0 + lr].
  floatx4 s[2];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int r = 0; r < 4; ++r) s[tt][r] = sg[(32 * wave + 16 * tt + 4 * lk + r) * kChunkDim + c0 + lr];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) store_split_t<kLdK>(sh.st[0], sh.st[1], 32 * wave + 16 * tt, s[tt]);

  const bf16_bits *w_hi = &sh.w[0][0][0], *w_lo = &sh.w[1][0][0];
  const bf16_bits *q_hi = &sh.q[0][0][0], *q_lo = &sh.q[1][0][0];
  const bf16_bits *kt_hi = &sh.kt[0][0][0], *kt_lo = &sh.kt[1][0][0];
  const bf16_bits *m_hi = &sh.m[0][0][0], *m_lo = &sh.m[1][0][0];
  const int i0 = 16 * wave;
  for (std::size_t c = 0, t0 = 0; t0 < tokens; ++c, t0 += kChunk) {
    const int L = static_cast<int>(tokens - t0 < kChunk ? tokens - t0 : kChunk);
    const int parity = static_cast<int>(c & 1);
    const bool more = t0 + kChunk < tokens;
    const unsigned char *next = scratch.at(h, more ? c + 1 : c);
    wait_vm<Loads::kQmLoads>(); // this chunk's W, U, G and K^T (Q, M may be in flight)
    __syncthreads();            // G of every wave and S^T in LDS
    const float *g = sh.g[parity];
    const float glast = g[kChunk - 1]; // = G[L-1] (padded)
    // Per-row factors of this lane's rows i = i0 + 4 lk + r, computed before
    // the products so the exponentials overlap the MFMA latency:
    // e^{G_last - G_i} for D~ (0 past L) and e^{G_i} for O.
    floatx4 u, fdec, eq;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = i0 + 4 * lk + r;
      const float gi = g[i];
      u[r] = sh.u[i][lr];
      fdec[r] = i < L ? __expf(glast - gi) : 0.f;
      eq[r] = __expf(gi);
    }
    // D = U - W S for rows i0 .. i0+15 (S^T is the B operand), and
    // D~ = e^{G_last - G} D for the S update (rows past L get weight 0).
    // Operands are read before any product, and the three hi/lo products
    // accumulate separately (chains of 4 MFMAs instead of 12).
    {
      bf16x8 wh[4], wl[4], sth[4], stl[4];
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const int ka = 32 * n + 8 * lk, wa = swz128(i0 + lr, 4 * n + lk);
        wh[n] = lds8(w_hi + wa);
        wl[n] = lds8(w_lo + wa);
        sth[n] = lds8(&sh.st[0][lr][ka]);
        stl[n] = lds8(&sh.st[1][lr][ka]);
      }
      floatx4 a0 = floatx4{}, a1 = floatx4{}, a2 = floatx4{};
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        a0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wh[n], sth[n], a0, 0, 0, 0);
        a1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wh[n], stl[n], a1, 0, 0, 0);
        a2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wl[n], sth[n], a2, 0, 0, 0);
      }
      floatx4 acc;
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = a0[r] + (a1[r] + a2[r]);
      floatx4 dv, fv;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        dv[r] = u[r] - acc[r];
        fv[r] = fdec[r] * dv[r];
      }
      store_split_t<kLdJ>(sh.dt[0], sh.dt[1], i0, dv);
      store_split_t<kLdJ>(sh.ft[0], sh.ft[1], i0, fv);
    }
    wait_lgkm0(); // this wave's reads of W and U are done
    if (more) Loads::first(sh, next, wave, c0, parity ^ 1);
    __syncthreads(); // D^T and D~^T of every row tile written
    // S'[d][c] = e^{G_last} S[d][c] + sum_j K[j][d] D~[j][c], rows 32 wave + 16 tt
    // (registers only: S^T in LDS keeps the old state for O).
    const float egl = __expf(glast);
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int d0 = 32 * wave + 16 * tt;
      bf16x8 kh[2], kl[2], fh[2], fl[2];
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        const int ja = 32 * n + 8 * lk, ka = swz64(d0 + lr, 4 * n + lk);
        kh[n] = lds8(kt_hi + ka);
        kl[n] = lds8(kt_lo + ka);
        fh[n] = lds8(&sh.ft[0][lr][ja]);
        fl[n] = lds8(&sh.ft[1][lr][ja]);
      }
      floatx4 s0 = floatx4{}, s1 = floatx4{}, s2 = floatx4{};
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh[n], fh[n], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh[n], fl[n], s1, 0, 0, 0);
        s2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kl[n], fh[n], s2, 0, 0, 0);
      }
      floatx4 acc;
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = s0[r] + (s1[r] + s2[r]);
#pragma unroll
      for (int r = 0; r < 4; ++r) s[tt][r] = fmaf(egl, s[tt][r], acc[r]);
    }
    wait_lgkm0(); // this wave's reads of K^T are done
    if (more) {
      Loads::kt(sh, next, wave);
      wait_vm<Loads::kFirstLoads + Loads::kKtLoads>(); // this chunk's Q and M
    } else {
      wait_vm<0>();
    }
    // O = e^G (Q S) + M D for rows i0 .. i0+15.
    {
      bf16x8 qh[4], ql[4], sth[4], stl[4], mh[2], ml[2], dth[2], dtl[2];
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const int ka = 32 * n + 8 * lk, qo = swz128(i0 + lr, 4 * n + lk);
        qh[n] = lds8(q_hi + qo);
        ql[n] = lds8(q_lo + qo);
        sth[n] = lds8(&sh.st[0][lr][ka]);
        stl[n] = lds8(&sh.st[1][lr][ka]);
      }
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        const int ja = 32 * n + 8 * lk, mo = swz64(i0 + lr, 4 * n + lk);
        mh[n] = lds8(m_hi + mo);
        ml[n] = lds8(m_lo + mo);
        dth[n] = lds8(&sh.dt[0][lr][ja]);
        dtl[n] = lds8(&sh.dt[1][lr][ja]);
      }
      floatx4 q0 = floatx4{}, q1 = floatx4{}, q2 = floatx4{}, m0 = floatx4{}, m1 = floatx4{}, m2 = floatx4{};
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        q0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qh[n], sth[n], q0, 0, 0, 0);
        q1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qh[n], stl[n], q1, 0, 0, 0);
        q2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ql[n], sth[n], q2, 0, 0, 0);
      }
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        m0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mh[n], dth[n], m0, 0, 0, 0);
        m1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mh[n], dtl[n], m1, 0, 0, 0);
        m2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ml[n], dth[n], m2, 0, 0, 0);
      }
      floatx4 qa, ma;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        qa[r] = q0[r] + (q1[r] + q2[r]);
        ma[r] = m0[r] + (m1[r] + m2[r]);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = i0 + 4 * lk + r;
        if (i < L)
          Elem<OutT>::store(out, ((t0 + i) * hv + h) * kChunkDim + c0 + lr, fmaf(eq[r], qa[r], ma[r]));
      }
    }
    wait_lgkm0(); // this wave's reads of Q and M are done
    if (more) Loads::qm(sh, next, wave);
    __syncthreads(); // every wave is done reading S^T, D^T and D~^T
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) store_split_t<kLdK>(sh.st[0], sh.st[1], 32 * wave + 16 * tt, s[tt]);
  }
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int r = 0; r < 4; ++r) sg[(32 * wave + 16 * tt + 4 * lk + r) * kChunkDim + c0 + lr] = s[tt][r];
}

// ------------------------------------- stage 2b, bf16 inputs: T records
// With q, k and v exact in bf16 the scan takes Q, K and V straight from the
// inputs, and the per-chunk record holds only Tb = T diag(beta), M and G
// (33 KB instead of the 148 KB W/U/Q/K^T/M record): the chunk update is
// regrouped as
//   D = U - W S = Tb (v_scale V - diag(e^G) k_scale K S).

// Per (value head, chunk): A = beta_i e^{G_i-G_j} k_i.k_j (j < i) and
// M = q_scale k_scale e^{G_i-G_j} q_i.k_j (j <= i) on exact bf16 MFMA,
// T = (I + A)^-1, and the record (Tb split, M split, G).
// kSplit: q and k arrive as (hi, lo) bf16 planes (fp32 values split), and
// each product is formed as hi*hi + hi*lo + lo*hi.
template <bool kSplit> struct TbShared {
  bf16_bits k[kSplit ? 2 : 1][kChunk][kChunkDim + 8];
  bf16_bits q[kSplit ? 2 : 1][kChunk][kChunkDim + 8];
  float a[kChunk][kLdC];
  float tm[kChunk][kLdC];
  float mm[kChunk][kLdC];
  float y[32][36];
  float g[kChunk];
  float beta[kChunk];
};

// Writes a [64][64] fp32 LDS tile (times the per-column factor col[j] when
// kCol) to a record as split bf16 [2][64][64]: thread -> row tid / 4,
// columns 16 (tid % 4) .. +15.  All LDS reads go out before the first use.
template <bool kCol>
__device__ __forceinline__ void write_split_64(const float (*src)[kLdC], const float *col, bf16_bits *dst) {
  const int i = threadIdx.x >> 2, j0 = 16 * (threadIdx.x & 3);
  float v[16];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float4 x = *reinterpret_cast<const float4 *>(&src[i][j0 + 4 * e]);
    v[4 * e] = x.x;
    v[4 * e + 1] = x.y;
    v[4 * e + 2] = x.z;
    v[4 * e + 3] = x.w;
  }
  if constexpr (kCol) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float4 c = *reinterpret_cast<const float4 *>(&col[j0 + 4 * e]);
      v[4 * e] *= c.x;
      v[4 * e + 1] *= c.y;
      v[4 * e + 2] *= c.z;
      v[4 * e + 3] *= c.w;
    }
  }
  u32x4 hi[2], lo[2];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    std::uint32_t hw, lw;
    split2(v[2 * e], v[2 * e + 1], hw, lw);
    hi[e >> 2][e & 3] = hw;
    lo[e >> 2][e & 3] = lw;
  }
  bf16_bits *row = dst + i * kChunk + j0;
  reinterpret_cast<u32x4 *>(row)[0] = hi[0];
  reinterpret_cast<u32x4 *>(row)[1] = hi[1];
  reinterpret_cast<u32x4 *>(row + kChunk * kChunk)[0] = lo[0];
  reinterpret_cast<u32x4 *>(row + kChunk * kChunk)[1] = lo[1];
}

template <bool kSplit>
__global__ __launch_bounds__(256) void chunk_tb_kernel(Src<bf16_bits> qs, Src<bf16_bits> ks, std::size_t lo_plane,
                                                       const float *__restrict__ beta,
                                                       const float *__restrict__ gdecay,
                                                       ChunkScratch scratch, std::size_t tokens,
                                                       std::size_t hk, std::size_t hv) {
  constexpr int kHalves = kSplit ? 2 : 1;
  __shared__ TbShared<kSplit> sh;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, lk = lane >> 4;
  const std::size_t h = blockIdx.x;
  const std::size_t kh = h % hk;
  const std::size_t t0 = static_cast<std::size_t>(blockIdx.y) * kChunk;
  const int L = static_cast<int>(tokens - t0 < kChunk ? tokens - t0 : kChunk);
  unsigned char *record = scratch.at(h, blockIdx.y);

  // K and Q rows (each plane): item tid + 256 r -> row item / 16, dims
  // 8 (item % 16) .. +7; rows past L repeat row L-1.
  u32x4 kv[kHalves][4], qv[kHalves][4];
#pragma unroll
  for (int hl = 0; hl < kHalves; ++hl)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int p = tid + 256 * r, i = p >> 4, d = 8 * (p & 15);
      const std::size_t t = t0 + (i < L ? i : L - 1);
      kv[hl][r] = *reinterpret_cast<const u32x4 *>(src_row(ks, t, kh, d) + hl * lo_plane);
      qv[hl][r] = *reinterpret_cast<const u32x4 *>(src_row(qs, t, kh, d) + hl * lo_plane);
    }
  float bt = 0.f, gt = 0.f;
  if (tid < L) {
    bt = beta[(t0 + tid) * hv + h];
    gt = gdecay[(t0 + tid) * hv + h];
  }
#pragma unroll
  for (int hl = 0; hl < kHalves; ++hl)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int p = tid + 256 * r, i = p >> 4, d = 8 * (p & 15);
      *reinterpret_cast<u32x4 *>(&sh.k[hl][i][d]) = kv[hl][r];
      *reinterpret_cast<u32x4 *>(&sh.q[hl][i][d]) = qv[hl][r];
    }
  if (tid < kChunk) {
    sh.beta[tid] = bt;
    sh.g[tid] = gt;
  }
  __syncthreads();
  if (wave == 0) sh.g[lane] = wave_prefix_sum(sh.g[lane]); // rows past L repeat G[L-1] (g = 0)
  __syncthreads();
  // A and M: wave w takes row tile w and column tiles 0 .. w (tiles right of
  // the diagonal are 0).
  {
    const float kk_scale = ks.scale * ks.scale, qk_scale = qs.scale * ks.scale;
    float gi[4], bi[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      gi[r] = sh.g[16 * wave + 4 * lk + r];
      bi[r] = sh.beta[16 * wave + 4 * lk + r] * kk_scale;
    }
    bf16x8 krow[kHalves][4], qrow[kHalves][4];
#pragma unroll
    for (int hl = 0; hl < kHalves; ++hl)
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        krow[hl][n] = lds8(&sh.k[hl][16 * wave + lr][32 * n + 8 * lk]);
        qrow[hl][n] = lds8(&sh.q[hl][16 * wave + lr][32 * n + 8 * lk]);
      }
    floatx4 diag = floatx4{}; // this lane's part of A's diagonal tile (w, w)
    for (int tj = 0; tj < 4; ++tj) {
      const int j = 16 * tj + lr;
      if (tj > wave) {
#pragma unroll
        for (int r = 0; r < 4; ++r) sh.mm[16 * wave + 4 * lk + r][j] = 0.f;
        continue;
      }
      bf16x8 kcol[kHalves][4];
#pragma unroll
      for (int hl = 0; hl < kHalves; ++hl)
#pragma unroll
        for (int n = 0; n < 4; ++n) kcol[hl][n] = lds8(&sh.k[hl][16 * tj + lr][32 * n + 8 * lk]);
      floatx4 aa = floatx4{}, am = floatx4{};
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        aa = __builtin_amdgcn_mfma_f32_16x16x32_bf16(krow[0][n], kcol[0][n], aa, 0, 0, 0);
        am = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qrow[0][n], kcol[0][n], am, 0, 0, 0);
      }
      if constexpr (kSplit) {
        // hi*lo and lo*hi terms (lo*lo is below 2^-16 of the product).
        floatx4 aa2 = floatx4{}, am2 = floatx4{};
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          aa2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(krow[0][n], kcol[kHalves - 1][n], aa2, 0, 0, 0);
          am2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qrow[0][n], kcol[kHalves - 1][n], am2, 0, 0, 0);
          aa2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(krow[kHalves - 1][n], kcol[0][n], aa2, 0, 0, 0);
          am2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qrow[kHalves - 1][n], kcol[0][n], am2, 0, 0, 0);
        }
        aa += aa2;
        am += am2;
      }
      const float gj = sh.g[j];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * wave + 4 * lk + r;
        const float e = __expf(gi[r] - gj);
        const float av = (j < i && i < L) ? bi[r] * e * aa[r] : 0.f;
        sh.a[i][j] = av;
        if (tj == wave) diag[r] = av;
        sh.mm[i][j] = (j <= i && i < L) ? qk_scale * e * am[r] : 0.f;
      }
    }
    // Step 1 of the inverse straight from the registers: A[16w + r][16w + j]
    // is element r % 4 of lane 16 (r / 4) + j.
    invert_step1(sh.tm, wave, [&](int r, int j) {
      return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(diag[r & 3]), 16 * (r >> 2) + j));
    });
  }
  __syncthreads();
  // M and G are final here: their record stores drain during the inverse.
  write_split_64<false>(sh.mm, nullptr, reinterpret_cast<bf16_bits *>(record + rec2::kM));
  if (tid < kChunk) reinterpret_cast<float *>(record + rec2::kG)[tid] = sh.g[tid];
  invert_steps23(sh.a, sh.tm, sh.y);
  write_split_64<true>(sh.tm, sh.beta, reinterpret_cast<bf16_bits *>(record + rec2::kTb));
}

// Operands of one chunk, staged in LDS by LDS-direct loads.  Q and K rows use
// the 128-wide swizzle (16-byte chunk c of row r at c ^ (r & 15)), Tb and M
// the 64-wide one (c ^ ((r >> 1) & 7)).
struct TScanBuf {
  bf16_bits q[kChunk][kChunkDim];
  bf16_bits k[kChunk][kChunkDim];
  bf16_bits tb[2][kChunk][kChunk];
  bf16_bits m[2][kChunk][kChunk];
  bf16_bits v[kChunk][kColBlock]; // V[i][c0 ..]
  float g[kChunk];
};

struct TScanShared {
  TScanBuf buf[2];                  // chunk c in buf[c & 1]
  bf16_bits st[2][kColBlock][kLdK]; // S^T (hi, lo), [c][d]
  bf16_bits yt[2][kColBlock][kLdJ]; // (v_scale V - e^G k_scale K S)^T (hi, lo), [c][j]
  bf16_bits dt[2][kColBlock][kLdJ]; // D^T (hi, lo)
  bf16_bits ft[2][kColBlock][kLdJ]; // (e^{G_last-G} D)^T (hi, lo)
  float qo[kChunk][kColBlock];      // e^G q_scale Q S, from waves 0-3 to waves 4-7
};

constexpr int kTScanThreads = 512;

typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4v;
// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element i % 4
// of the 8 bytes that lanes 4 e + i / 4 (e = 0..3) address.
__device__ __forceinline__ u32x2 lds_tr16_b64(const bf16_bits *p) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v *)(p)));
}

// Issues the LDS-direct loads of chunk t0 (L tokens) into `b` from loader
// wave u = 0..3: Q and K rows 16u .. 16u+15, half u / 2 of Tb and M (rows
// 32 (u % 2) .. +31); loaders 0 and 1 load V rows 32u .. +31 (this block's 16
// columns), loader 2 loads G.  Rows past L repeat row L-1.
__device__ __forceinline__ void tscan_issue(TScanBuf &b, const Src<bf16_bits> &qs, const Src<bf16_bits> &ks,
                                            const Src<bf16_bits> &vs, const unsigned char *record,
                                            std::size_t t0, int L, std::size_t h, std::size_t kh, int c0,
                                            int u) {
  const int lane = threadIdx.x & 63;
  const bf16_bits *qb = qs.base + t0 * qs.row + kh * qs.head_stride;
  const bf16_bits *kb = ks.base + t0 * ks.row + kh * ks.head_stride;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row0 = 16 * u + 4 * j, row = row0 + (lane >> 4), p = lane & 15;
    const int src = row < L ? row : L - 1;
    const std::uint32_t chunk = static_cast<std::uint32_t>((p ^ (row & 15)) * 16);
    load_lds_b128(qb, static_cast<std::uint32_t>(src * qs.row * 2) + chunk, lds_address(&b.q[row0][0]));
    load_lds_b128(kb, static_cast<std::uint32_t>(src * ks.row * 2) + chunk, lds_address(&b.k[row0][0]));
  }
  const int half = u >> 1, rows = 32 * (u & 1);
  load_rows_lds<kChunk, kChunk, 32, 1>(record, static_cast<std::uint32_t>(rec2::kTb + half * kChunk * kChunk * 2),
                                       &b.tb[half], rows);
  load_rows_lds<kChunk, kChunk, 32, 1>(record, static_cast<std::uint32_t>(rec2::kM + half * kChunk * kChunk * 2),
                                       &b.m[half], rows);
  if (u < 2) {
    const int row = 32 * u + (lane >> 1), src = row < L ? row : L - 1;
    const bf16_bits *vb = vs.base + t0 * vs.row + h * vs.head_stride + c0;
    load_lds_b128(vb, static_cast<std::uint32_t>(src * vs.row * 2 + (lane & 1) * 16),
                  lds_address(&b.v[32 * u][0]));
  } else if (u == 2 && lane < 16) {
    load_lds_b128(record, static_cast<std::uint32_t>(rec2::kG + 16 * lane), lds_address(&b.g[0]));
  }
}

// Block (value head, 16-column block), sequential over chunks, 8 waves.  Per
// chunk, with row tiles rt = 0..3 of the chunk and S^T / D^T in LDS:
//   1. waves 0-3: X = K S and QS for rows rt = w (one read of S^T for both),
//      Y = v_scale V - e^G k_scale X -> yt;
//   2. waves 0-3: D = Tb Y (rows w) -> dt, e^{G_last-G} D -> ft;
//   3. waves 0-3: S' = e^{G_last} S + k_scale K^T ft for state rows 32w ..
//      +31 (fp32 in VGPRs, then S'^T -> st); waves 4-7: O = e^G q_scale QS +
//      M D for rows w-4 (QS handed over through LDS in step 1).
// Waves 4-7, idle in steps 1 and 2, issue the loads of the next chunk's
// operands into the other buffer, so waves 0-3 never wait on memory.
template <typename OutT>
__global__ __launch_bounds__(kTScanThreads) void chunk_tscan_kernel(Src<bf16_bits> qs, Src<bf16_bits> ks,
                                                                    Src<bf16_bits> vs, ChunkScratch scratch,
                                                                    float *__restrict__ state,
                                                                    OutT *__restrict__ out,
                                                                    std::size_t tokens, std::size_t hk,
                                                                    std::size_t hv) {
  __shared__ TScanShared sh;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lk = lane >> 4;
  const std::size_t h = blockIdx.x;
  const std::size_t kh = h % hk;
  const int c0 = blockIdx.y * kColBlock;
  const float q_scale = qs.scale, k_scale = ks.scale, v_scale = vs.scale;
  float *sg = state + h * kChunkDim * kChunkDim;
  if (wave >= 4)
    tscan_issue(sh.buf[0], qs, ks, vs, scratch.at(h, 0), 0, static_cast<int>(tokens < kChunk ? tokens : kChunk),
                h, kh, c0, wave - 4);
  // fp32 state: waves 0-3 hold s[tt] = S[32 w + 16 tt + 4 lk + r][c0 + lr].
  floatx4 s[2];
  if (wave < 4) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int r = 0; r < 4; ++r) s[tt][r] = sg[(32 * wave + 16 * tt + 4 * lk + r) * kChunkDim + c0 + lr];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) store_split_t<kLdK>(sh.st[0], sh.st[1], 32 * wave + 16 * tt, s[tt]);
  }
  // Waves 4-7 store a chunk's output rows at the start of the next chunk, so
  // the wait for that chunk's loads does not also wait for fresh stores.
  floatx4 pend_o = floatx4{};
  std::size_t pend_t0 = 0;
  int pend_l = 0;
  auto store_o = [&](std::size_t ot0, int ol) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * (wave & 3) + 4 * lk + r;
      if (i < ol) Elem<OutT>::store(out, ((ot0 + i) * hv + h) * kChunkDim + c0 + lr, pend_o[r]);
    }
  };
  const int rt = wave & 3, i0 = 16 * rt;
  for (std::size_t c = 0, t0 = 0; t0 < tokens; ++c, t0 += kChunk) {
    const int L = static_cast<int>(tokens - t0 < kChunk ? tokens - t0 : kChunk);
    const TScanBuf &b = sh.buf[c & 1];
    if (wave >= 4) wait_vm<0>(); // loads of chunk c (and the stores of chunk c - 2)
    __syncthreads();             // every loader's loads, S^T, and the last chunk's reads done
    if (wave >= 4) {
      store_o(pend_t0, pend_l); // chunk c - 1 (none before chunk 1: pend_l = 0)
      if (t0 + kChunk < tokens) {
        const std::size_t t1 = t0 + kChunk;
        tscan_issue(sh.buf[(c + 1) & 1], qs, ks, vs, scratch.at(h, c + 1), t1,
                    static_cast<int>(tokens - t1 < kChunk ? tokens - t1 : kChunk), h, kh, c0, wave - 4);
      }
    }
    const float glast = b.g[kChunk - 1]; // = G[L-1] (padded)
    // ---- 1
    if (wave < 4) {
      floatx4 x0 = floatx4{}, x1 = floatx4{}, q0 = floatx4{}, q1 = floatx4{};
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const int ro = swz128(i0 + lr, 4 * n + lk);
        const bf16x8 ka = lds8(&b.k[0][0] + ro), qa = lds8(&b.q[0][0] + ro);
        const bf16x8 sth = lds8(&sh.st[0][lr][32 * n + 8 * lk]), stl = lds8(&sh.st[1][lr][32 * n + 8 * lk]);
        x0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, sth, x0, 0, 0, 0);
        x1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, stl, x1, 0, 0, 0);
        q0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa, sth, q0, 0, 0, 0);
        q1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa, stl, q1, 0, 0, 0);
      }
      floatx4 y, o;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = i0 + 4 * lk + r;
        const float eg = __expf(b.g[i]);
        y[r] = v_scale * bf16_lo(b.v[i][lr]) - eg * k_scale * (x0[r] + x1[r]);
        o[r] = eg * q_scale * (q0[r] + q1[r]);
      }
      store_split_t<kLdJ>(sh.yt[0], sh.yt[1], i0, y);
#pragma unroll
      for (int r = 0; r < 4; ++r) sh.qo[i0 + 4 * lk + r][lr] = o[r];
    }
    __syncthreads();
    // ---- 2
    if (wave < 4) {
      floatx4 fdec;
#pragma unroll
      for (int r = 0; r < 4; ++r) fdec[r] = __expf(glast - b.g[i0 + 4 * lk + r]);
      floatx4 d0 = floatx4{}, d1 = floatx4{}, d2 = floatx4{};
      const int steps = rt < 2 ? 1 : 2; // Tb is lower triangular
      for (int n = 0; n < steps; ++n) {
        const int to = swz64(i0 + lr, 4 * n + lk);
        const bf16x8 th = lds8(&b.tb[0][0][0] + to), tl = lds8(&b.tb[1][0][0] + to);
        const bf16x8 yh = lds8(&sh.yt[0][lr][32 * n + 8 * lk]), yl = lds8(&sh.yt[1][lr][32 * n + 8 * lk]);
        d0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(th, yh, d0, 0, 0, 0);
        d1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(th, yl, d1, 0, 0, 0);
        d2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(tl, yh, d2, 0, 0, 0);
      }
      // The decay factors are formed unconditionally (G is padded past L, so
      // they are finite there) and masked by a multiply: a select on i < L
      // would put each G read behind its own branch and LDS round trip.
      floatx4 dv, fv;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = i0 + 4 * lk + r;
        dv[r] = d0[r] + (d1[r] + d2[r]);
        fv[r] = (i < L ? 1.f : 0.f) * (fdec[r] * dv[r]);
      }
      store_split_t<kLdJ>(sh.dt[0], sh.dt[1], i0, dv);
      store_split_t<kLdJ>(sh.ft[0], sh.ft[1], i0, fv);
    }
    __syncthreads();
    // ---- 3
    if (wave < 4) {
      const float egl = __expf(glast);
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int d0 = 32 * wave + 16 * tt;
        // K^T operand (rows d0 + lr, keys 32 n + 8 lk .. +7) by transposed
        // reads of the K rows: source lane r of a 16-lane group supplies dims
        // d0 + 4 (r & 3) .. +3 of key (r >> 2) of a 4-key block.
        const int dsrc = d0 + 4 * (lr & 3);
        floatx4 a0 = floatx4{}, a1 = floatx4{};
#pragma unroll
        for (int n = 0; n < 2; ++n) {
          u32x2 part[2];
#pragma unroll
          for (int hq = 0; hq < 2; ++hq) {
            const int j = 32 * n + 8 * lk + 4 * hq + (lr >> 2);
            part[hq] = lds_tr16_b64(&b.k[0][0] + swz128(j, dsrc >> 3) + (dsrc & 7));
          }
          const bf16x8 kt = __builtin_bit_cast(bf16x8, u32x4{part[0][0], part[0][1], part[1][0], part[1][1]});
          const bf16x8 fh = lds8(&sh.ft[0][lr][32 * n + 8 * lk]), fl = lds8(&sh.ft[1][lr][32 * n + 8 * lk]);
          a0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kt, fh, a0, 0, 0, 0);
          a1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kt, fl, a1, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) s[tt][r] = fmaf(egl, s[tt][r], k_scale * (a0[r] + a1[r]));
        store_split_t<kLdK>(sh.st[0], sh.st[1], d0, s[tt]);
      }
    } else {
      floatx4 m0 = floatx4{}, m1 = floatx4{}, m2 = floatx4{};
      const int steps = rt < 2 ? 1 : 2; // M is lower triangular
      for (int n = 0; n < steps; ++n) {
        const int mo = swz64(i0 + lr, 4 * n + lk);
        const bf16x8 mh = lds8(&b.m[0][0][0] + mo), ml = lds8(&b.m[1][0][0] + mo);
        const bf16x8 dh = lds8(&sh.dt[0][lr][32 * n + 8 * lk]), dl = lds8(&sh.dt[1][lr][32 * n + 8 * lk]);
        m0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mh, dh, m0, 0, 0, 0);
        m1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mh, dl, m1, 0, 0, 0);
        m2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ml, dh, m2, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) pend_o[r] = sh.qo[i0 + 4 * lk + r][lr] + (m0[r] + (m1[r] + m2[r]));
      pend_t0 = t0;
      pend_l = L;
    }
  }
  if (wave >= 4) store_o(pend_t0, pend_l);
  if (wave < 4) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int r = 0; r < 4; ++r) sg[(32 * wave + 16 * tt + 4 * lk + r) * kChunkDim + c0 + lr] = s[tt][r];
  }
}

// ------------------------------ stage 2b, fp32 inputs as (hi, lo) planes
// The full entry's q / k / v are fp32 convolution outputs, written as bf16
// (hi, lo) planes (x = hi + lo); the scan is chunk_tscan_kernel's with every
// product over q, k or v taken as hi*hi + hi*lo + lo*hi.  The planes double
// the operand bytes, so only K (read in steps 1 and 3) is double-buffered;
// Q and V are reloaded once step 1 has read them, Tb once step 2 has, and M
// at the start of the chunk whose step 3 reads it.
struct TScanSplitShared {
  bf16_bits k[2][2][kChunk][kChunkDim]; // [chunk parity][hi, lo] K rows, 128-wide swizzle
  bf16_bits q[2][kChunk][kChunkDim];    // [hi, lo] Q rows
  bf16_bits tb[2][kChunk][kChunk];      // Tb (hi, lo), 64-wide swizzle
  bf16_bits m[2][kChunk][kChunk];       // M (hi, lo)
  bf16_bits v[2][kChunk][kColBlock];    // [hi, lo] V[i][c0 ..]
  float g[2][kChunk];                   // [chunk parity] G
  bf16_bits st[2][kColBlock][kLdK];
  bf16_bits yt[2][kColBlock][kLdJ];
  bf16_bits dt[2][kColBlock][kLdJ];
  bf16_bits ft[2][kColBlock][kLdJ];
  float qo[kChunk][kColBlock];
};

// LDS-direct loads of loader wave u = 0..3 (rows past L repeat row L-1):
//   K: rows 16u .. +15 of both planes (8 instructions), and G (loader 2, one
//      more);
//   M, Tb: half u / 2, rows 32 (u % 2) .. +31 (4 each);
//   Q: rows 16u .. +15 of both planes (8), V: plane u / 2, rows 32 (u % 2) ..
//      +31 of this block's 16 columns (1).
struct TScanSplitLoads {
  static constexpr int kM = 4, kTb = 4, kQv = 9;
  __device__ static constexpr int k_count(int u) { return 8 + (u == 2 ? 1 : 0); }
  __device__ static void rows128(bf16_bits (*dst)[kChunkDim], const bf16_bits *base, std::size_t row,
                                 int L, int u) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row0 = 16 * u + 4 * j, r = row0 + (lane >> 4), p = lane & 15;
      const int src = r < L ? r : L - 1;
      load_lds_b128(base, static_cast<std::uint32_t>(src * row * 2 + (p ^ (r & 15)) * 16),
                    lds_address(&dst[row0][0]));
    }
  }
  __device__ static void k(TScanSplitShared &sh, int parity, const Src<bf16_bits> &ks, std::size_t lo_plane,
                           const unsigned char *record, std::size_t t0, int L, std::size_t kh, int u) {
    const bf16_bits *kb = ks.base + t0 * ks.row + kh * ks.head_stride;
    rows128(sh.k[parity][0], kb, ks.row, L, u);
    rows128(sh.k[parity][1], kb + lo_plane, ks.row, L, u);
    if (u == 2 && (threadIdx.x & 63) < 16)
      load_lds_b128(record, static_cast<std::uint32_t>(rec2::kG + 16 * (threadIdx.x & 63)),
                    lds_address(&sh.g[parity][0]));
  }
  __device__ static void m(TScanSplitShared &sh, const unsigned char *record, int u) {
    const int half = u >> 1;
    load_rows_lds<kChunk, kChunk, 32, 1>(record, static_cast<std::uint32_t>(rec2::kM + half * kChunk * kChunk * 2),
                                         &sh.m[half], 32 * (u & 1));
  }
  __device__ static void tb(TScanSplitShared &sh, const unsigned char *record, int u) {
    const int half = u >> 1;
    load_rows_lds<kChunk, kChunk, 32, 1>(record, static_cast<std::uint32_t>(rec2::kTb + half * kChunk * kChunk * 2),
                                         &sh.tb[half], 32 * (u & 1));
  }
  __device__ static void qv(TScanSplitShared &sh, const Src<bf16_bits> &qs, const Src<bf16_bits> &vs,
                            std::size_t lo_plane, std::size_t t0, int L, std::size_t h, std::size_t kh, int c0,
                            int u) {
    const bf16_bits *qb = qs.base + t0 * qs.row + kh * qs.head_stride;
    rows128(sh.q[0], qb, qs.row, L, u);
    rows128(sh.q[1], qb + lo_plane, qs.row, L, u);
    const int lane = threadIdx.x & 63;
    const int row = 32 * (u & 1) + (lane >> 1), src = row < L ? row : L - 1;
    const bf16_bits *vb = vs.base + t0 * vs.row + h * vs.head_stride + c0 + (u >> 1) * lo_plane;
    load_lds_b128(vb, static_cast<std::uint32_t>(src * vs.row * 2 + (lane & 1) * 16),
                  lds_address(&sh.v[u >> 1][32 * (u & 1)][0]));
  }
  // Waits until at most `later` of this wave's loads are outstanding (loads
  // return in order).  The count must be an immediate, hence the branches.
  template <int kFixed> __device__ static void wait_k_later(int u, bool more) {
    if (!more)
      wait_vm<kFixed>();
    else if (u == 2)
      wait_vm<kFixed + 9>();
    else
      wait_vm<kFixed + 8>();
  }
};

template <typename OutT>
__global__ __launch_bounds__(kTScanThreads) void chunk_tscan_split_kernel(Src<bf16_bits> qs, Src<bf16_bits> ks,
                                                                          Src<bf16_bits> vs, std::size_t lo_plane,
                                                                          ChunkScratch scratch,
                                                                          float *__restrict__ state,
                                                                          OutT *__restrict__ out,
                                                                          std::size_t tokens, std::size_t hk,
                                                                          std::size_t hv) {
  using Loads = TScanSplitLoads;
  __shared__ TScanSplitShared sh;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lk = lane >> 4;
  const int u = wave - 4; // loader index of waves 4-7
  const std::size_t h = blockIdx.x;
  const std::size_t kh = h % hk;
  const int c0 = blockIdx.y * kColBlock;
  const float q_scale = qs.scale, k_scale = ks.scale, v_scale = vs.scale;
  float *sg = state + h * kChunkDim * kChunkDim;
  if (wave >= 4) {
    const int L0 = static_cast<int>(tokens < kChunk ? tokens : kChunk);
    const unsigned char *rec0 = scratch.at(h, 0);
    Loads::k(sh, 0, ks, lo_plane, rec0, 0, L0, kh, u);
    Loads::m(sh, rec0, u);
    Loads::qv(sh, qs, vs, lo_plane, 0, L0, h, kh, c0, u);
    Loads::tb(sh, rec0, u);
  }
  floatx4 s[2];
  if (wave < 4) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int r = 0; r < 4; ++r) s[tt][r] = sg[(32 * wave + 16 * tt + 4 * lk + r) * kChunkDim + c0 + lr];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) store_split_t<kLdK>(sh.st[0], sh.st[1], 32 * wave + 16 * tt, s[tt]);
  }
  floatx4 pend_o = floatx4{};
  std::size_t pend_t0 = 0;
  int pend_l = 0;
  auto store_o = [&](std::size_t ot0, int ol) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * (wave & 3) + 4 * lk + r;
      if (i < ol) Elem<OutT>::store(out, ((ot0 + i) * hv + h) * kChunkDim + c0 + lr, pend_o[r]);
    }
  };
  const int rt = wave & 3, i0 = 16 * rt;
  for (std::size_t c = 0, t0 = 0; t0 < tokens; ++c, t0 += kChunk) {
    const int L = static_cast<int>(tokens - t0 < kChunk ? tokens - t0 : kChunk);
    const int par = static_cast<int>(c & 1);
    const bool more = t0 + kChunk < tokens;
    const std::size_t t1 = t0 + kChunk;
    const int L1 = more ? static_cast<int>(tokens - t1 < kChunk ? tokens - t1 : kChunk) : 0;
    // K, G, Q, V of chunk c are in (Tb of chunk c, 4 loads, was issued later).
    if (wave >= 4) {
      if (c == 0)
        wait_vm<0>();
      else
        wait_vm<Loads::kTb>();
    }
    __syncthreads();
    if (wave >= 4) {
      store_o(pend_t0, pend_l); // chunk c - 1
      if (more) Loads::k(sh, par ^ 1, ks, lo_plane, scratch.at(h, c + 1), t1, L1, kh, u);
      if (c > 0) Loads::m(sh, scratch.at(h, c), u); // step 3 of chunk c - 1 has read M
    }
    const float *g = sh.g[par];
    const float glast = g[kChunk - 1];
    // ---- 1
    if (wave < 4) {
      const bf16_bits *kh0 = &sh.k[par][0][0][0], *kh1 = &sh.k[par][1][0][0];
      floatx4 x0 = floatx4{}, x1 = floatx4{}, x2 = floatx4{}, q0 = floatx4{}, q1 = floatx4{}, q2 = floatx4{};
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const int ro = swz128(i0 + lr, 4 * n + lk);
        const bf16x8 kh = lds8(kh0 + ro), kl = lds8(kh1 + ro);
        const bf16x8 qh = lds8(&sh.q[0][0][0] + ro), ql = lds8(&sh.q[1][0][0] + ro);
        const bf16x8 sth = lds8(&sh.st[0][lr][32 * n + 8 * lk]), stl = lds8(&sh.st[1][lr][32 * n + 8 * lk]);
        x0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, sth, x0, 0, 0, 0);
        x1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, stl, x1, 0, 0, 0);
        x2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kl, sth, x2, 0, 0, 0);
        q0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qh, sth, q0, 0, 0, 0);
        q1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qh, stl, q1, 0, 0, 0);
        q2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ql, sth, q2, 0, 0, 0);
      }
      floatx4 y, o;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = i0 + 4 * lk + r;
        const float eg = __expf(g[i]);
        const float vv = bf16_lo(sh.v[0][i][lr]) + bf16_lo(sh.v[1][i][lr]);
        y[r] = v_scale * vv - eg * k_scale * (x0[r] + (x1[r] + x2[r]));
        o[r] = eg * q_scale * (q0[r] + (q1[r] + q2[r]));
      }
      store_split_t<kLdJ>(sh.yt[0], sh.yt[1], i0, y);
#pragma unroll
      for (int r = 0; r < 4; ++r) sh.qo[i0 + 4 * lk + r][lr] = o[r];
    }
    // Tb of chunk c: issued before the K of chunk c + 1 and this chunk's M.
    if (wave >= 4 && c > 0) {
      if (more) {
        if (u == 2)
          wait_vm<Loads::kM + 9>();
        else
          wait_vm<Loads::kM + 8>();
      } else {
        wait_vm<Loads::kM>();
      }
    }
    __syncthreads();
    if (wave >= 4 && more) Loads::qv(sh, qs, vs, lo_plane, t1, L1, h, kh, c0, u); // step 1 has read Q, V
    // ---- 2
    if (wave < 4) {
      floatx4 fdec;
#pragma unroll
      for (int r = 0; r < 4; ++r) fdec[r] = __expf(glast - g[i0 + 4 * lk + r]);
      floatx4 d0 = floatx4{}, d1 = floatx4{}, d2 = floatx4{};
      const int steps = rt < 2 ? 1 : 2;
      for (int n = 0; n < steps; ++n) {
        const int to = swz64(i0 + lr, 4 * n + lk);
        const bf16x8 th = lds8(&sh.tb[0][0][0] + to), tl = lds8(&sh.tb[1][0][0] + to);
        const bf16x8 yh = lds8(&sh.yt[0][lr][32 * n + 8 * lk]), yl = lds8(&sh.yt[1][lr][32 * n + 8 * lk]);
        d0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(th, yh, d0, 0, 0, 0);
        d1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(th, yl, d1, 0, 0, 0);
        d2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(tl, yh, d2, 0, 0, 0);
      }
      floatx4 dv, fv;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = i0 + 4 * lk + r;
        dv[r] = d0[r] + (d1[r] + d2[r]);
        fv[r] = (i < L ? 1.f : 0.f) * (fdec[r] * dv[r]);
      }
      store_split_t<kLdJ>(sh.dt[0], sh.dt[1], i0, dv);
      store_split_t<kLdJ>(sh.ft[0], sh.ft[1], i0, fv);
    }
    // M of chunk c: only this chunk's Q and V (if any) were issued after it.
    if (wave >= 4 && c > 0) {
      if (more)
        wait_vm<Loads::kQv>();
      else
        wait_vm<0>();
    }
    __syncthreads();
    if (wave >= 4 && more) Loads::tb(sh, scratch.at(h, c + 1), u); // step 2 has read Tb
    // ---- 3
    if (wave < 4) {
      const bf16_bits *kh0 = &sh.k[par][0][0][0], *kh1 = &sh.k[par][1][0][0];
      const float egl = __expf(glast);
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int d0 = 32 * wave + 16 * tt;
        const int dsrc = d0 + 4 * (lr & 3);
        floatx4 a0 = floatx4{}, a1 = floatx4{}, a2 = floatx4{};
#pragma unroll
        for (int n = 0; n < 2; ++n) {
          u32x2 ph[2], pl[2];
#pragma unroll
          for (int hq = 0; hq < 2; ++hq) {
            const int j = 32 * n + 8 * lk + 4 * hq + (lr >> 2);
            const int off = swz128(j, dsrc >> 3) + (dsrc & 7);
            ph[hq] = lds_tr16_b64(kh0 + off);
            pl[hq] = lds_tr16_b64(kh1 + off);
          }
          const bf16x8 kth = __builtin_bit_cast(bf16x8, u32x4{ph[0][0], ph[0][1], ph[1][0], ph[1][1]});
          const bf16x8 ktl = __builtin_bit_cast(bf16x8, u32x4{pl[0][0], pl[0][1], pl[1][0], pl[1][1]});
          const bf16x8 fh = lds8(&sh.ft[0][lr][32 * n + 8 * lk]), fl = lds8(&sh.ft[1][lr][32 * n + 8 * lk]);
          a0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kth, fh, a0, 0, 0, 0);
          a1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kth, fl, a1, 0, 0, 0);
          a2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ktl, fh, a2, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) s[tt][r] = fmaf(egl, s[tt][r], k_scale * (a0[r] + (a1[r] + a2[r])));
        store_split_t<kLdK>(sh.st[0], sh.st[1], d0, s[tt]);
      }
    } else {
      floatx4 m0 = floatx4{}, m1 = floatx4{}, m2 = floatx4{};
      const int steps = rt < 2 ? 1 : 2;
      for (int n = 0; n < steps; ++n) {
        const int mo = swz64(i0 + lr, 4 * n + lk);
        const bf16x8 mh = lds8(&sh.m[0][0][0] + mo), ml = lds8(&sh.m[1][0][0] + mo);
        const bf16x8 dh = lds8(&sh.dt[0][lr][32 * n + 8 * lk]), dl = lds8(&sh.dt[1][lr][32 * n + 8 * lk]);
        m0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mh, dh, m0, 0, 0, 0);
        m1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mh, dl, m1, 0, 0, 0);
        m2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ml, dh, m2, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) pend_o[r] = sh.qo[i0 + 4 * lk + r][lr] + (m0[r] + (m1[r] + m2[r]));
      pend_t0 = t0;
      pend_l = L;
    }
  }
  if (wave >= 4) store_o(pend_t0, pend_l);
  if (wave < 4) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int r = 0; r < 4; ++r) sg[(32 * wave + 16 * tt + 4 * lk + r) * kChunkDim + c0 + lr] = s[tt][r];
  }
}

// ----------------------------------------------------- stage 3 kernel
// Block (token, value head): RMSNorm over dv, x weight, x SiLU(z)
// (cpp/kernels/qwen35_delta.cu:578-621).
template <typename T, typename Wt>
__global__ __launch_bounds__(256) void out_norm_kernel(DeltaRows<T> in,
                                                       const Wt *__restrict__ norm_w,
                                                       const float *__restrict__ raw,
                                                       T *__restrict__ output, std::size_t hv,
                                                       std::size_t dv, float eps) {
  __shared__ float red[4];
  const std::size_t t = blockIdx.x / hv, h = blockIdx.x % hv;
  const std::size_t base = (t * hv + h) * dv;
  float ss = 0.f;
  for (std::size_t i = threadIdx.x; i < dv; i += 256) ss += raw[base + i] * raw[base + i];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float total = red[0] + red[1] + red[2] + red[3];
  const float scale = rsqrtf(total / static_cast<float>(dv) + eps);
  const std::size_t zb = h * dv;
  for (std::size_t i = threadIdx.x; i < dv; i += 256) {
    const float n = raw[base + i] * scale * Elem<Wt>::load(norm_w, i);
    Elem<T>::store(output, base + i, n * silu(in.gate(t, zb + i)));
  }
}

// One-token call of the Qwen3.5 shape in one kernel: convolution, SiLU,
// q/k L2 norm, beta / decay, recurrence and output norm.  One workgroup per
// key head kh with two 8-wave groups, one per value head kh + g * hk (g = 0,
// 1; hv = 2 hk), so the key head's q/k channels are convolved, and their
// history shifted, by one workgroup only: no workgroup reads a history that
// another one writes.  Thread cs < 512 of the workgroup owns channel slot cs
// (q 0..127, k 128..255, v of group 0 256..383, v of group 1 384..511) and
// shifts that channel's history itself.  The recurrence part is
// recurrent_head_norm_kernel's, with q, k, v from LDS.
template <typename T, typename Wt>
__global__ __launch_bounds__(1024) void decode_step_fused_kernel(
    DeltaRows<T> in, const Wt *__restrict__ conv_w, float *__restrict__ conv_state,
    const Wt *__restrict__ recurrent_a, const Wt *__restrict__ dt_bias, float *__restrict__ state,
    const Wt *__restrict__ norm_w, T *__restrict__ output, std::size_t hk, float eps) {
  constexpr int kDim = 128, kRows = 8, H = 3;
  __shared__ float cv[4][kDim];         // normalised q, k; v of groups 0, 1
  __shared__ float part_ss[4];          // q / k sum-of-squares halves (wave 0..3)
  __shared__ float bd[2][2];            // [group][beta, decay]
  __shared__ float4 red[2][2][8][32];   // [group][kv / o][wave][column quad]
  const int tid = threadIdx.x, lane = tid & 63;
  const int g = tid >> 9, lt = tid & 511, wave = lt >> 6;
  const std::size_t kh = blockIdx.x;
  const std::size_t h = kh + g * hk;
  const std::size_t key_size = hk * kDim;
  const int cq = lt & 31, rg = lt >> 5;
  const int c0 = 4 * cq, r0 = kRows * rg;
  // This group's state rows go to LDS by LDS-direct loads (the CU fetches
  // about twice as fast that way as into registers), issued before anything
  // else; each thread reads its own 8 rows x 16 bytes back after the
  // convolution.  Instruction i of a wave moves row r0 + i of both row groups
  // of the wave (lanes 0-31, 32-63).
  __shared__ float4 stage[16][kRows][64];
  float *sh = state + h * kDim * kDim;
#pragma unroll
  for (int i = 0; i < kRows; ++i)
    load_lds_b128(sh, static_cast<std::uint32_t>(((r0 + i) * kDim + c0) * 4), lds_address(&stage[tid >> 6][i][0]));
  float nw[4], z[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    nw[i] = Elem<Wt>::load(norm_w, c0 + i);
    z[i] = in.gate(0, h * kDim + c0 + i);
  }
  if (tid < 512) {
    const int cs = tid;
    const std::size_t ch = cs < 128   ? kh * kDim + cs
                           : cs < 256 ? key_size + kh * kDim + (cs - 128)
                                      : 2 * key_size + (kh + (cs >= 384 ? hk : 0)) * kDim + (cs & 127);
    const float cur = in.x(0, ch);
    float hist[H], w[H + 1];
#pragma unroll
    for (int j = 0; j < H; ++j) hist[j] = conv_state[ch * H + j];
#pragma unroll
    for (int j = 0; j <= H; ++j) w[j] = Elem<Wt>::load(conv_w, ch * (H + 1) + j);
    float sum = cur * w[H];
#pragma unroll
    for (int j = 0; j < H; ++j) sum += hist[j] * w[j];
    const float y = silu(sum);
    conv_state[ch * H + 0] = hist[1];
    conv_state[ch * H + 1] = hist[2];
    conv_state[ch * H + 2] = cur;
    float ss = y * y;
    ss = sum_xor32(sum_xor16(row16_sum(ss)));
    if (cs < 256 && lane == 0) part_ss[cs >> 6] = ss;
    cv[cs >> 7][cs & 127] = y;
  } else if (tid < 514) {
    const int gg = tid - 512;
    const std::size_t hh = kh + gg * hk;
    const float b = Elem<T>::load(in.b, hh);
    const float a = Elem<T>::load(in.a, hh);
    bd[gg][0] = sigmoid(b);
    bd[gg][1] = __expf(Elem<Wt>::load(recurrent_a, hh) * softplus(a + Elem<Wt>::load(dt_bias, hh)));
  }
  __syncthreads();
  const float qn = (1.0f / sqrtf(static_cast<float>(kDim))) / sqrtf(part_ss[0] + part_ss[1] + kQkNormEpsilon);
  const float kn = 1.0f / sqrtf(part_ss[2] + part_ss[3] + kQkNormEpsilon);
  auto row_sum = [&](float4 x, int which) {
    // lane ^ 32 holds the other row group of this wave for the same quad
    x.x = sum_xor32(x.x);
    x.y = sum_xor32(x.y);
    x.z = sum_xor32(x.z);
    x.w = sum_xor32(x.w);
    if (lane < 32) red[g][which][wave][cq] = x;
    __syncthreads();
    float4 t = red[g][which][0][cq];
#pragma unroll
    for (int w = 1; w < 8; ++w) {
      const float4 u = red[g][which][w][cq];
      t.x += u.x; t.y += u.y; t.z += u.z; t.w += u.w;
    }
    return t;
  };
  const float b = bd[g][0], decay = bd[g][1];
  wait_vm<0>(); // this thread's state rows have landed (the barrier above waited for every wave's)
  float4 s[kRows];
#pragma unroll
  for (int i = 0; i < kRows; ++i) s[i] = stage[tid >> 6][i][lane];
  float kr[kRows], qr[kRows];
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    kr[i] = cv[1][r0 + i] * kn;
    qr[i] = cv[0][r0 + i] * qn;
  }
  float vv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) vv[i] = cv[2 + g][c0 + i];
  float4 part = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    s[i].x *= decay; s[i].y *= decay; s[i].z *= decay; s[i].w *= decay;
    part.x = fmaf(s[i].x, kr[i], part.x);
    part.y = fmaf(s[i].y, kr[i], part.y);
    part.z = fmaf(s[i].z, kr[i], part.z);
    part.w = fmaf(s[i].w, kr[i], part.w);
  }
  const float4 kv = row_sum(part, 0);
  const float4 d = make_float4((vv[0] - kv.x) * b, (vv[1] - kv.y) * b, (vv[2] - kv.z) * b, (vv[3] - kv.w) * b);
  float4 po = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    s[i].x = fmaf(kr[i], d.x, s[i].x);
    s[i].y = fmaf(kr[i], d.y, s[i].y);
    s[i].z = fmaf(kr[i], d.z, s[i].z);
    s[i].w = fmaf(kr[i], d.w, s[i].w);
    po.x = fmaf(s[i].x, qr[i], po.x);
    po.y = fmaf(s[i].y, qr[i], po.y);
    po.z = fmaf(s[i].z, qr[i], po.z);
    po.w = fmaf(s[i].w, qr[i], po.w);
  }
  const float4 o = row_sum(po, 1);
  if (wave == 0) {
    // lanes 0..31 cover the 32 column quads (lanes 32..63 repeat them)
    float ss = o.x * o.x + o.y * o.y + o.z * o.z + o.w * o.w;
    ss = sum_xor16(row16_sum(ss));
    const float scale = rsqrtf(ss / static_cast<float>(kDim) + eps);
    if (lane < 32) {
      const std::size_t base = h * kDim + c0;
      const float ov[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) Elem<T>::store(output, base + i, ov[i] * scale * nw[i] * silu(z[i]));
    }
  }
#pragma unroll
  for (int i = 0; i < kRows; ++i) *reinterpret_cast<float4 *>(sh + (r0 + i) * kDim + c0) = s[i];
}

// ------------------------------------------------------------ launchers

template <typename InT, typename OutT>
void launch_recurrence(Src<InT> q, Src<InT> k, Src<InT> v, const float *beta, const float *g,
                       float *state, OutT *out, ChunkScratch scratch, std::size_t tokens,
                       std::size_t hk, std::size_t hv, std::size_t dk, std::size_t dv, bool chunked,
                       hipStream_t stream) {
  if (chunked) {
    const dim3 pgrid{static_cast<unsigned>(hv), static_cast<unsigned>(ceil_div_unchecked(tokens, kChunk)), 1};
    const dim3 sgrid{static_cast<unsigned>(hv), kChunkDim / kColBlock, 1};
    if constexpr (std::is_same_v<InT, bf16_bits>) {
      chunk_tb_kernel<false><<<pgrid, 256, 0, stream>>>(q, k, 0, beta, g, scratch, tokens, hk, hv);
      check_launch<Err>("qwen35_gated_delta chunk preparation");
      chunk_tscan_kernel<OutT><<<sgrid, kTScanThreads, 0, stream>>>(q, k, v, scratch, state, out, tokens, hk, hv);
      check_launch<Err>("qwen35_gated_delta chunk scan");
    } else {
      chunk_prep_kernel<InT><<<pgrid, 256, 0, stream>>>(q, k, v, beta, g, scratch, tokens, hk, hv);
      check_launch<Err>("qwen35_gated_delta chunk preparation");
      chunk_scan_kernel<OutT><<<sgrid, 256, 0, stream>>>(scratch, state, out, tokens, hv);
      check_launch<Err>("qwen35_gated_delta chunk scan");
    }
    return;
  }
  if (dk == 128 && dv == 128 && (reinterpret_cast<std::uintptr_t>(state) & 15u) == 0) {
    const dim3 g128{static_cast<unsigned>(hv), 128 / kRec128Cols, 1};
    recurrent_128_kernel<InT, OutT><<<g128, 256, 0, stream>>>(q, k, v, beta, g, state, out, tokens, hk, hv);
    check_launch<Err>("qwen35_gated_delta register recurrent update");
    return;
  }
  const dim3 grid{static_cast<unsigned>(hv), static_cast<unsigned>(ceil_div_unchecked(dv, 64)), 1};
  if (dk <= kRecWaves * 16)
    recurrent_kernel<InT, OutT, 16><<<grid, kRecWaves * 64, 0, stream>>>(q, k, v, beta, g, state, out,
                                                                         tokens, hk, hv, dk, dv);
  else
    recurrent_kernel<InT, OutT, 32><<<grid, kRecWaves * 64, 0, stream>>>(q, k, v, beta, g, state, out,
                                                                         tokens, hk, hv, dk, dv);
  check_launch<Err>("qwen35_gated_delta register recurrent update");
}

// Host-side, type-erased DeltaRows: base pointers and strides in elements.
struct DeltaSources {
  const void *qkv;
  std::size_t qkv_stride;
  const void *b;
  std::size_t b_stride;
  const void *a;
  std::size_t a_stride;
  const void *z;
  std::size_t z_stride;
};

bool use_chunked(const GatedDeltaShape &s, const GatedDeltaLaunchPolicy &p) {
  if (s.key_dim != kChunkDim || s.value_dim != kChunkDim) return false;
  if (p.schedule == GatedDeltaSchedule::register_resident_prefill_sm120) return true;
  if (p.schedule == GatedDeltaSchedule::register_resident_decode_sm120) return false;
  return s.tokens >= kChunkThreshold;
}

template <typename T, typename Wt>
void launch_typed(const DeltaSources &src, const void *conv_weight, const void *recurrent_a,
                  const void *dt_bias, const void *norm_w, void *output, float *conv_state,
                  float *rec_state, float *ws, const GatedDeltaShape &s, const CheckedShape &c,
                  const GatedDeltaLaunchPolicy &policy, hipStream_t stream) {
  const DeltaRows<T> in{static_cast<const T *>(src.qkv), src.qkv_stride,
                        static_cast<const T *>(src.b),   src.b_stride,
                        static_cast<const T *>(src.a),   src.a_stride,
                        static_cast<const T *>(src.z),   src.z_stride};
  float *convolved = ws;
  float *raw = convolved + s.tokens * c.conv_dim;
  float *beta = raw + s.tokens * s.hidden_size;
  float *gdecay = beta + s.tokens * s.value_heads;
  ChunkScratch scratch{};
  if (chunk_record_bytes(s.tokens, s.value_heads, s.key_dim, s.value_dim) != 0) {
    scratch.rec = reinterpret_cast<unsigned char *>(ws) +
                  record_offset(s.tokens * (c.conv_dim + s.hidden_size + 2 * s.value_heads) * sizeof(float));
    scratch.chunks = ceil_div_unchecked(s.tokens, kChunk);
    scratch.bytes = rec::kBytes;
  }

  const bool fast = s.key_dim == kChunkDim && s.value_dim == kChunkDim && s.conv_width == 4 &&
                    c.conv_dim % 2048 == 0 && s.hidden_size % 2048 == 0 &&
                    src.qkv_stride % 8 == 0 && src.z_stride % 8 == 0 &&
                    ((reinterpret_cast<std::uintptr_t>(src.qkv) | reinterpret_cast<std::uintptr_t>(src.z) |
                      reinterpret_cast<std::uintptr_t>(ws)) & 15u) == 0;
  // The channel-spread convolution also reads weights and history as vectors.
  const bool wide = fast && ((reinterpret_cast<std::uintptr_t>(conv_weight) |
                              reinterpret_cast<std::uintptr_t>(conv_state)) & 15u) == 0;
  const bool chunk_eligible = use_chunked(s, policy) && (reinterpret_cast<std::uintptr_t>(ws) & 15u) == 0;
  const bool one_token_state = wide && s.tokens == 1;
  // The chunked path on the wide convolution takes q / k / v as (hi, lo)
  // bf16 planes (chunk_tb_kernel<true> + chunk_tscan_split_kernel).
  const bool split_chunked = wide && chunk_eligible && !one_token_state && s.key_dim == kChunkDim &&
                             s.value_dim == kChunkDim;
  // The W/U-record path needs records of rec::kBytes, which the workspace
  // holds only for shapes that are not channel-spread; a channel-spread shape
  // whose pointers rule out the wide convolution runs the recurrent kernels.
  const bool chunked = chunk_eligible && (split_chunked || !channel_spread_shape(s, c.conv_dim));
  constexpr int kConvTokens = 4; // tokens per workgroup of the multi-token convolution
  // A one-token call of the model shape (two value heads per key head): the
  // convolution, recurrence and output norm in one kernel.
  if (one_token_state && s.value_heads == 2 * s.key_heads && !chunked &&
      (reinterpret_cast<std::uintptr_t>(rec_state) & 15u) == 0) {
    decode_step_fused_kernel<T, Wt><<<static_cast<unsigned>(s.key_heads), 1024, 0, stream>>>(
        in, static_cast<const Wt *>(conv_weight), conv_state, static_cast<const Wt *>(recurrent_a),
        static_cast<const Wt *>(dt_bias), rec_state, static_cast<const Wt *>(norm_w), static_cast<T *>(output),
        s.key_heads, s.epsilon);
    check_launch<Err>("qwen35_gated_delta fused decode step");
    return;
  }
  if (wide) {
    const unsigned blocks_y = static_cast<unsigned>(c.conv_dim / kConvWideChannels);
    if (one_token_state)
      conv_norm_wide_kernel<T, Wt, 4, 1, true><<<dim3(1, blocks_y, 1), 64, 0, stream>>>(
          in, static_cast<const Wt *>(conv_weight), conv_state, static_cast<const Wt *>(recurrent_a),
          static_cast<const Wt *>(dt_bias), convolved, beta, gdecay, s.tokens,
          c.conv_dim, 2 * c.key_size, s.value_heads);
    else if (split_chunked) // (an extra row of blocks computes beta and the decay)
      conv_norm_wide_kernel<T, Wt, 4, kConvTokens, false, true>
          <<<dim3(static_cast<unsigned>(ceil_div_unchecked(s.tokens, kConvTokens)), blocks_y + 1, 1), 64, 0,
             stream>>>(
              in, static_cast<const Wt *>(conv_weight), conv_state, static_cast<const Wt *>(recurrent_a),
              static_cast<const Wt *>(dt_bias), convolved, beta, gdecay, s.tokens,
              c.conv_dim, 2 * c.key_size, s.value_heads);
    else
      conv_norm_wide_kernel<T, Wt, 4, kConvTokens, false>
          <<<dim3(static_cast<unsigned>(ceil_div_unchecked(s.tokens, kConvTokens)), blocks_y, 1), 64, 0,
             stream>>>(
              in, static_cast<const Wt *>(conv_weight), conv_state, static_cast<const Wt *>(recurrent_a),
              static_cast<const Wt *>(dt_bias), convolved, beta, gdecay, s.tokens,
              c.conv_dim, 2 * c.key_size, s.value_heads);
  } else if (fast) {
    conv_norm_fast_kernel<T, Wt, 4><<<static_cast<unsigned>(s.tokens), 256, 0, stream>>>(
        in, static_cast<const Wt *>(conv_weight), conv_state, static_cast<const Wt *>(recurrent_a),
        static_cast<const Wt *>(dt_bias), convolved, beta, gdecay, c.conv_dim,
        2 * c.key_size, s.value_heads);
  } else {
    const dim3 cgrid{static_cast<unsigned>(s.tokens), static_cast<unsigned>(2 * s.key_heads + s.value_heads), 1};
    conv_norm_kernel<T, Wt><<<cgrid, 256, 0, stream>>>(
        in, static_cast<const Wt *>(conv_weight), conv_state, static_cast<const Wt *>(recurrent_a),
        static_cast<const Wt *>(dt_bias), convolved, beta, gdecay, s.tokens, c.conv_dim,
        s.key_heads, s.value_heads, s.key_dim, s.value_dim, s.conv_width);
  }
  check_launch<Err>("qwen35_gated_delta batched convolution");
  // The wide path shifts the history inside its last kernel (the one-token
  // convolution already did).
  if (s.conv_width > 1 && !wide) {
    conv_state_kernel<T><<<static_cast<unsigned>(ceil_div_unchecked(c.conv_dim, 256)), 256, 0, stream>>>(
        in, conv_state, s.tokens, c.conv_dim, s.conv_width);
    check_launch<Err>("qwen35_gated_delta convolution state update");
  }
  const Src<float> q{convolved, c.conv_dim, s.key_dim, 1.0f};
  const Src<float> k{convolved + c.key_size, c.conv_dim, s.key_dim, 1.0f};
  const Src<float> v{convolved + 2 * c.key_size, c.conv_dim, s.value_dim, 1.0f};
  if (fast && !chunked && (reinterpret_cast<std::uintptr_t>(rec_state) & 15u) == 0) {
    // recurrence and output norm in one kernel (one workgroup per value head)
    recurrent_head_norm_kernel<T, Wt><<<static_cast<unsigned>(s.value_heads), 512, 0, stream>>>(
        q, k, v, beta, gdecay, rec_state, in, static_cast<const Wt *>(norm_w),
        static_cast<T *>(output), s.tokens, s.key_heads, s.value_heads, c.conv_dim,
        s.epsilon, wide && !one_token_state ? conv_state : nullptr);
    check_launch<Err>("qwen35_gated_delta register recurrent update");
    return;
  }
  if (split_chunked) {
    const bf16_bits *planes = reinterpret_cast<const bf16_bits *>(convolved);
    const Src<bf16_bits> qh{planes, c.conv_dim, s.key_dim, 1.0f};
    const Src<bf16_bits> kh{planes + c.key_size, c.conv_dim, s.key_dim, 1.0f};
    const Src<bf16_bits> vh{planes + 2 * c.key_size, c.conv_dim, s.value_dim, 1.0f};
    const std::size_t lo_plane = s.tokens * c.conv_dim;
    ChunkScratch rec = scratch;
    rec.bytes = rec2::kBytes;
    const dim3 pgrid{static_cast<unsigned>(s.value_heads), static_cast<unsigned>(rec.chunks), 1};
    chunk_tb_kernel<true><<<pgrid, 256, 0, stream>>>(qh, kh, lo_plane, beta, gdecay, rec, s.tokens, s.key_heads,
                                                     s.value_heads);
    check_launch<Err>("qwen35_gated_delta chunk preparation");
    const dim3 sgrid{static_cast<unsigned>(s.value_heads), kChunkDim / kColBlock, 1};
    chunk_tscan_split_kernel<float><<<sgrid, kTScanThreads, 0, stream>>>(qh, kh, vh, lo_plane, rec, rec_state, raw,
                                                                         s.tokens, s.key_heads, s.value_heads);
    check_launch<Err>("qwen35_gated_delta chunk scan");
  } else {
    launch_recurrence<float, float>(q, k, v, beta, gdecay, rec_state, raw, scratch, s.tokens,
                                    s.key_heads, s.value_heads, s.key_dim, s.value_dim, chunked,
                                    stream);
  }
  if (fast)
    out_norm_fast_kernel<T, Wt><<<static_cast<unsigned>(s.tokens), 256, 0, stream>>>(
        in, static_cast<const Wt *>(norm_w), raw, static_cast<T *>(output), c.conv_dim,
        s.value_heads, s.epsilon, wide && !one_token_state ? conv_state : nullptr, s.tokens);
  else
    out_norm_kernel<T, Wt><<<static_cast<unsigned>(s.tokens * s.value_heads), 256, 0, stream>>>(
        in, static_cast<const Wt *>(norm_w), raw, static_cast<T *>(output), s.value_heads,
        s.value_dim, s.epsilon);
  check_launch<Err>("qwen35_gated_delta batched output normalization");
}

template <typename T>
void launch_for_weights(RaftInferDataType wdt, const DeltaSources &input, const void *conv_weight,
                        const void *recurrent_a, const void *dt_bias, const void *norm_w,
                        void *output, float *conv_state, float *rec_state, float *ws,
                        const GatedDeltaShape &s, const CheckedShape &c,
                        const GatedDeltaLaunchPolicy &policy, hipStream_t stream) {
  if (wdt == RAFTINFER_DTYPE_F32)
    launch_typed<T, float>(input, conv_weight, recurrent_a, dt_bias, norm_w, output, conv_state,
                           rec_state, ws, s, c, policy, stream);
  else if (wdt == RAFTINFER_DTYPE_F16)
    launch_typed<T, _Float16>(input, conv_weight, recurrent_a, dt_bias, norm_w, output, conv_state,
                              rec_state, ws, s, c, policy, stream);
  else
    launch_typed<T, bf16_bits>(input, conv_weight, recurrent_a, dt_bias, norm_w, output, conv_state,
                               rec_state, ws, s, c, policy, stream);
}

} // namespace

std::size_t qwen35_gated_delta_workspace_bytes(const GatedDeltaShape &shape) {
  return validate_shape(shape).workspace_bytes;
}

// The chunked schedule is the gfx950 counterpart of the reference's prefill
// candidate; auto selection (register_resident_current) picks chunked for
// >= 64 tokens of 128-dim heads and the register recurrence otherwise.
GatedDeltaLaunchPolicy qwen35_gated_delta_select_policy(const GatedDeltaShape &,
                                                        std::size_t) noexcept {
  return GatedDeltaLaunchPolicy{GatedDeltaSchedule::register_resident_current, 4, false};
}

GatedDeltaScheduleDiagnostic qwen35_gated_delta_schedule_diagnostic(const GatedDeltaShape &shape,
                                                                    std::size_t bucket) noexcept {
  const auto p = qwen35_gated_delta_select_policy(shape, bucket);
  GatedDeltaScheduleDiagnostic d;
  d.bucket_tokens = bucket;
  d.key_dim = shape.key_dim;
  d.value_dim = shape.value_dim;
  d.candidate_schedule = bucket == 1 ? GatedDeltaSchedule::register_resident_decode_sm120
                                     : GatedDeltaSchedule::register_resident_prefill_sm120;
  d.schedule = p.schedule;
  d.warps_per_block = p.warps_per_block;
  d.transposed_boundary_state = p.transposed_boundary_state;
  d.candidate_accepted = p.schedule != GatedDeltaSchedule::register_resident_current;
  d.correctness_passed = false;
  d.rejection_reason = "not_tuned";
  return d;
}

void qwen35_gated_delta(const void *input, const void *conv_weight, const void *recurrent_a,
                        const void *dt_bias, const void *norm_w, void *output, float *conv_state,
                        float *rec_state, void *workspace, std::size_t workspace_bytes,
                        GatedDeltaShape shape, RaftInferDataType dtype,
                        RaftInferDataType weight_dtype, hipStream_t stream) {
  qwen35_gated_delta(input, conv_weight, recurrent_a, dt_bias, norm_w, output, conv_state,
                     rec_state, workspace, workspace_bytes, shape,
                     qwen35_gated_delta_select_policy(shape, shape.tokens), dtype, weight_dtype,
                     stream);
}

namespace {
// Validation of everything but the input rows, in the reference's order
// (cpp/kernels/qwen35_delta.cu:811-897); `check_inputs` runs where the
// reference checks its input pointer and its alignment.
template <typename InputCheck, typename AlignCheck>
CheckedShape validate_call(InputCheck check_inputs, AlignCheck align_inputs, const void *conv_weight,
                           const void *recurrent_a, const void *dt_bias, const void *norm_w,
                           const void *output, const float *conv_state, const float *rec_state,
                           const void *workspace, std::size_t workspace_bytes,
                           const GatedDeltaShape &shape, const GatedDeltaLaunchPolicy &policy,
                           RaftInferDataType dtype, RaftInferDataType weight_dtype,
                           hipStream_t stream) {
  const CheckedShape c = validate_shape(shape);
  validate_policy(policy, shape);
  require_dtype(dtype);
  require_weight_dtype(dtype, weight_dtype);
  check_inputs();
  require<Err>(conv_weight != nullptr, "gated-delta convolution weight pointer is null");
  require<Err>(recurrent_a != nullptr, "gated-delta recurrent coefficient pointer is null");
  require<Err>(dt_bias != nullptr, "gated-delta dt-bias pointer is null");
  require<Err>(norm_w != nullptr, "gated-delta output norm weight pointer is null");
  require<Err>(output != nullptr, "gated-delta output pointer is null");
  require<Err>(c.convolution_elements == 0 || conv_state != nullptr,
               "gated-delta convolution state pointer is null");
  require<Err>(c.recurrent_elements == 0 || rec_state != nullptr,
               "gated-delta recurrent state pointer is null");
  require<Err>(workspace != nullptr, "gated-delta workspace pointer is null");
  require<Err>(workspace_bytes >= c.workspace_bytes, "gated-delta workspace is too small");
  const std::size_t da = dtype == RAFTINFER_DTYPE_F32 ? 4 : 2;
  const std::size_t wa = weight_dtype == RAFTINFER_DTYPE_F32 ? 4 : 2;
  align_inputs(da);
  require_aligned(conv_weight, wa, "gated-delta convolution weight is not dtype-aligned");
  require_aligned(recurrent_a, wa, "gated-delta recurrent coefficient is not dtype-aligned");
  require_aligned(dt_bias, wa, "gated-delta dt-bias weight is not dtype-aligned");
  require_aligned(norm_w, wa, "gated-delta output norm weight is not dtype-aligned");
  require_aligned(output, da, "gated-delta output is not dtype-aligned");
  require_aligned(workspace, 4, "gated-delta workspace is not float-aligned");
  require_aligned(rec_state, 4, "gated-delta recurrent state is not float-aligned");
  if (c.convolution_elements != 0)
    require_aligned(conv_state, 4, "gated-delta convolution state is not float-aligned");
  require<Err>(stream != nullptr, "HIP stream is null");
  // Register recurrence keeps at most 32 rows per lane across 8 waves.
  require<Err>(shape.key_dim <= kRecWaves * 32, "gated-delta key_dim above 256 is not supported");
  return c;
}

void dispatch(const DeltaSources &src, const void *conv_weight, const void *recurrent_a,
              const void *dt_bias, const void *norm_w, void *output, float *conv_state,
              float *rec_state, void *workspace, const GatedDeltaShape &shape, const CheckedShape &c,
              const GatedDeltaLaunchPolicy &policy, RaftInferDataType dtype,
              RaftInferDataType weight_dtype, hipStream_t stream) {
  auto *ws = static_cast<float *>(workspace);
  if (dtype == RAFTINFER_DTYPE_F32)
    launch_for_weights<float>(weight_dtype, src, conv_weight, recurrent_a, dt_bias, norm_w, output,
                              conv_state, rec_state, ws, shape, c, policy, stream);
  else if (dtype == RAFTINFER_DTYPE_F16)
    launch_for_weights<_Float16>(weight_dtype, src, conv_weight, recurrent_a, dt_bias, norm_w,
                                 output, conv_state, rec_state, ws, shape, c, policy, stream);
  else
    launch_for_weights<bf16_bits>(weight_dtype, src, conv_weight, recurrent_a, dt_bias, norm_w,
                                  output, conv_state, rec_state, ws, shape, c, policy, stream);
}
} // namespace

// Validation order and messages: cpp/kernels/qwen35_delta.cu:811-897.
void qwen35_gated_delta(const void *input, const void *conv_weight, const void *recurrent_a,
                        const void *dt_bias, const void *norm_w, void *output, float *conv_state,
                        float *rec_state, void *workspace, std::size_t workspace_bytes,
                        GatedDeltaShape shape, GatedDeltaLaunchPolicy policy,
                        RaftInferDataType dtype, RaftInferDataType weight_dtype,
                        hipStream_t stream) {
  const CheckedShape c = validate_call(
      [&] { require<Err>(input != nullptr, "gated-delta input pointer is null"); },
      [&](std::size_t da) { require_aligned(input, da, "gated-delta input is not dtype-aligned"); },
      conv_weight, recurrent_a, dt_bias, norm_w, output, conv_state, rec_state, workspace,
      workspace_bytes, shape, policy, dtype, weight_dtype, stream);
  // The packed row [q k v | b | a | z] (cpp/kernels/qwen35_delta.cuh:77-86).
  const std::size_t es = dtype == RAFTINFER_DTYPE_F32 ? 4 : 2;
  const auto *base = static_cast<const unsigned char *>(input);
  const DeltaSources src{base, c.token_stride,
                         base + c.conv_dim * es, c.token_stride,
                         base + (c.conv_dim + shape.value_heads) * es, c.token_stride,
                         base + (c.conv_dim + 2 * shape.value_heads) * es, c.token_stride};
  dispatch(src, conv_weight, recurrent_a, dt_bias, norm_w, output, conv_state, rec_state, workspace,
           shape, c, policy, dtype, weight_dtype, stream);
}

void qwen35_gated_delta_unpacked(const void *qkv, const void *beta, const void *alpha,
                                 const void *gate, const void *conv_weight, const void *recurrent_a,
                                 const void *dt_bias, const void *norm_w, void *output,
                                 float *conv_state, float *rec_state, void *workspace,
                                 std::size_t workspace_bytes, GatedDeltaShape shape,
                                 GatedDeltaLaunchPolicy policy, RaftInferDataType dtype,
                                 RaftInferDataType weight_dtype, hipStream_t stream) {
  const CheckedShape c = validate_call(
      [&] {
        // the pack's own pointer checks (cpp/kernels/qwen35_primitives.cu:768-800)
        require<Err>(qkv != nullptr, "gated-delta qkv pointer is null");
        require<Err>(beta != nullptr, "gated-delta beta pointer is null");
        require<Err>(alpha != nullptr, "gated-delta alpha pointer is null");
        require<Err>(gate != nullptr, "gated-delta gate pointer is null");
      },
      [&](std::size_t da) {
        require_aligned(qkv, da, "gated-delta qkv is not dtype-aligned");
        require_aligned(beta, da, "gated-delta beta is not dtype-aligned");
        require_aligned(alpha, da, "gated-delta alpha is not dtype-aligned");
        require_aligned(gate, da, "gated-delta gate is not dtype-aligned");
      },
      conv_weight, recurrent_a, dt_bias, norm_w, output, conv_state, rec_state, workspace,
      workspace_bytes, shape, policy, dtype, weight_dtype, stream);
  // The projection outputs, each [tokens][width]: qkv conv_dim wide, beta and
  // alpha value_heads wide, gate hidden_size wide.
  const DeltaSources src{qkv, c.conv_dim, beta, shape.value_heads, alpha, shape.value_heads,
                         gate, shape.hidden_size};
  dispatch(src, conv_weight, recurrent_a, dt_bias, norm_w, output, conv_state, rec_state, workspace,
           shape, c, policy, dtype, weight_dtype, stream);
}

// ------------------------------------------------------- core-only entry
std::size_t qwen35_gated_delta_core_workspace_bytes(GatedDeltaCoreShape s) {
  require<Err>(s.tokens > 0 && s.key_heads > 0 && s.value_heads > 0 && s.key_dim > 0 && s.value_dim > 0,
               "gated-delta core shape must be positive");
  return chunk_record_bytes(s.tokens, s.value_heads, s.key_dim, s.value_dim, rec2::kBytes);
}

void qwen35_gated_delta_core(const void *q, const void *k, const void *v, const float *beta,
                             const float *log_decay, float q_scale, float *state, void *output,
                             void *workspace, std::size_t workspace_bytes, GatedDeltaCoreShape s,
                             bool chunked, hipStream_t stream) {
  require<Err>(q && k && v && beta && log_decay && state && output, "gated-delta core pointer is null");
  require<Err>(stream != nullptr, "HIP stream is null");
  require<Err>(s.value_heads % s.key_heads == 0, "gated-delta value_heads must be divisible by key_heads");
  require<Err>(s.key_dim <= kRecWaves * 32, "gated-delta key_dim above 256 is not supported");
  require<Err>(s.value_heads <= 65535 && s.tokens <= 0x7FFFFFFF, "gated-delta core grid overflow");
  if (chunked) {
    require<Err>(s.key_dim == kChunkDim && s.value_dim == kChunkDim,
                 "chunked gated-delta requires key_dim = value_dim = 128");
    require<Err>(((reinterpret_cast<std::uintptr_t>(q) | reinterpret_cast<std::uintptr_t>(k) |
                   reinterpret_cast<std::uintptr_t>(v) | reinterpret_cast<std::uintptr_t>(workspace)) &
                  15u) == 0,
                 "chunked gated-delta needs 16-byte aligned q, k, v and workspace");
    require<Err>(workspace != nullptr && workspace_bytes >= qwen35_gated_delta_core_workspace_bytes(s),
                 "gated-delta core workspace is too small");
  }
  const Src<bf16_bits> qs{static_cast<const bf16_bits *>(q), s.key_heads * s.key_dim, s.key_dim, q_scale};
  const Src<bf16_bits> ks{static_cast<const bf16_bits *>(k), s.key_heads * s.key_dim, s.key_dim, 1.0f};
  const Src<bf16_bits> vs{static_cast<const bf16_bits *>(v), s.value_heads * s.value_dim, s.value_dim, 1.0f};
  ChunkScratch scratch{};
  if (chunked) {
    scratch.rec = static_cast<unsigned char *>(workspace);
    scratch.chunks = ceil_div_unchecked(s.tokens, kChunk);
    scratch.bytes = rec2::kBytes;
  }
  launch_recurrence<bf16_bits, bf16_bits>(qs, ks, vs, beta, log_decay, state,
                                          static_cast<bf16_bits *>(output), scratch, s.tokens,
                                          s.key_heads, s.value_heads, s.key_dim, s.value_dim,
                                          chunked, stream);
}

} // namespace raftinfer::kernels
