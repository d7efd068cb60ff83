// Producers of the attention and delta kernels for gfx950: the query/gate
// split of the q projection, the per-head RMSNorm + NeoX partial RoPE of q and
// k, and the packing of the delta layer's input rows
// (cpp/kernels/qwen35_primitives.cu:158-210, :366-420, host :574-623, :743-800).
//
// norm_rope_kernel: one workgroup per token.  Threads first compute the
// rotation (cos, sin) of every pair for the token's position in double
// precision (as cpp/reference/qwen35.cpp:169-186 does) into LDS; then each
// wave takes one (token, head) vector at a time: sum of squares by lane
// partials and a wave reduction, scale = 1/sqrt(mean + eps), and each lane
// writes its dims d = lane, lane + 64, ... with the rotation applied to
// d < rotary_dim (partner d +- rotary_dim/2).  The same kernel reads the
// query half of a [heads][2][head_dim] q projection and copies the gate half
// for the fused split.
#include "common.hpp"
#include "norm_rope.hpp"
#include "raftinfer_amd/qwen35_primitives.hpp"

#include <cmath>
#include <limits>

namespace raftinfer::kernels {
namespace {

using namespace raftinfer::amd;
using Err = Qwen35PrimitiveError;

constexpr int kNormThreads = 256;

template <typename T, typename Wt>
__global__ __launch_bounds__(kNormThreads) void norm_rope_kernel(
    const T *__restrict__ input, const Wt *__restrict__ weight, T *__restrict__ output,
    T *__restrict__ gate, std::size_t heads, std::size_t head_dim, std::size_t in_stride,
    std::size_t rotary_dim, std::size_t position_offset, float rope_base, float epsilon,
    const std::uint32_t *device_position) {
  extern __shared__ float rot[]; // [pairs] cos then [pairs] sin
  const std::size_t token = blockIdx.x;
  const std::size_t pairs = rotary_dim / 2;
  const std::size_t position =
      (device_position != nullptr ? static_cast<std::size_t>(*device_position) : position_offset) + token;
  for (std::size_t p = threadIdx.x; p < pairs; p += kNormThreads) {
    const double exponent = static_cast<double>(2 * p) / static_cast<double>(rotary_dim);
    const double theta = static_cast<double>(position) / pow(static_cast<double>(rope_base), exponent);
    rot[p] = static_cast<float>(cos(theta));
    rot[pairs + p] = static_cast<float>(sin(theta));
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (std::size_t h = wave; h < heads; h += kNormThreads / 64) {
    const T *src = input + (token * heads + h) * in_stride;
    T *dst = output + (token * heads + h) * head_dim;
    float ss = 0.f;
    for (std::size_t d = lane; d < head_dim; d += 64) {
      const float x = Elem<T>::load(src, d);
      ss = fmaf(x, x, ss);
    }
    ss = wave_sum(ss);
    const float scale = 1.0f / sqrtf(ss / static_cast<float>(head_dim) + epsilon);
    for (std::size_t d = lane; d < head_dim; d += 64) {
      float v = Elem<T>::load(src, d) * scale * Elem<Wt>::load(weight, d);
      if (d < rotary_dim) {
        const bool first = d < pairs;
        const std::size_t p = first ? d : d - pairs;
        const std::size_t partner = first ? d + pairs : p;
        const float w = Elem<T>::load(src, partner) * scale * Elem<Wt>::load(weight, partner);
        const float c = rot[p], s = rot[pairs + p];
        v = first ? v * c - w * s : w * s + v * c;
      }
      Elem<T>::store(dst, d, v);
    }
    if (gate != nullptr) {
      T *gdst = gate + (token * heads + h) * head_dim;
      for (std::size_t d = lane; d < head_dim; d += 64) gdst[d] = src[head_dim + d];
    }
  }
}

// Vector of 4 consecutive elements.
template <typename T> struct Vec4;
template <> struct Vec4<bf16_bits> {
  using Raw = u32x2;
  static __device__ __forceinline__ void load(const bf16_bits *p, float (&v)[4]) {
    const u32x2 w = *reinterpret_cast<const u32x2 *>(p);
    v[0] = bf16_lo(w[0]); v[1] = bf16_hi(w[0]); v[2] = bf16_lo(w[1]); v[3] = bf16_hi(w[1]);
  }
  static __device__ __forceinline__ void store(bf16_bits *p, const float (&v)[4]) {
    *reinterpret_cast<u32x2 *>(p) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  }
};
template <> struct Vec4<float> {
  static __device__ __forceinline__ void load(const float *p, float (&v)[4]) {
    const float4 w = *reinterpret_cast<const float4 *>(p);
    v[0] = w.x; v[1] = w.y; v[2] = w.z; v[3] = w.w;
  }
  static __device__ __forceinline__ void store(float *p, const float (&v)[4]) {
    *reinterpret_cast<float4 *>(p) = make_float4(v[0], v[1], v[2], v[3]);
  }
};
template <> struct Vec4<_Float16> {
  static __device__ __forceinline__ void load(const _Float16 *p, float (&v)[4]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = static_cast<float>(p[e]);
  }
  static __device__ __forceinline__ void store(_Float16 *p, const float (&v)[4]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) p[e] = static_cast<_Float16>(v[e]);
  }
};

// head_dim 256 (the Qwen3.5 attention heads), rotary_dim a multiple of 8:
// lane l owns dims 4l .. 4l+3 of a head vector (whole-row loads and stores);
// the rotation partner of dims 4l.. sits in lane l +- rotary_dim/8 and comes
// over the lane crossbar.  Rotation angles: inv_freq_p = r^p with
// r = base^(-2/rotary_dim) (one double pow on the host, passed in; double
// products here), theta = position * inv_freq_p reduced modulo 2 pi in
// double, then a float sincos of the reduced angle.
template <typename T, typename Wt>
__global__ __launch_bounds__(kNormThreads) void norm_rope_256_kernel(
    const T *__restrict__ input, const Wt *__restrict__ weight, T *__restrict__ output,
    T *__restrict__ gate, std::size_t heads, std::size_t in_stride, std::size_t rotary_dim,
    std::size_t position_offset, double ratio, float epsilon,
    const std::uint32_t *device_position) {
  __shared__ float rot[256]; // [pairs] cos, then [pairs] sin (pairs <= 128)
  constexpr int kWaves = kNormThreads / 64, kBatch = 4;
  const std::size_t token = blockIdx.x;
  const int pairs = static_cast<int>(rotary_dim / 2);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int d0 = 4 * lane;
  // Heads wave, wave + 4, ... in groups of four whose loads are all issued
  // before any is used; the first group's loads go out before the angles are
  // computed.
  float x[kBatch][4], g[kBatch][4], w[4];
  auto load_batch = [&](std::size_t h0) {
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const std::size_t h = h0 + kWaves * b < heads ? h0 + kWaves * b : h0;
      const T *src = input + (token * heads + h) * in_stride;
      Vec4<T>::load(src + d0, x[b]);
      if (gate != nullptr) Vec4<T>::load(src + 256 + d0, g[b]);
    }
  };
  if (static_cast<std::size_t>(wave) < heads) load_batch(wave);
  Vec4<Wt>::load(weight + d0, w);
  if (static_cast<int>(threadIdx.x) < pairs) {
    const int p = threadIdx.x;
    const std::size_t position =
        (device_position != nullptr ? static_cast<std::size_t>(*device_position) : position_offset) + token;
    float cs, sn;
    rope_cos_sin(p, position, ratio, cs, sn);
    rot[p] = cs;
    rot[pairs + p] = sn;
  }
  __syncthreads();
  for (std::size_t h0 = wave; h0 < heads; h0 += kWaves * kBatch) {
    if (h0 != static_cast<std::size_t>(wave)) load_batch(h0);
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const std::size_t h = h0 + kWaves * b;
      if (h >= heads) break; // uniform across the wave
      float v[4];
      norm_rope_256_lane(x[b], w, lane, pairs, rot, epsilon, v);
      Vec4<T>::store(output + (token * heads + h) * 256 + d0, v);
      if (gate != nullptr) Vec4<T>::store(gate + (token * heads + h) * 256 + d0, g[b]);
    }
  }
}

// Pure copy of the two halves of each [2][head_dim] block: 16-byte pieces
// when the rows allow it, elements otherwise.
template <typename E>
__global__ __launch_bounds__(256) void split_kernel(const E *__restrict__ src, E *__restrict__ query,
                                                    E *__restrict__ gate, std::size_t vectors,
                                                    std::size_t row) {
  const std::size_t total = vectors * row;
  for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<std::size_t>(gridDim.x) * 256) {
    const std::size_t v = i / row, e = i - v * row;
    query[i] = src[2 * v * row + e];
    gate[i] = src[2 * v * row + row + e];
  }
}

// Row concatenation: item = (token, segment, piece); 16-byte pieces when every
// width allows it, elements otherwise.
template <typename E>
__global__ __launch_bounds__(256) void pack_kernel(const E *__restrict__ s0, const E *__restrict__ s1,
                                                   const E *__restrict__ s2, const E *__restrict__ s3,
                                                   E *__restrict__ packed, std::size_t tokens,
                                                   std::size_t w0, std::size_t w1, std::size_t w2,
                                                   std::size_t w3) {
  const std::size_t width = w0 + w1 + w2 + w3;
  const std::size_t total = tokens * width;
  for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<std::size_t>(gridDim.x) * 256) {
    const std::size_t t = i / width, c = i - t * width;
    E v;
    if (c < w0)
      v = s0[t * w0 + c];
    else if (c < w0 + w1)
      v = s1[t * w1 + (c - w0)];
    else if (c < w0 + w1 + w2)
      v = s2[t * w2 + (c - w0 - w1)];
    else
      v = s3[t * w3 + (c - w0 - w1 - w2)];
    packed[i] = v;
  }
}

void require_dtype(RaftInferDataType d) {
  require<Err>(d == RAFTINFER_DTYPE_F32 || d == RAFTINFER_DTYPE_F16 || d == RAFTINFER_DTYPE_BF16,
               "unsupported Qwen3.5 primitive dtype");
}

void require_weight_dtype(RaftInferDataType d, RaftInferDataType w) {
  require<Err>(w == d || w == RAFTINFER_DTYPE_F32 ||
                   (d == RAFTINFER_DTYPE_F32 && (w == RAFTINFER_DTYPE_F16 || w == RAFTINFER_DTYPE_BF16)),
               "Qwen3.5 primitive weight dtype is incompatible with activations");
}

// cpp/kernels/qwen35_primitives.cu:580-601 (validation order and messages).
void validate_norm_rope(const void *input, const void *weight, const void *output,
                        const QkNormRopeShape &s, float epsilon, RaftInferDataType dtype,
                        RaftInferDataType wdt, hipStream_t stream) {
  require<Err>(input != nullptr, "qk_norm_rope input pointer is null");
  require<Err>(weight != nullptr, "qk_norm_rope weight pointer is null");
  require<Err>(output != nullptr, "qk_norm_rope output pointer is null");
  require<Err>(s.tokens > 0, "qk_norm_rope tokens must be positive");
  require<Err>(s.heads > 0, "qk_norm_rope heads must be positive");
  require<Err>(s.head_dim > 0, "qk_norm_rope head_dim must be positive");
  require<Err>(s.rotary_dim > 0, "qk_norm_rope rotary_dim must be positive");
  require<Err>(s.rotary_dim <= s.head_dim, "qk_norm_rope rotary_dim exceeds head_dim");
  require<Err>(s.rotary_dim % 2 == 0, "qk_norm_rope rotary_dim must be even");
  require<Err>(std::isfinite(s.rope_base) && s.rope_base > 0.0f,
               "qk_norm_rope rope_base must be finite and positive");
  require<Err>(std::isfinite(epsilon) && epsilon >= 0.0f,
               "qk_norm_rope epsilon must be finite and non-negative");
  require<Err>(s.position_offset <= std::numeric_limits<std::size_t>::max() - (s.tokens - 1),
               "qk_norm_rope position range overflow");
  require<Err>(stream != nullptr, "HIP stream is null");
  require_dtype(dtype);
  require_weight_dtype(dtype, wdt);
  const std::size_t vectors = checked_mul<Err>(s.tokens, s.heads, "qk_norm_rope vector overflow");
  (void)checked_mul<Err>(vectors, s.head_dim, "qk_norm_rope shape overflow");
  require<Err>(s.tokens <= 0x7FFFFFFFu, "qk_norm_rope grid dimension overflow");
  require<Err>(s.rotary_dim / 2 <= 8192, "qk_norm_rope rotary_dim above 16384 is not supported");
}

template <typename T, typename Wt>
void launch_norm_rope(const void *input, const void *weight, void *output, void *gate,
                      std::size_t in_stride, const QkNormRopeShape &s, float epsilon,
                      const std::uint32_t *device_position, hipStream_t stream) {
  const std::size_t vec_bytes = 4 * sizeof(T), wvec_bytes = 4 * sizeof(Wt);
  const auto aligned = [](const void *p, std::size_t a) {
    return p == nullptr || (reinterpret_cast<std::uintptr_t>(p) & (a - 1)) == 0;
  };
  if (s.head_dim == 256 && s.rotary_dim % 8 == 0 && aligned(input, vec_bytes) &&
      aligned(output, vec_bytes) && aligned(gate, vec_bytes) && aligned(weight, wvec_bytes)) {
    norm_rope_256_kernel<T, Wt><<<static_cast<unsigned>(s.tokens), kNormThreads, 0, stream>>>(
        static_cast<const T *>(input), static_cast<const Wt *>(weight), static_cast<T *>(output),
        static_cast<T *>(gate), s.heads, in_stride, s.rotary_dim, s.position_offset,
        std::pow(static_cast<double>(s.rope_base), -2.0 / static_cast<double>(s.rotary_dim)), epsilon,
        device_position);
    return;
  }
  const std::size_t lds = (s.rotary_dim / 2) * 2 * sizeof(float);
  norm_rope_kernel<T, Wt><<<static_cast<unsigned>(s.tokens), kNormThreads, lds, stream>>>(
      static_cast<const T *>(input), static_cast<const Wt *>(weight), static_cast<T *>(output),
      static_cast<T *>(gate), s.heads, s.head_dim, in_stride, s.rotary_dim, s.position_offset,
      s.rope_base, epsilon, device_position);
}

void dispatch_norm_rope(const void *input, const void *weight, void *output, void *gate,
                        std::size_t in_stride, const QkNormRopeShape &s, float epsilon,
                        RaftInferDataType dtype, RaftInferDataType wdt,
                        const std::uint32_t *device_position, hipStream_t stream) {
  auto go = [&]<typename T>() {
    if (wdt == RAFTINFER_DTYPE_F32)
      launch_norm_rope<T, float>(input, weight, output, gate, in_stride, s, epsilon, device_position,
                                 stream);
    else if (wdt == RAFTINFER_DTYPE_F16)
      launch_norm_rope<T, _Float16>(input, weight, output, gate, in_stride, s, epsilon,
                                    device_position, stream);
    else
      launch_norm_rope<T, bf16_bits>(input, weight, output, gate, in_stride, s, epsilon,
                                     device_position, stream);
  };
  if (dtype == RAFTINFER_DTYPE_F32)
    go.operator()<float>();
  else if (dtype == RAFTINFER_DTYPE_F16)
    go.operator()<_Float16>();
  else
    go.operator()<bf16_bits>();
}

} // namespace

void qwen35_qk_norm_rope(const void *input, const void *weight, void *output, QkNormRopeShape shape,
                         float epsilon, RaftInferDataType dtype, RaftInferDataType weight_dtype,
                         hipStream_t stream, const std::uint32_t *device_position) {
  validate_norm_rope(input, weight, output, shape, epsilon, dtype, weight_dtype, stream);
  dispatch_norm_rope(input, weight, output, nullptr, shape.head_dim, shape, epsilon, dtype,
                     weight_dtype, device_position, stream);
  check_launch<Err>("qwen35_qk_norm_rope");
}

void qwen35_split_full_query_gate(const void *query_gate, void *query, void *gate,
                                  std::size_t tokens, std::size_t heads, std::size_t head_dim,
                                  RaftInferDataType dtype, hipStream_t stream) {
  // cpp/kernels/qwen35_primitives.cu:747-761
  require<Err>(query_gate != nullptr, "split_full_query_gate input pointer is null");
  require<Err>(query != nullptr, "split_full_query_gate query pointer is null");
  require<Err>(gate != nullptr, "split_full_query_gate gate pointer is null");
  require<Err>(tokens > 0, "split_full_query_gate tokens must be positive");
  require<Err>(heads > 0, "split_full_query_gate heads must be positive");
  require<Err>(head_dim > 0, "split_full_query_gate head_dim must be positive");
  require<Err>(stream != nullptr, "HIP stream is null");
  require_dtype(dtype);
  const std::size_t hidden = checked_mul<Err>(heads, head_dim, "split_full_query_gate hidden overflow");
  (void)checked_mul<Err>(tokens, hidden, "split_full_query_gate shape overflow");
  const std::size_t es = dtype == RAFTINFER_DTYPE_F32 ? 4 : 2;
  const std::size_t vectors = tokens * heads;
  const std::size_t row_bytes = head_dim * es;
  const bool wide = row_bytes % 16 == 0 &&
                    ((reinterpret_cast<std::uintptr_t>(query_gate) | reinterpret_cast<std::uintptr_t>(query) |
                      reinterpret_cast<std::uintptr_t>(gate)) & 15u) == 0;
  auto grid = [](std::size_t items) {
    return static_cast<unsigned>(std::min<std::size_t>(ceil_div_unchecked(items, 256), 65536));
  };
  if (wide) {
    const std::size_t row = row_bytes / 16;
    split_kernel<u32x4><<<grid(vectors * row), 256, 0, stream>>>(
        static_cast<const u32x4 *>(query_gate), static_cast<u32x4 *>(query), static_cast<u32x4 *>(gate),
        vectors, row);
  } else if (es == 4) {
    split_kernel<std::uint32_t><<<grid(vectors * head_dim), 256, 0, stream>>>(
        static_cast<const std::uint32_t *>(query_gate), static_cast<std::uint32_t *>(query),
        static_cast<std::uint32_t *>(gate), vectors, head_dim);
  } else {
    split_kernel<std::uint16_t><<<grid(vectors * head_dim), 256, 0, stream>>>(
        static_cast<const std::uint16_t *>(query_gate), static_cast<std::uint16_t *>(query),
        static_cast<std::uint16_t *>(gate), vectors, head_dim);
  }
  check_launch<Err>("qwen35_split_full_query_gate");
}

void qwen35_pack_linear_delta_input(const void *qkv, const void *beta, const void *alpha,
                                    const void *gate, void *packed, std::size_t tokens,
                                    std::size_t qkv_width, std::size_t beta_width,
                                    std::size_t alpha_width, std::size_t gate_width,
                                    RaftInferDataType dtype, hipStream_t stream) {
  // cpp/kernels/qwen35_primitives.cu:768-800 (validation order and messages)
  require<Err>(qkv != nullptr, "pack_linear_delta_input qkv pointer is null");
  require<Err>(beta != nullptr, "pack_linear_delta_input beta pointer is null");
  require<Err>(alpha != nullptr, "pack_linear_delta_input alpha pointer is null");
  require<Err>(gate != nullptr, "pack_linear_delta_input gate pointer is null");
  require<Err>(packed != nullptr, "pack_linear_delta_input output pointer is null");
  require<Err>(tokens > 0, "pack_linear_delta_input tokens must be positive");
  require<Err>(qkv_width > 0, "pack_linear_delta_input qkv_width must be positive");
  require<Err>(beta_width > 0, "pack_linear_delta_input beta_width must be positive");
  require<Err>(alpha_width > 0, "pack_linear_delta_input alpha_width must be positive");
  require<Err>(gate_width > 0, "pack_linear_delta_input gate_width must be positive");
  require<Err>(stream != nullptr, "HIP stream is null");
  require_dtype(dtype);
  const std::size_t beta_end = checked_add<Err>(qkv_width, beta_width, "pack_linear_delta_input width overflow");
  const std::size_t alpha_end = checked_add<Err>(beta_end, alpha_width, "pack_linear_delta_input width overflow");
  const std::size_t width = checked_add<Err>(alpha_end, gate_width, "pack_linear_delta_input width overflow");
  (void)checked_mul<Err>(tokens, width, "pack_linear_delta_input shape overflow");
  const std::size_t es = dtype == RAFTINFER_DTYPE_F32 ? 4 : 2;
  const std::uintptr_t addr = reinterpret_cast<std::uintptr_t>(qkv) | reinterpret_cast<std::uintptr_t>(beta) |
                              reinterpret_cast<std::uintptr_t>(alpha) | reinterpret_cast<std::uintptr_t>(gate) |
                              reinterpret_cast<std::uintptr_t>(packed);
  const bool wide = (addr & 15u) == 0 && (qkv_width * es) % 16 == 0 && (beta_width * es) % 16 == 0 &&
                    (alpha_width * es) % 16 == 0 && (gate_width * es) % 16 == 0;
  auto grid = [](std::size_t items) {
    return static_cast<unsigned>(std::min<std::size_t>(ceil_div_unchecked(items, 256), 65536));
  };
  if (wide) {
    const std::size_t k = 16 / es;
    pack_kernel<u32x4><<<grid(tokens * width / k), 256, 0, stream>>>(
        static_cast<const u32x4 *>(qkv), static_cast<const u32x4 *>(beta), static_cast<const u32x4 *>(alpha),
        static_cast<const u32x4 *>(gate), static_cast<u32x4 *>(packed), tokens, qkv_width / k,
        beta_width / k, alpha_width / k, gate_width / k);
  } else if (es == 4) {
    pack_kernel<std::uint32_t><<<grid(tokens * width), 256, 0, stream>>>(
        static_cast<const std::uint32_t *>(qkv), static_cast<const std::uint32_t *>(beta),
        static_cast<const std::uint32_t *>(alpha), static_cast<const std::uint32_t *>(gate),
        static_cast<std::uint32_t *>(packed), tokens, qkv_width, beta_width, alpha_width, gate_width);
  } else {
    pack_kernel<std::uint16_t><<<grid(tokens * width), 256, 0, stream>>>(
        static_cast<const std::uint16_t *>(qkv), static_cast<const std::uint16_t *>(beta),
        static_cast<const std::uint16_t *>(alpha), static_cast<const std::uint16_t *>(gate),
        static_cast<std::uint16_t *>(packed), tokens, qkv_width, beta_width, alpha_width, gate_width);
  }
  check_launch<Err>("qwen35_pack_linear_delta_input");
}

void qwen35_split_query_gate_norm_rope(const void *query_gate, const void *weight, void *query,
                                       void *gate, QkNormRopeShape shape, float epsilon,
                                       RaftInferDataType dtype, RaftInferDataType weight_dtype,
                                       hipStream_t stream, const std::uint32_t *device_position) {
  require<Err>(gate != nullptr, "split_full_query_gate gate pointer is null");
  validate_norm_rope(query_gate, weight, query, shape, epsilon, dtype, weight_dtype, stream);
  (void)checked_mul<Err>(shape.head_dim, 2, "qk_norm_rope shape overflow");
  dispatch_norm_rope(query_gate, weight, query, gate, 2 * shape.head_dim, shape, epsilon, dtype,
                     weight_dtype, device_position, stream);
  check_launch<Err>("qwen35_split_query_gate_norm_rope");
}

} // namespace raftinfer::kernels
