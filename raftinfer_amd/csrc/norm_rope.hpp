// Per-head RMSNorm + NeoX partial RoPE of a 256-dim head vector, shared by the
// producer kernels (qwen35_qk_norm_rope, qwen35_split_query_gate_norm_rope)
// and the attention kernels that apply it to q and k themselves, so the fused
// and the separate paths compute bit-identical vectors
// (cpp/kernels/qwen35_primitives.cu:158-210, cpp/reference/qwen35.cpp:169-186).
#pragma once

#include "common.hpp"

namespace raftinfer::amd {

// cos / sin of rotation pair p at `position`: inv_freq_p = ratio^p with
// ratio = base^(-2/rotary_dim) (one double pow on the host), theta =
// position * inv_freq_p reduced modulo 2 pi in double, then a float sincos of
// the reduced angle.
__device__ __forceinline__ void rope_cos_sin(int p, std::size_t position, double ratio, float &cs,
                                             float &sn) {
  double inv = 1.0, bsq = ratio;
  for (int e = p; e != 0; e >>= 1, bsq *= bsq)
    if (e & 1) inv *= bsq;
  const double theta = static_cast<double>(position) * inv;
  constexpr double kTwoPi = 6.283185307179586476925286766559;
  const double t = theta - kTwoPi * rint(theta / kTwoPi);
  sincosf(static_cast<float>(t), &sn, &cs);
}

// Lane l of a wave owns dims 4l .. 4l+3 of one head vector: x (raw) -> v =
// RoPE(x / rms(x) * w).  rot holds cos[pairs] then sin[pairs] (pairs =
// rotary_dim / 2, rotary_dim a multiple of 8); the partner of dims 4l.. sits
// in lane l +- pairs/4.  Every lane of the wave must call it (wave reduction,
// lane shuffle).
__device__ __forceinline__ void norm_rope_256_lane(const float (&x)[4], const float (&w)[4], int lane,
                                                   int pairs, const float *rot, float epsilon,
                                                   float (&v)[4]) {
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) ss = fmaf(x[e], x[e], ss);
  ss = wave_sum(ss);
  const float scale = 1.0f / sqrtf(ss * (1.0f / 256.0f) + epsilon);
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = x[e] * scale * w[e];
  const int d0 = 4 * lane;
  const int shift = pairs / 4; // lanes between a dim and its partner
  const bool rotated = d0 < 2 * pairs, first = d0 < pairs;
  const int src_lane = first ? lane + shift : lane - shift;
  float pv[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) pv[e] = __shfl(v[e], src_lane);
  if (rotated) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int p = first ? d0 + e : d0 + e - pairs;
      const float c = rot[p], sn = rot[pairs + p];
      v[e] = first ? v[e] * c - pv[e] * sn : pv[e] * sn + v[e] * c;
    }
  }
}

// Sliced form of norm_rope_256_lane for rotary pairs a multiple of 32: eight
// consecutive lanes hold one row, lane g of the row (g = lane % 8) owning dims
// 32g .. 32g+31 in x (raw) and w (weights).  The sum of squares is formed as
// the same tree of additions the lane-wise form builds across 64 lanes: per
// 4 dims an fma chain, then pairwise sums of neighbouring partials in dim
// order (three levels in the lane, three by DPP over the row's lanes); each
// level adds the same two operands, so v is bit-identical to the lane-wise
// result.  The RoPE partner of a dim sits in lane g +- pairs / 32 at the same
// offset.  rot: cos[pairs] then sin[pairs] of the row's position (16-byte
// aligned).  Every lane of the wave must call it.
__device__ __forceinline__ void norm_rope_256_slice(const float (&x)[32], const float (&w)[32], int g, int pairs,
                                                    const float *rot, float epsilon, float (&v)[32]) {
  float pp[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) s = fmaf(x[4 * k + e], x[4 * k + e], s);
    pp[k] = s;
  }
  float ss = ((pp[0] + pp[1]) + (pp[2] + pp[3])) + ((pp[4] + pp[5]) + (pp[6] + pp[7]));
  ss += dpp<kDppXor1>(ss);
  ss += dpp<kDppXor2>(ss);
  ss += dpp<kDppHalfMirror>(ss);
  const float scale = 1.0f / sqrtf(ss * (1.0f / 256.0f) + epsilon);
#pragma unroll
  for (int i = 0; i < 32; ++i) v[i] = x[i] * scale * w[i];
  const int pg = pairs / 32; // lane groups between a dim and its partner
  const bool rotated = g < 2 * pg, first = g < pg;
  // Partner lane: g xor 1 (pg = 1) or g xor 2 (pg = 2) among the row's lanes,
  // by DPP; other widths through the LDS crossbar.
  float pv[32];
  if (pg == 1) {
#pragma unroll
    for (int i = 0; i < 32; ++i) pv[i] = dpp<kDppXor1>(v[i]);
  } else if (pg == 2) {
#pragma unroll
    for (int i = 0; i < 32; ++i) pv[i] = dpp<kDppXor2>(v[i]);
  } else {
    const int lane = threadIdx.x & 63;
    const int src_lane = first ? lane + pg : lane - pg;
#pragma unroll
    for (int i = 0; i < 32; ++i) pv[i] = __shfl(v[i], src_lane);
  }
  if (rotated) {
    // cos and sin of pairs p0 .. p0+31, read as 16 vectors before any is used.
    const int p0 = 32 * (first ? g : g - pg);
    float4 cs4[8], sn4[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      cs4[k] = reinterpret_cast<const float4 *>(rot + p0)[k];
      sn4[k] = reinterpret_cast<const float4 *>(rot + pairs + p0)[k];
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const float4 &c4 = cs4[i >> 2], &s4 = sn4[i >> 2];
      const float c = (i & 3) == 0 ? c4.x : (i & 3) == 1 ? c4.y : (i & 3) == 2 ? c4.z : c4.w;
      const float sn = (i & 3) == 0 ? s4.x : (i & 3) == 1 ? s4.y : (i & 3) == 2 ? s4.z : s4.w;
      v[i] = first ? v[i] * c - pv[i] * sn : pv[i] * sn + v[i] * c;
    }
  }
}

// 32 bf16 (four 16-byte pieces) <-> floats, in order.
__device__ __forceinline__ void unpack_bf16x32(const u32x4 (&raw)[4], float (&x)[32]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const std::uint32_t b[4] = {raw[j][0], raw[j][1], raw[j][2], raw[j][3]};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[8 * j + 2 * e] = bf16_lo(b[e]);
      x[8 * j + 2 * e + 1] = bf16_hi(b[e]);
    }
  }
}
__device__ __forceinline__ void pack_bf16x32(const float (&v)[32], u32x4 (&out)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j)
    out[j] = u32x4{pack_bf16x2(v[8 * j], v[8 * j + 1]), pack_bf16x2(v[8 * j + 2], v[8 * j + 3]),
                   pack_bf16x2(v[8 * j + 4], v[8 * j + 5]), pack_bf16x2(v[8 * j + 6], v[8 * j + 7])};
}

// Weights of dims 32g .. 32g+31 from a 256-entry f32 or bf16 array (global
// memory or LDS, 16-byte aligned).
__device__ __forceinline__ void load_slice_weights(const void *weight, bool weight_f32, int g, float (&w)[32]) {
  if (weight_f32) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float4 t = reinterpret_cast<const float4 *>(weight)[8 * g + k];
      w[4 * k] = t.x; w[4 * k + 1] = t.y; w[4 * k + 2] = t.z; w[4 * k + 3] = t.w;
    }
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const u32x4 t = reinterpret_cast<const u32x4 *>(weight)[4 * g + k];
      const std::uint32_t b[4] = {t[0], t[1], t[2], t[3]};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        w[8 * k + 2 * e] = bf16_lo(b[e]);
        w[8 * k + 2 * e + 1] = bf16_hi(b[e]);
      }
    }
  }
}

} // namespace raftinfer::amd
