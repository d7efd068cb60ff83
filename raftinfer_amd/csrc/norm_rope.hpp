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

} // namespace raftinfer::amd
