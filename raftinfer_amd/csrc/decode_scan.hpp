// Device core shared by the single-block, split-K and batched decode kernels:
// one workgroup scans a token range of one KV head for NH query heads of its
// GQA group, keeping an online-softmax state per head.
//
// Lane layout (wave64 = 4 row-groups of 16 lanes): row-group g takes one
// token per step, lane r of the group owns dims [8r, 8r+8) and
// [128+8r, 128+8r+8) of the 256-wide head, so one 16-byte load per lane per
// half-row gives each 16-lane group a contiguous 256-byte half of a K or V
// row (full 128-byte lines, coalesced).  q.k partial dots reduce inside the
// 16-lane row with four DPP steps; the softmax runs in the exp2 domain with
// log2(e)/sqrt(D) folded into q.
#pragma once

#include "common.hpp"

namespace raftinfer::amd {

constexpr int kHeadDim = 256;
constexpr int kQueryHeads = 16;
constexpr int kKvHeads = 4;
constexpr int kGroup = kQueryHeads / kKvHeads;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

template <typename T> struct Chunk8;
template <> struct Chunk8<bf16_bits> {
  u32x4 w;
  __device__ __forceinline__ void load(const bf16_bits *p) {
    w = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
  }
  __device__ __forceinline__ void zero() { w = u32x4{0u, 0u, 0u, 0u}; }
  __device__ __forceinline__ float get(int i) const {
    const std::uint32_t x = w[i >> 1];
    return (i & 1) ? bf16_hi(x) : bf16_lo(x);
  }
};
template <> struct Chunk8<float> {
  float4 a, b;
  __device__ __forceinline__ void load(const float *p) {
    a = reinterpret_cast<const float4 *>(p)[0];
    b = reinterpret_cast<const float4 *>(p)[1];
  }
  __device__ __forceinline__ void zero() {
    a = make_float4(0.f, 0.f, 0.f, 0.f);
    b = a;
  }
  __device__ __forceinline__ float get(int i) const {
    switch (i) {
    case 0: return a.x; case 1: return a.y; case 2: return a.z; case 3: return a.w;
    case 4: return b.x; case 5: return b.y; case 6: return b.z; default: return b.w;
    }
  }
};

// Element index of (token, kv_head, dim 0) in one cache plane
// (cpp/kernels/qwen35_online_attention.cu:240-252).
__device__ __forceinline__ std::size_t cache_row(bool head_major, std::size_t token,
                                                 std::size_t kv_head, std::size_t max_ctx) {
  return head_major ? (kv_head * max_ctx + token) * kHeadDim
                    : (token * kKvHeads + kv_head) * kHeadDim;
}

// Per-head combined state after a workgroup scan, staged in LDS.
template <int NH, int WAVES> struct ScanShared {
  float m[WAVES][NH];
  float l[WAVES][NH];
  float acc[WAVES][NH][kHeadDim];
};

// Scans tokens [begin, end) of kv_head for query heads first_head..+NH and
// leaves the per-wave states in `sh`.  Every wave returns after writing its
// slot; the caller synchronizes.
template <typename ActT, typename CacheT, int NH, int WAVES, int U>
__device__ __forceinline__ void scan_range(const ActT *__restrict__ query, std::size_t first_head,
                                           const CacheT *__restrict__ k_plane,
                                           const CacheT *__restrict__ v_plane, bool head_major,
                                           std::size_t max_ctx, std::size_t kv_head,
                                           std::size_t begin, std::size_t end,
                                           ScanShared<NH, WAVES> &sh) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4;
  const int r = lane & 15;
  const float qscale = kLog2e / 16.0f; // log2(e) / sqrt(256)

  float q[NH][16];
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const ActT *qh = query + (first_head + h) * kHeadDim;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      q[h][i] = Elem<ActT>::load(qh, 8 * r + i) * qscale;
      q[h][8 + i] = Elem<ActT>::load(qh, 128 + 8 * r + i) * qscale;
    }
  }

  float m[NH], l[NH], acc[NH][16];
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[h][i] = 0.f;
  }

  constexpr int kTile = 4 * U; // tokens per wave step
  for (std::size_t tile = begin + static_cast<std::size_t>(wave) * kTile; tile < end;
       tile += static_cast<std::size_t>(WAVES) * kTile) {
    Chunk8<CacheT> ka[U], kb[U], va[U], vb[U];
    bool valid[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const std::size_t tok = tile + 4 * u + g;
      valid[u] = tok < end;
      if (valid[u]) {
        const std::size_t row = cache_row(head_major, tok, kv_head, max_ctx) + 8 * r;
        ka[u].load(k_plane + row);
        kb[u].load(k_plane + row + 128);
        va[u].load(v_plane + row);
        vb[u].load(v_plane + row + 128);
      } else {
        ka[u].zero();
        kb[u].zero();
        va[u].zero();
        vb[u].zero();
      }
    }
    float s[NH][U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        float d0 = 0.f, d1 = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          d0 = fmaf(q[h][i], ka[u].get(i), d0);
          d1 = fmaf(q[h][8 + i], kb[u].get(i), d1);
        }
        s[h][u] = row16_sum(d0 + d1);
      }
    }
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      float mt = m[h];
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (valid[u]) mt = fmaxf(mt, s[h][u]);
      const float so = m[h] == -INFINITY ? 0.f : exp2f(m[h] - mt);
      float p[U];
      float psum = 0.f;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        p[u] = valid[u] ? exp2f(s[h][u] - mt) : 0.f;
        psum += p[u];
      }
      l[h] = l[h] * so + psum;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float a0 = acc[h][i] * so, a1 = acc[h][8 + i] * so;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          a0 = fmaf(p[u], va[u].get(i), a0);
          a1 = fmaf(p[u], vb[u].get(i), a1);
        }
        acc[h][i] = a0;
        acc[h][8 + i] = a1;
      }
      m[h] = mt;
    }
  }

  // Combine the four row-groups of the wave (lanes r, r^16, r^32, r^48 own
  // the same dims).
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    float mm = fmaxf(m[h], xor16(m[h]));
    mm = fmaxf(mm, xor32(mm));
    const float w = m[h] == -INFINITY ? 0.f : exp2f(m[h] - mm);
    float lw = l[h] * w;
    lw += xor16(lw);
    lw += xor32(lw);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float a = acc[h][i] * w;
      a += xor16(a);
      a += xor32(a);
      acc[h][i] = a;
    }
    if (lane == 0) {
      sh.m[wave][h] = mm;
      sh.l[wave][h] = lw;
    }
    if (lane < 16) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        sh.acc[wave][h][8 * r + i] = acc[h][i];
        sh.acc[wave][h][128 + 8 * r + i] = acc[h][8 + i];
      }
    }
  }
}

// Merges the per-wave states of `sh` for output element (h, d): returns the
// exp2-domain max, the sum and the unnormalised accumulator.
template <int NH, int WAVES>
__device__ __forceinline__ void combine_waves(const ScanShared<NH, WAVES> &sh, int h, int d,
                                              float &m_out, float &l_out, float &a_out) {
  float mm = -INFINITY;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) mm = fmaxf(mm, sh.m[w][h]);
  float l = 0.f, a = 0.f;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) {
    const float mw = sh.m[w][h];
    const float sc = mw == -INFINITY ? 0.f : exp2f(mw - mm);
    l = fmaf(sh.l[w][h], sc, l);
    a = fmaf(sh.acc[w][h][d], sc, a);
  }
  m_out = mm;
  l_out = l;
  a_out = a;
}

// sigmoid(x) = 1 / (1 + 2^(-x log2 e)) with the hardware exp2 and reciprocal
// (about 1 ulp each; outputs are rounded to bf16 or compared at 1e-2).
__device__ __forceinline__ float sigmoid_gate(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * kLog2e));
}

} // namespace raftinfer::amd
