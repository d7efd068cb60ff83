// Causal gated GQA prefill attention for the Qwen3.5 signature (16 query
// heads, 4 KV heads, head_dim 256) on gfx950 bf16 MFMA.
//
// Workgroup = 4 waves = one KV head x a 32-token query tile; wave w computes
// query head 4*kv_head + w, so every K/V tile staged in LDS serves the four
// heads of the GQA group.  Per 32-key tile and wave:
//   S^T = K Q^T      16 x v_mfma_f32_32x32x16_bf16 (K row-major in LDS, Q in VGPRs)
//                    -> lane l owns query l%32 and 16 of its 32 keys, so the row
//                    max is 15 in-register maxes plus one lane exchange;
//   online softmax   exp2 domain; the running max only moves when a row max
//                    grows by more than 2^8 (lazy rescaling), so the 128-register
//                    O rescale is rare;
//   O^T += V^T P^T   16 x v_mfma_f32_32x32x16_bf16: P^T stays in VGPRs as the B
//                    operand; its key order is the S^T accumulator order, and
//                    the V^T operand (V transposed in LDS) is read in that same
//                    permuted key order, so P needs no LDS round trip.
// The next tile's K/V loads are issued before the current tile's math.  The
// sigmoid gate is applied in the epilogue; tiles past the causal diagonal are
// skipped and the diagonal tile is masked per element.
#include "decode_scan.hpp"
#include "prefill_mfma.hpp"

namespace raftinfer::amd {
namespace {

constexpr int kQTile = 32;
constexpr int kKTile = 32;
constexpr int kKStride = kHeadDim + 8; // bf16 per K row in LDS (528 B)
constexpr int kVStride = kKTile + 4;   // bf16 per transposed V row (72 B)
constexpr float kLazyRescale = 8.0f;   // log2 units

struct PrefillShared {
  // K tile; reused by the epilogue as 4 x [32][33] fp32 output staging.
  bf16_bits k[kKTile][kKStride];
  bf16_bits vt[kHeadDim][kVStride];
};

__device__ __forceinline__ bf16x8 lds_b128(const bf16_bits *p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(p));
}

__device__ __forceinline__ std::uint32_t cvt_pk_bf16(float lo, float hi) {
  return static_cast<std::uint32_t>(f32_to_bf16(lo)) |
         (static_cast<std::uint32_t>(f32_to_bf16(hi)) << 16);
}

__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

__global__ __launch_bounds__(256) void prefill_mfma_kernel(
    const bf16_bits *__restrict__ query, const bf16_bits *__restrict__ gate,
    bf16_bits *__restrict__ output, const bf16_bits *__restrict__ cache, std::size_t tokens,
    std::size_t max_ctx, std::size_t past, bool head_major) {
  __shared__ PrefillShared sh;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int col = lane & 31;  // query column of S^T / O^T
  const int half = lane >> 5; // k-half of the operands
  const std::size_t qtile = gridDim.x - 1 - blockIdx.x; // longest tiles first
  const std::size_t kv_head = blockIdx.y;
  const std::size_t head = kv_head * kGroup + wave;
  const std::size_t t0 = qtile * kQTile;
  const std::size_t q_rows = tokens - t0 < kQTile ? tokens - t0 : kQTile;
  const std::size_t key_end = past + t0 + q_rows;
  const std::size_t plane = max_ctx * kKvHeads * kHeadDim;
  const float scale = kLog2e / 16.0f;
  const std::size_t my_qpos = past + t0 + col;

  // Q as the B operand: lane holds query `col`, dims kb*16 + half*8 .. +8.
  bf16x8 qb[16];
  {
    // Query rows past the tile's end read the last row; they are never stored.
    const std::size_t qr = static_cast<std::size_t>(col) < q_rows ? col : q_rows - 1;
    const bf16_bits *qrow = query + ((t0 + qr) * kQueryHeads + head) * kHeadDim + half * 8;
#pragma unroll
    for (int kb = 0; kb < 16; ++kb)
      qb[kb] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(qrow + kb * 16));
  }

  floatx16 o[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) o[nb] = floatx16{};
  float m_run = -INFINITY; // running max of query `col` (exp2 domain)
  float l_run = 0.f;       // partial sum over this lane's keys

  // Staging map: thread -> keys 4*kg .. 4*kg+3, dims 8*db .. 8*db+7; kg varies
  // fastest inside a wave so each load instruction covers 8 full 128-byte lines.
  const int kg = tid & 7;
  const int db = tid >> 3;
  u32x4 kc[4], vc[4];
  auto load_tile = [&](std::size_t k0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // Keys past key_end read row key_end-1 (in bounds); their scores are
      // masked to -inf, so no branch splits the batch of loads.
      std::size_t key = k0 + 4 * kg + j;
      key = key < key_end ? key : key_end - 1;
      const std::size_t row = cache_row(head_major, key, kv_head, max_ctx) + 8 * db;
      kc[j] = *reinterpret_cast<const u32x4 *>(cache + row);
      vc[j] = *reinterpret_cast<const u32x4 *>(cache + plane + row);
    }
  };
  load_tile(0);

  for (std::size_t k0 = 0; k0 < key_end; k0 += kKTile) {
    __syncthreads(); // previous tile fully consumed
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<u32x4 *>(&sh.k[4 * kg + j][8 * db]) = kc[j];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int word = e >> 1;
      const int shift = (e & 1) * 16;
      const std::uint32_t v0 = (vc[0][word] >> shift) & 0xFFFFu, v1 = (vc[1][word] >> shift) & 0xFFFFu;
      const std::uint32_t v2 = (vc[2][word] >> shift) & 0xFFFFu, v3 = (vc[3][word] >> shift) & 0xFFFFu;
      *reinterpret_cast<u32x2 *>(&sh.vt[8 * db + e][4 * kg]) = u32x2{v0 | (v1 << 16), v2 | (v3 << 16)};
    }
    __syncthreads();
    if (k0 + kKTile < key_end) load_tile(k0 + kKTile); // prefetch the next tile

    // S^T = K Q^T: rows = keys, column = query `col`.
    floatx16 s = floatx16{};
#pragma unroll
    for (int kb = 0; kb < 16; ++kb)
      s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lds_b128(&sh.k[col][kb * 16 + half * 8]), qb[kb],
                                                  s, 0, 0, 0);

    // Key of accumulator register i: 8*(i/4) + half*4 + i%4.
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const std::size_t key = k0 + (i >> 2) * 8 + half * 4 + (i & 3);
      s[i] = (key > my_qpos || key >= key_end) ? -INFINITY : s[i] * scale;
      mx = fmaxf(mx, s[i]);
    }
    mx = fmaxf(mx, xor32(mx));
    // Lazy rescale: move the reference max only when it grows by > 2^8.
    const bool grow = mx > m_run + kLazyRescale;
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
      const float m_new = grow ? mx : m_run;
      const float sc = fexp2(m_run - m_new); // -inf -> 0 on the first tile
      l_run *= sc;
#pragma unroll
      for (int nb = 0; nb < 8; ++nb)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[nb][i] *= sc;
      m_run = m_new;
    }
    u32x4 pw[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      float p[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        p[j] = fexp2(s[8 * kb + j] - m_run);
        l_run += p[j];
      }
      pw[kb] = u32x4{cvt_pk_bf16(p[0], p[1]), cvt_pk_bf16(p[2], p[3]), cvt_pk_bf16(p[4], p[5]),
                     cvt_pk_bf16(p[6], p[7])};
    }
    // O^T += V^T P^T.  k-slot (kb, j) of this lane <-> key
    // 16kb + 4*half + j (j < 4) and 16kb + 8 + 4*half + (j-4) (j >= 4).
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bf16_bits *vrow = &sh.vt[nb * 32 + col][16 * kb + 4 * half];
        const u32x2 lo = *reinterpret_cast<const u32x2 *>(vrow);
        const u32x2 hi = *reinterpret_cast<const u32x2 *>(vrow + 8);
        const bf16x8 a = __builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
        o[nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, __builtin_bit_cast(bf16x8, pw[kb]),
                                                        o[nb], 0, 0, 0);
      }
    }
  }

  // Epilogue: O^T register i of block nb = dim nb*32 + 8*(i/4) + half*4 + i%4
  // of query `col`.  Each 32x32 block goes through LDS so gate reads and output
  // writes are row-contiguous (lane pair -> one query's 32 dims).
  const float l = l_run + xor32(l_run);
  const float inv = 1.0f / l;
  __syncthreads(); // every wave is done with sh.k
  float(*buf)[33] = reinterpret_cast<float(*)[33]>(&sh.k[0][0]) + wave * 32;
  const int qq = lane >> 1;
  const int d0 = (lane & 1) * 16;
  const bool row_ok = static_cast<std::size_t>(qq) < q_rows;
  const std::size_t base = ((t0 + qq) * kQueryHeads + head) * kHeadDim;
  // All gate loads are issued before the first block so their latency overlaps.
  u32x4 gv[8][2];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) {
    const std::size_t idx = base + nb * 32 + d0;
    const std::size_t gidx = row_ok ? idx : nb * 32 + d0 + ((t0 * kQueryHeads + head) * kHeadDim);
    gv[nb][0] = *reinterpret_cast<const u32x4 *>(gate + gidx);
    gv[nb][1] = *reinterpret_cast<const u32x4 *>(gate + gidx + 8);
  }
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) {
#pragma unroll
    for (int i = 0; i < 16; ++i) buf[col][(i >> 2) * 8 + half * 4 + (i & 3)] = o[nb][i] * inv;
    wave_lds_order();
    if (row_ok) {
      const std::size_t idx = base + nb * 32 + d0;
      u32x4 w0, w1;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        w0[e] = cvt_pk_bf16(buf[qq][d0 + 2 * e] * sigmoid_gate(bf16_lo(gv[nb][0][e])),
                            buf[qq][d0 + 2 * e + 1] * sigmoid_gate(bf16_hi(gv[nb][0][e])));
        w1[e] = cvt_pk_bf16(buf[qq][d0 + 8 + 2 * e] * sigmoid_gate(bf16_lo(gv[nb][1][e])),
                            buf[qq][d0 + 8 + 2 * e + 1] * sigmoid_gate(bf16_hi(gv[nb][1][e])));
      }
      *reinterpret_cast<u32x4 *>(output + idx) = w0;
      *reinterpret_cast<u32x4 *>(output + idx + 8) = w1;
    }
    wave_lds_order();
  }
}

} // namespace

void launch_prefill_mfma(const bf16_bits *q, const bf16_bits *gate, bf16_bits *out,
                         const bf16_bits *cache, std::size_t tokens, std::size_t max_ctx,
                         std::size_t past, bool head_major, hipStream_t stream) {
  const dim3 grid{static_cast<unsigned>(ceil_div_unchecked(tokens, kQTile)), kKvHeads, 1};
  prefill_mfma_kernel<<<grid, 256, 0, stream>>>(q, gate, out, cache, tokens, max_ctx, past,
                                                head_major);
}

} // namespace raftinfer::amd
