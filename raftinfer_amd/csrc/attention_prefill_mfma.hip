// Causal gated GQA prefill attention for the Qwen3.5 signature (16 query
// heads, 4 KV heads, head_dim 256) on gfx950 bf16 MFMA.
//
// Workgroup = 8 waves = one KV head x a 32-token query tile, as two key-split
// groups of 4 waves: group g takes key tiles g, g+2, ...; wave w of a group
// computes query head 4*kv_head + w, so every K/V tile staged in LDS serves
// the four heads of the GQA group.  The two groups' partial (max, sum, O)
// are merged through LDS, each group finishing one half of the head dims.  Per 32-key tile and wave:
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
constexpr int kSplits = 2;             // key-split groups per workgroup
constexpr int kThreads = 256 * kSplits;
constexpr int kEpiStride = 128 + 4;   // fp32 per epilogue row

struct StageTile {
  bf16_bits k[kKTile][kKStride];
  bf16_bits vt[kHeadDim][kVStride];
};
struct MainPhase {
  // Q tile of the four heads (the B operand of S^T = K Q^T), shared by both groups.
  bf16_bits q[kGroup][kQTile][kKStride];
  StageTile stage[kSplits];
};
union PrefillShared {
  MainPhase main;
  // Merge: wave w of group g leaves the half of O^T that group 1-g finishes
  // (64 registers, lane-major), with its running max and partial sums.
  struct {
    float o[8][64][64];
    float m[8][64];
    float l[8][64];
  } merge;
  // Epilogue: one [query][128 dims] fp32 tile per wave.
  float epi[8][kQTile][kEpiStride];
};

__device__ __forceinline__ bf16x8 lds_b128(const bf16_bits *p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(p));
}

__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Merge and epilogue of one key-split group; GRP selects the half of the
// head dims it finishes.
template <int GRP>
__device__ __forceinline__ void prefill_tail(floatx16 (&o)[8], float m_run, float l_run,
                                             PrefillShared &sh, const bf16_bits *__restrict__ gate,
                                             bf16_bits *__restrict__ output, std::size_t t0,
                                             std::size_t q_rows, std::size_t head, int wave,
                                             int lane, int col, int half) {
  constexpr int mine = 4 * GRP, theirs = 4 * (1 - GRP), grp = GRP;
  // Gate loads of this lane's output rows are issued before the merge.
  const int rq = lane >> 4;       // query of this lane within a group of 4
  const int c8 = (lane & 15) * 8; // first dim of this lane's 8-dim chunk
  u32x4 gv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    // Rows past the tile's end read the last row; they are never stored.
    const std::size_t qq = 4 * j + rq;
    const std::size_t qr = qq < q_rows ? qq : q_rows - 1;
    gv[j] = *reinterpret_cast<const u32x4 *>(gate + ((t0 + qr) * kQueryHeads + head) * kHeadDim +
                                             128 * grp + c8);
  }
  __syncthreads(); // every wave is done with Q and the stage tiles
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int i = 0; i < 16; ++i) sh.merge.o[wave][nb * 16 + i][lane] = o[theirs + nb][i];
  sh.merge.m[wave][lane] = m_run;
  sh.merge.l[wave][lane] = l_run;
  __syncthreads();
  const int peer = wave ^ 4; // same head, other group
  {
    const float m1 = sh.merge.m[peer][lane];
    const float mm = fmaxf(m_run, m1);
    const float a0 = fexp2(m_run - mm);
    const float a1 = fexp2(m1 - mm);
    l_run = l_run * a0 + sh.merge.l[peer][lane] * a1;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        o[mine + nb][i] = o[mine + nb][i] * a0 + sh.merge.o[peer][nb * 16 + i][lane] * a1;
  }
  const float l = l_run + xor32(l_run);
  const float inv = 1.0f / l; // for query `col`

  // Epilogue: each wave writes its half of O^T (register i of block nb = dim
  // nb*32 + 8*(i/4) + half*4 + i%4 of query `col`) to its own LDS tile
  // [query][dim], then reads it back row-major so every gate load and output
  // store covers whole 256-byte row segments.
  __syncthreads(); // merge buffer consumed
  float(*ot)[kEpiStride] = sh.epi[wave];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const floatx16 &ob = o[mine + nb];
      *reinterpret_cast<float4 *>(&ot[col][nb * 32 + 8 * i4 + half * 4]) =
          make_float4(ob[4 * i4] * inv, ob[4 * i4 + 1] * inv, ob[4 * i4 + 2] * inv,
                      ob[4 * i4 + 3] * inv);
    }
  wave_lds_order();
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const std::size_t qq = 4 * j + rq;
    if (qq < q_rows) {
      const float4 x0 = *reinterpret_cast<const float4 *>(&ot[qq][c8]);
      const float4 x1 = *reinterpret_cast<const float4 *>(&ot[qq][c8 + 4]);
      const u32x4 g = gv[j];
      const u32x4 w{pack_bf16x2(x0.x * sigmoid_gate(bf16_lo(g[0])), x0.y * sigmoid_gate(bf16_hi(g[0]))),
                    pack_bf16x2(x0.z * sigmoid_gate(bf16_lo(g[1])), x0.w * sigmoid_gate(bf16_hi(g[1]))),
                    pack_bf16x2(x1.x * sigmoid_gate(bf16_lo(g[2])), x1.y * sigmoid_gate(bf16_hi(g[2]))),
                    pack_bf16x2(x1.z * sigmoid_gate(bf16_lo(g[3])), x1.w * sigmoid_gate(bf16_hi(g[3])))};
      *reinterpret_cast<u32x4 *>(output + ((t0 + qq) * kQueryHeads + head) * kHeadDim + 128 * grp +
                                 c8) = w;
    }
  }
}

__global__ __launch_bounds__(kThreads) void prefill_mfma_kernel(
    const bf16_bits *__restrict__ query, const bf16_bits *__restrict__ gate,
    bf16_bits *__restrict__ output, const bf16_bits *__restrict__ cache, std::size_t tokens,
    std::size_t max_ctx, std::size_t past, bool head_major) {
  __shared__ PrefillShared sh;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int grp = wave >> 2;  // key-split group: tiles grp, grp + kSplits, ...
  const int hw = wave & 3;    // query head of the GQA group
  const int gtid = tid & 255; // thread index inside the group
  const int col = lane & 31;  // query column of S^T / O^T
  const int half = lane >> 5; // k-half of the operands
  const std::size_t qtile = gridDim.x - 1 - blockIdx.x; // longest tiles first
  const std::size_t kv_head = blockIdx.y;
  const std::size_t head = kv_head * kGroup + hw;
  const std::size_t t0 = qtile * kQTile;
  const std::size_t q_rows = tokens - t0 < kQTile ? tokens - t0 : kQTile;
  const std::size_t key_end = past + t0 + q_rows;
  const std::size_t n_tiles = (key_end + kKTile - 1) / kKTile;
  const std::size_t plane = max_ctx * kKvHeads * kHeadDim;
  const float scale = kLog2e / 16.0f;
  const std::size_t my_qpos = past + t0 + col;
  StageTile &st = sh.main.stage[grp];

  // Q tile -> LDS: thread -> (head, query row, 64-dim quarter); rows past the
  // tile's end repeat the last row (their outputs are never stored).
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int idx = tid + kThreads * r;          // 0 .. 1023
    const int qh = idx >> 8, qrow = (idx >> 3) & 31, seg = idx & 7;
    const std::size_t qr = static_cast<std::size_t>(qrow) < q_rows ? qrow : q_rows - 1;
    const bf16_bits *src = query + ((t0 + qr) * kQueryHeads + kv_head * kGroup + qh) * kHeadDim + seg * 32;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      *reinterpret_cast<u32x4 *>(&sh.main.q[qh][qrow][seg * 32 + c * 8]) =
          *reinterpret_cast<const u32x4 *>(src + c * 8);
  }

  floatx16 o[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) o[nb] = floatx16{};
  float m_run = -INFINITY; // running reference max of query `col` (exp2 domain)
  float l_run = 0.f;       // partial sum over this lane's keys

  // Staging map: thread -> keys 4*kg .. 4*kg+3, dims 8*db .. 8*db+7; kg varies
  // fastest inside a wave so each load instruction covers 8 full 128-byte lines.
  const int kg = gtid & 7;
  const int db = gtid >> 3;
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
  // Every group runs the same number of steps (so the barriers match); a
  // group whose tile index is past the end idles through the last step.
  const std::size_t steps = (n_tiles + kSplits - 1) / kSplits;
  if (static_cast<std::size_t>(grp) < n_tiles) load_tile(static_cast<std::size_t>(grp) * kKTile);

  for (std::size_t step = 0; step < steps; ++step) {
    const std::size_t tile = step * kSplits + grp;
    const bool active = tile < n_tiles;
    const std::size_t k0 = tile * kKTile;
    __syncthreads(); // previous tile fully consumed
    if (active) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        *reinterpret_cast<u32x4 *>(&st.k[4 * kg + j][8 * db]) = kc[j];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int word = e >> 1;
        const int shift = (e & 1) * 16;
        const std::uint32_t v0 = (vc[0][word] >> shift) & 0xFFFFu, v1 = (vc[1][word] >> shift) & 0xFFFFu;
        const std::uint32_t v2 = (vc[2][word] >> shift) & 0xFFFFu, v3 = (vc[3][word] >> shift) & 0xFFFFu;
        *reinterpret_cast<u32x2 *>(&st.vt[8 * db + e][4 * kg]) = u32x2{v0 | (v1 << 16), v2 | (v3 << 16)};
      }
    }
    __syncthreads();
    if (!active) continue;
    if (tile + kSplits < n_tiles) load_tile(k0 + kSplits * kKTile); // prefetch the next tile

    // S^T = K Q^T: rows = keys, column = query `col`.
    floatx16 s = floatx16{};
#pragma unroll
    for (int kb = 0; kb < 16; ++kb)
      s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lds_b128(&st.k[col][kb * 16 + half * 8]),
                                                  lds_b128(&sh.main.q[hw][col][kb * 16 + half * 8]), s,
                                                  0, 0, 0);

    // Key of accumulator register i: 8*(i/4) + half*4 + i%4.
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const std::size_t key = k0 + (i >> 2) * 8 + half * 4 + (i & 3);
      s[i] = (key > my_qpos || key >= key_end) ? -INFINITY : s[i] * scale;
      mx = fmaxf(mx, s[i]);
    }
    mx = max_xor32(mx);
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
      pw[kb] = u32x4{pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(p[4], p[5]),
                     pack_bf16x2(p[6], p[7])};
    }
    // O^T += V^T P^T.  k-slot (kb, j) of this lane <-> key
    // 16kb + 4*half + j (j < 4) and 16kb + 8 + 4*half + (j-4) (j >= 4).
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bf16_bits *vrow = &st.vt[nb * 32 + col][16 * kb + 4 * half];
        const u32x2 lo = *reinterpret_cast<const u32x2 *>(vrow);
        const u32x2 hi = *reinterpret_cast<const u32x2 *>(vrow + 8);
        const bf16x8 a = __builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
        o[nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, __builtin_bit_cast(bf16x8, pw[kb]),
                                                        o[nb], 0, 0, 0);
      }
    }
  }

  // Each group finishes one half of the dims (group g: dims 128g .. 128g+127,
  // O^T blocks 4g .. 4g+3) for its head: it takes the other group's partial
  // of that half, M = max(m_own, m_other), O = O_own 2^(m_own-M) +
  // O_other 2^(m_other-M), likewise l.  A group that saw no key has m = -inf
  // (weight 0); group 0 always saw key 0.
  // Register indices must be compile-time constants (a run-time index into
  // o[] would move the accumulators to scratch), so each group runs its own
  // instantiation of the tail.
  if (grp == 0)
    prefill_tail<0>(o, m_run, l_run, sh, gate, output, t0, q_rows, head, wave, lane, col, half);
  else
    prefill_tail<1>(o, m_run, l_run, sh, gate, output, t0, q_rows, head, wave, lane, col, half);
}

} // namespace

void launch_prefill_mfma(const bf16_bits *q, const bf16_bits *gate, bf16_bits *out,
                         const bf16_bits *cache, std::size_t tokens, std::size_t max_ctx,
                         std::size_t past, bool head_major, hipStream_t stream) {
  const dim3 grid{static_cast<unsigned>(ceil_div_unchecked(tokens, kQTile)), kKvHeads, 1};
  prefill_mfma_kernel<<<grid, kThreads, 0, stream>>>(q, gate, out, cache, tokens, max_ctx, past,
                                                head_major);
}

} // namespace raftinfer::amd
