// bf16 decode attention core on gfx950 MFMA, used by the single-block,
// split-K and batched decode kernels for bf16 activations and bf16 caches.
//
// Work split: a workgroup owns one KV head, one token range (a split-K
// partition or the whole context) and one slice of DIMS = 256/DS output dims.
// Every workgroup computes the full q.k scores of its range for the four query
// heads of the GQA group (cheap on MFMA) but reads and accumulates only its
// V slice, so a 256-token partition is shared by DS workgroups without any
// cross-workgroup reduction or scratch memory: each writes its own dims of
// the partial (max and sum are identical across the DS siblings).  Blocks are
// numbered so the DS siblings of a partition land on the same XCD and share
// its L2 (workgroups are dispatched round-robin over the 8 XCDs).
//
// Per wave, tokens are consumed 32 at a time:
//   S[token][head] = v_mfma_f32_16x16x32_bf16 on whole-line K loads
//   online softmax in the exp2 domain (log2(e)/16 folded into the scale)
//   O[head][dims] += p * V  on VALU (lane = 16-byte V segment x token phase)
#pragma once

#include "decode_scan.hpp"

#include <type_traits>

namespace raftinfer::amd {

struct DecodeMfmaArgs {
  const bf16_bits *query;   // [16][256] for this sequence
  const bf16_bits *key_new; // [4][256] token appended at position ctx-1
  const bf16_bits *value_new;
  const bf16_bits *cache;   // K plane then V plane
  bf16_bits *cache_rw;
  std::size_t max_ctx;
  bool head_major;
};

// q of one GQA group and the new token's k after RMSNorm + RoPE, computed by
// the decode kernel itself when the producers are fused into it; rot holds the
// rotation table (cos then sin) of the decode position.
struct DecodeFusedQK {
  bf16_bits q[kGroup][kHeadDim];
  bf16_bits k[kHeadDim];
  float rot[kHeadDim];
};

template <int DS, int WAVES, int CT = 32> struct DecodeMfmaShared {
  static constexpr int DIMS = kHeadDim / DS;
  float p[WAVES][CT][4];
  float m[WAVES][4];
  float l[WAVES][4];
  float acc[WAVES][4][DIMS];
};

// LDS stage of the DMA-fed scan: per wave, one chunk's K rows (16-byte piece
// c of row t at piece c ^ (2 * (t % 8)), so the score reads of 8 tokens x 2
// pieces hit distinct banks) and its V slice.
template <int DS, int WAVES, int CT = 32> struct DecodeStage {
  alignas(16) unsigned char k[WAVES][CT * kHeadDim * 2];
  alignas(16) bf16_bits v[WAVES][CT * (kHeadDim / DS)];
  // q of the GQA group and the new token's K and V rows (each row twice: one
  // load instruction moves 1 KiB), written alike by every wave.
  alignas(16) bf16_bits q[kGroup][kHeadDim];
  alignas(16) bf16_bits knew[2][kHeadDim];
  alignas(16) bf16_bits vnew[2][kHeadDim];
};

// PV lane mapping for a DIMS-wide slice and CT-token chunks: a lane owns VEC
// consecutive dims (one 2*VEC-byte load per token) and one of TL token phases.
template <int DIMS, int CT = 32> struct PvMap {
  static constexpr int VEC = DIMS / 8 > 8 ? 8 : DIMS / 8;
  static constexpr int DL = DIMS / VEC;
  static constexpr int TL = 64 / DL;
  static constexpr int TPL = CT / TL;
  static_assert(DL * VEC == DIMS && DL * TL == 64 && TPL * TL == CT && DL >= 8, "bad PV map");
};

template <int VEC> struct VRow {
  std::uint32_t w[VEC / 2];
  __device__ __forceinline__ void load(const bf16_bits *p) {
    if constexpr (VEC == 8) {
      // Each V slice is read by one workgroup only: a non-temporal load keeps
      // it from displacing the K lines that sibling workgroups re-read.
      const u32x4 x = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
      w[0] = x[0]; w[1] = x[1]; w[2] = x[2]; w[3] = x[3];
    } else if constexpr (VEC == 4) {
      const u32x2 x = *reinterpret_cast<const u32x2 *>(p);
      w[0] = x[0]; w[1] = x[1];
    } else {
      w[0] = *reinterpret_cast<const std::uint32_t *>(p);
    }
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < VEC / 2; ++i) w[i] = 0u;
  }
  __device__ __forceinline__ float get(int e) const {
    return (e & 1) ? bf16_hi(w[e >> 1]) : bf16_lo(w[e >> 1]);
  }
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Scans tokens [begin, end) of kv_head for the dims slice dq; leaves
// per-wave (m, l, acc) in sh.  Row `pos` (the token being appended) is read
// from key_new / value_new instead of the cache.
//
// Scores: a group of 8 tokens is read with 8 lanes per 128-byte line (4 loads
// cover the 512-byte rows), so every load instruction fetches 8 whole lines,
// and goes straight into v_mfma_f32_16x16x32_bf16 as the A operand: lane l
// holds 16 bytes of token t = (l%16)/2 at segment 2*(l/16) + l%2 of the line,
// i.e. A row m = 2t + half (half = l%2) with k = (l/16)*8 + j.  The B operand
// holds, in column n = 4*half' + h (n < 8), head h's q at the same segments
// for half' (columns 8..15 are zero), so C[2t + half][4*half + h] is the dot
// over half of the line and the score is C[2t][h] + C[2t+1][4+h], two values
// 4 lanes apart in a row (one DPP add).  After it, lane l with l%16 < 4 holds
// head l%16's scores of tokens 2*(l/16) and 2*(l/16)+1 of the group.
//
// kFused: q comes from fq->q and the new token's key row from fq->k (both in
// LDS) instead of a.query and a.key_new.
struct NoPrologue {
  __device__ void operator()() const {}
};

// pro (kFused, register-fed scan only): the workgroup's q / k prologue, which
// fills fq and holds workgroup barriers.  Each wave runs it once, right after
// issuing its first chunk's loads (a wave without a chunk right away), so the
// cache rows stream in while q and k are normalised; q is read from fq only
// after it.
template <int DS, int WAVES, int CT = 32, bool kFused = false, bool kDma = false, typename Pro = NoPrologue>
__device__ __forceinline__ void decode_mfma_scan(const DecodeMfmaArgs &a, std::size_t kv_head,
                                                 int dq, std::size_t begin, std::size_t end,
                                                 std::size_t pos, DecodeMfmaShared<DS, WAVES, CT> &sh,
                                                 const DecodeFusedQK *fq = nullptr,
                                                 DecodeStage<DS, WAVES, CT> *stage = nullptr,
                                                 Pro pro = Pro{}) {
  constexpr bool kPro = !std::is_same_v<Pro, NoPrologue>;
  static_assert(!kPro || (kFused && !kDma), "the overlapped prologue is for the fused register-fed scan");
  constexpr int DIMS = kHeadDim / DS;
  constexpr int G = CT / 8; // 8-token groups per chunk
  // K is read non-temporally when at most 4 sibling workgroups share it
  // (split-K: 4096 -> 9.7 us per call, batched x32: 406 -> 375 us); the 16
  // single-block siblings need it to stay in L2 (7.1 -> 8.0 us otherwise).
  constexpr bool kNtKeys = DS <= 4;
  using Map = PvMap<DIMS, CT>;
  constexpr int VEC = Map::VEC, DL = Map::DL, TL = Map::TL, TPL = Map::TPL;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n = lane & 15;              // MFMA column (B / C) and row (A)
  const int kq = lane >> 4;             // k-quarter (A / B), row quarter (C)
  const int seg = 2 * kq + (lane & 1);  // 16-byte segment of the line this lane loads
  const int rt = n >> 1;                // token of the group this lane loads
  const bool head_lane = n < kGroup;    // lane holds scores of head n
  const int dl = lane % DL;
  const int tl = lane / DL;
  const float scale = kLog2e / 16.0f;
  const std::size_t plane = a.max_ctx * kKvHeads * kHeadDim;
  const bf16_bits *kplane = a.cache;
  const bf16_bits *vplane = a.cache + plane;

  // kDma: the chunk's K rows and V slice go straight to this wave's LDS
  // stage (global_load_lds_dwordx4) and are read back before the next
  // chunk's loads are issued into the same place, so the next chunk streams
  // in while this one is used.  Rows past `end` read row end-1.  Every load of
  // the scan goes through the stage (q and the new token's rows too), so all
  // its waits are counted by hand and the compiler places none of its own
  // between them.
  [[maybe_unused]] unsigned k_lds = 0, v_lds = 0;
  // Half h of a chunk: K rows 16h .. 16h+15 (8 instructions), and for h = 1
  // also the V slice of all 32 rows (1 instruction).
  auto dma_half = [&](std::size_t c0, int h) {
    const bf16_bits *kb = kplane + cache_row(a.head_major, c0, kv_head, a.max_ctx);
    const std::size_t row_elems = a.head_major ? kHeadDim : kKvHeads * kHeadDim;
#pragma unroll
    for (int jj = 0; jj < CT / 4; ++jj) {
      const int j = (CT / 4) * h + jj;
      const int r = 2 * j + (lane >> 5);
      const std::size_t tok = c0 + r < end ? c0 + r : end - 1;
      const std::uint32_t voff = static_cast<std::uint32_t>((tok - c0) * row_elems * 2) +
                                 16u * static_cast<std::uint32_t>((lane & 31) ^ (2 * (r & 7)));
      load_lds_b128(kb, voff, k_lds + 1024u * j);
    }
    if (h == 1) {
      const bf16_bits *vb = vplane + cache_row(a.head_major, c0, kv_head, a.max_ctx) + dq * DIMS;
      const int r = lane / (64 / CT);
      const std::size_t tok = c0 + r < end ? c0 + r : end - 1;
      load_lds_b128(vb, static_cast<std::uint32_t>((tok - c0) * row_elems * 2) + 16u * (lane % (64 / CT)),
                    v_lds);
    }
  };
  if constexpr (kDma) {
    static_assert(CT == 32 && DIMS * 2 * CT == 1024 && VEC == 2, "one V instruction per chunk");
    k_lds = lds_address(&stage->k[wave][0]);
    v_lds = lds_address(&stage->v[wave][0]);
    const std::uint32_t row_off = 16u * static_cast<std::uint32_t>(lane & 31);
    if constexpr (!kFused) {
      load_lds_b128(a.query + kv_head * kGroup * kHeadDim, 16u * lane, lds_address(&stage->q[0][0]));
      load_lds_b128(a.query + kv_head * kGroup * kHeadDim, 1024u + 16u * lane, lds_address(&stage->q[2][0]));
      load_lds_b128(a.key_new + kv_head * kHeadDim, row_off, lds_address(&stage->knew[0][0]));
    }
    load_lds_b128(a.value_new + kv_head * kHeadDim, row_off, lds_address(&stage->vnew[0][0]));
    if (begin + static_cast<std::size_t>(wave) * CT < end) {
      dma_half(begin + static_cast<std::size_t>(wave) * CT, 0);
      dma_half(begin + static_cast<std::size_t>(wave) * CT, 1);
      wait_vm<CT / 2 + 1>(); // q and the new rows have landed
    } else {
      wait_vm<0>();
    }
  }

  // B operand per line: column n < 8 = (half' = n/4, head n%4).
  bf16x8 qb[4];
  auto make_qb = [&] {
#pragma unroll
  for (int line = 0; line < 4; ++line) {
    u32x4 w = u32x4{0u, 0u, 0u, 0u};
    if (n < 8) {
      if constexpr (kDma && !kFused)
        w = *reinterpret_cast<const u32x4 *>(&stage->q[n & 3][line * 64 + (2 * kq + (n >> 2)) * 8]);
      else if constexpr (kFused)
        w = *reinterpret_cast<const u32x4 *>(&fq->q[n & 3][line * 64 + (2 * kq + (n >> 2)) * 8]);
      else
        w = *reinterpret_cast<const u32x4 *>(a.query + (kv_head * kGroup + (n & 3)) * kHeadDim + line * 64 +
                                             (2 * kq + (n >> 2)) * 8);
    }
    qb[line] = __builtin_bit_cast(bf16x8, w);
  }
  };
  bool pro_done = false;
  if constexpr (!kPro) make_qb();

  float m_run = -INFINITY; // for head n (head lanes)
  float l_run = 0.f;       // per-lane partial sum for head n
  float acc[4][VEC];
#pragma unroll
  for (int h = 0; h < 4; ++h)
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[h][e] = 0.f;

  for (std::size_t c0 = begin + static_cast<std::size_t>(wave) * CT; c0 < end;
       c0 += static_cast<std::size_t>(WAVES) * CT) {
    u32x4 kr[G][4];
    VRow<VEC> vv[TPL];
    [[maybe_unused]] bool issue_second = false;
    if constexpr (kDma) {
      // The stage is used in two halves so that the next chunk streams in
      // behind this one: once rows 0-15 have landed and been read, the next
      // chunk's rows 0-15 go out; then rows 16-31 and V, likewise.  Loads
      // retire in order, so "at most 9 outstanding" means this chunk's first
      // half has landed (its second half is the 9 youngest).
      const bool more = c0 + static_cast<std::size_t>(WAVES) * CT < end; // wave-uniform
      wait_vm<CT / 4 + 1>();
      const unsigned char *kst = reinterpret_cast<const unsigned char *>(&stage->k[wave][0]);
      auto read_groups = [&](int g0) {
#pragma unroll
        for (int g = g0; g < g0 + G / 2; ++g) {
          const int t = 8 * g + rt;
#pragma unroll
          for (int line = 0; line < 4; ++line)
            kr[g][line] = *reinterpret_cast<const u32x4 *>(kst + t * 512 + 16 * ((line * 8 + seg) ^ (2 * (t & 7))));
        }
      };
      read_groups(0);
      wait_lgkm0(); // rows 0-15 have been read
      if (more) {
        dma_half(c0 + static_cast<std::size_t>(WAVES) * CT, 0);
        wait_vm<CT / 4>(); // this chunk's second half has landed
      } else {
        wait_vm<0>();
      }
      read_groups(G / 2);
#pragma unroll
      for (int j = 0; j < TPL; ++j)
        vv[j].w[0] = *reinterpret_cast<const std::uint32_t *>(&stage->v[wave][(tl + TL * j) * DIMS + VEC * dl]);
      wait_lgkm0(); // rows 16-31 and V have been read
      issue_second = more; // goes out after the softmax, below (ctx 1024 cold 12.24 -> 11.93 us)
      if (pos >= c0 && pos < c0 + CT) { // this chunk holds the new token (wave-uniform)
#pragma unroll
        for (int g = 0; g < G; ++g) {
          if (c0 + 8 * g + rt == pos) {
#pragma unroll
            for (int line = 0; line < 4; ++line)
              kr[g][line] = *reinterpret_cast<const u32x4 *>(
                  kFused ? &fq->k[line * 64 + seg * 8] : &stage->knew[0][line * 64 + seg * 8]);
          }
        }
#pragma unroll
        for (int j = 0; j < TPL; ++j)
          if (c0 + tl + TL * j == pos)
            vv[j].w[0] = *reinterpret_cast<const std::uint32_t *>(&stage->vnew[0][dq * DIMS + VEC * dl]);
      }
    } else {
      // Issue every load of the chunk first: K for the scores, V for the slice.
      // Tokens past `end` read row end-1 (in bounds); they are masked below.
#pragma unroll
      for (int g = 0; g < G; ++g) {
        std::size_t tok = c0 + 8 * g + rt;
        tok = tok < end ? tok : end - 1;
        // (fused: the cache row of the new token is read too, and replaced below)
        const bf16_bits *row = !kFused && tok == pos ? a.key_new + kv_head * kHeadDim
                                                     : kplane + cache_row(a.head_major, tok, kv_head, a.max_ctx);
#pragma unroll
        for (int line = 0; line < 4; ++line)
          kr[g][line] = kNtKeys ? __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(row + line * 64 + seg * 8))
                                : *reinterpret_cast<const u32x4 *>(row + line * 64 + seg * 8);
      }
      if constexpr (kPro) {
        // V loads go out with K, then the prologue runs under them.
#pragma unroll
        for (int j = 0; j < TPL; ++j) {
          std::size_t tok = c0 + tl + TL * j;
          tok = tok < end ? tok : end - 1;
          const bf16_bits *row = tok == pos ? a.value_new + kv_head * kHeadDim
                                            : vplane + cache_row(a.head_major, tok, kv_head, a.max_ctx);
          vv[j].load(row + dq * DIMS + VEC * dl);
        }
        if (!pro_done) {
          pro();
          make_qb();
          pro_done = true;
        }
      }
      if constexpr (kFused) {
        if (pos >= c0 && pos < c0 + CT) { // this chunk holds the new token (wave-uniform)
#pragma unroll
          for (int g = 0; g < G; ++g) {
            if (c0 + 8 * g + rt == pos) {
#pragma unroll
              for (int line = 0; line < 4; ++line)
                kr[g][line] = *reinterpret_cast<const u32x4 *>(&fq->k[line * 64 + seg * 8]);
            }
          }
        }
      }
      if constexpr (!kPro) {
#pragma unroll
        for (int j = 0; j < TPL; ++j) {
          std::size_t tok = c0 + tl + TL * j;
          tok = tok < end ? tok : end - 1;
          const bf16_bits *row = tok == pos ? a.value_new + kv_head * kHeadDim
                                            : vplane + cache_row(a.head_major, tok, kv_head, a.max_ctx);
          vv[j].load(row + dq * DIMS + VEC * dl);
        }
      }
    }
    // Keep every load of the chunk ahead of the first wait: the scheduler
    // otherwise sinks V loads below the K waits, adding a second round trip.
    __builtin_amdgcn_sched_barrier(0);
    // Scores of tokens c0 + 8g + 2kq + {0, 1} for head n (head lanes).
    float sg[G][2];
    float mx = -INFINITY;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      floatx4 c = floatx4{};
#pragma unroll
      for (int line = 0; line < 4; ++line)
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kr[g][line]), qb[line], c,
                                                    0, 0, 0);
      // Scaled on VALU first, so the DPP reads a VALU result, not an MFMA one.
      const float s0 = c[0] * scale + dpp<kDppRor12>(c[1] * scale);
      const float s1 = c[2] * scale + dpp<kDppRor12>(c[3] * scale);
      const std::size_t t0 = c0 + 8 * g + 2 * kq;
      sg[g][0] = head_lane && t0 < end ? s0 : -INFINITY;
      sg[g][1] = head_lane && t0 + 1 < end ? s1 : -INFINITY;
      mx = fmaxf(mx, fmaxf(sg[g][0], sg[g][1]));
    }
    mx = max_xor32(max_xor16(mx));
    // Lanes that hold no head see m_new = -inf; their values are never used.
    const float m_new = fmaxf(m_run, mx);
    const float sc = fast_exp2(m_run - m_new); // m_run = -inf -> 0
    float psum = 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const float p = fast_exp2(sg[g][t] - m_new);
        psum += p;
        if (head_lane) sh.p[wave][8 * g + 2 * kq + t][n] = p;
      }
    l_run = l_run * sc + psum;
    m_run = m_new;
    if constexpr (kDma) {
      if (issue_second) dma_half(c0 + static_cast<std::size_t>(WAVES) * CT, 1);
    }
    wave_lds_order();
    float scl[4]; // lane h < 4 holds head h's rescale factor
#pragma unroll
    for (int h = 0; h < 4; ++h)
      scl[h] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc), h));
#pragma unroll
    for (int h = 0; h < 4; ++h)
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[h][e] *= scl[h];
#pragma unroll
    for (int j = 0; j < TPL; ++j) {
      const float4 p4 = *reinterpret_cast<const float4 *>(&sh.p[wave][tl + TL * j][0]);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float v = vv[j].get(e);
        acc[0][e] = fmaf(p4.x, v, acc[0][e]);
        acc[1][e] = fmaf(p4.y, v, acc[1][e]);
        acc[2][e] = fmaf(p4.z, v, acc[2][e]);
        acc[3][e] = fmaf(p4.w, v, acc[3][e]);
      }
    }
    wave_lds_order();
  }
  if constexpr (kPro) {
    if (!pro_done) pro(); // a wave without a chunk
  }
  // l: the lanes of head n are n, n+16, n+32, n+48.
  const float l_tot = sum_xor32(sum_xor16(l_run));
  if (lane < kGroup) {
    sh.m[wave][lane] = m_run;
    sh.l[wave][lane] = l_tot;
  }
  // Sum acc over the token phases (lane bits >= log2(DL)) by reduce-scatter:
  // value v = h*VEC + e; after the lane-32 step lane bit 5 selects the upper
  // half of the values, after the lane-16 step bit 4 the upper quarter, so
  // lane l ends with values i + NV/4 * b4 + NV/2 * b5 (or i + NV/2 * b5).
  constexpr int NV = 4 * VEC;
  float v[NV];
#pragma unroll
  for (int h = 0; h < 4; ++h)
#pragma unroll
    for (int e = 0; e < VEC; ++e) v[h * VEC + e] = acc[h][e];
#pragma unroll
  for (int i = 0; i < NV / 2; ++i) v[i] = swap_sum32(v[i], v[i + NV / 2]);
  const int b5 = (lane >> 5) & 1, b4 = (lane >> 4) & 1;
  if constexpr (TL >= 4) {
#pragma unroll
    for (int i = 0; i < NV / 4; ++i) v[i] = swap_sum16(v[i], v[i + NV / 4]);
    if constexpr (TL == 8) {
#pragma unroll
      for (int i = 0; i < NV / 4; ++i) v[i] = sum_xor8(v[i]);
    }
    if (TL < 8 || (lane & 8) == 0) {
#pragma unroll
      for (int i = 0; i < NV / 4; ++i) {
        const int idx = i + (NV / 4) * b4 + (NV / 2) * b5;
        sh.acc[wave][idx / VEC][VEC * dl + idx % VEC] = v[i];
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < NV / 2; ++i) {
      const int idx = i + (NV / 2) * b5;
      sh.acc[wave][idx / VEC][VEC * dl + idx % VEC] = v[i];
    }
  }
}

// Cold-cache prefetch for the single-block scan, whose DS sibling workgroups
// all stream the same K rows chunk by chunk (only ~128 tokens of a head in
// flight at a time).  Each sibling first touches 1/DS of the head's K and V
// rows of tokens [0, ctx), one dword per 128-byte line (which brings the whole
// line into L2; a touch per 64 or 32 bytes measured no faster cold and slower
// hot), dropped into a dummy LDS word per lane (sink), so the whole head is
// requested from HBM at once and the scan's loads then hit L2: ctx 512 cold
// 8.58 -> 8.25 us, ctx 1024 13.9 -> 12.25 us; hot it costs 0.2-0.3 us.  At
// most kRounds instructions per wave (all of ctx <= 2048 at 8 waves, DS = 16).
// These loads are older than every load of the scan, so its in-order vmcnt
// waits still name the same loads.  Head-major caches only (a token-major
// head is not contiguous).
template <int DS, int WAVES, int kRounds = 2>
__device__ __forceinline__ void prefetch_head_rows(const DecodeMfmaArgs &a, std::size_t kv_head, int dq,
                                                   std::size_t ctx, unsigned sink) {
  if (!a.head_major) return;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  constexpr std::size_t kLine = 128;                   // one touch per 128-byte line
  constexpr std::size_t kPieces = kHeadDim * 2 / kLine; // lines per row
  const std::size_t pieces = ctx * kPieces;       // per plane
  const std::size_t per = (pieces + DS - 1) / DS; // per sibling and plane
  const std::size_t first = static_cast<std::size_t>(dq) * per;
  if (first >= pieces) return; // (uniform)
  const std::size_t count = per < pieces - first ? per : pieces - first;
  const std::size_t blocks = (count + 63) / 64; // instructions per plane
  // The sibling's first line is folded into the (scalar) base, so the per-lane
  // offset stays below kRounds * WAVES * 64 lines (128 KiB) at any context.
  const bf16_bits *kb = a.cache + cache_row(true, 0, kv_head, a.max_ctx) + first * (kLine / 2);
  const bf16_bits *vb = kb + a.max_ctx * kKvHeads * kHeadDim;
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const std::size_t i = static_cast<std::size_t>(wave) + static_cast<std::size_t>(r) * WAVES;
    if (i >= 2 * blocks) break; // wave-uniform
    const bool second = i >= blocks;
    std::size_t line = (second ? i - blocks : i) * 64 + lane;
    line = line < count ? line : count - 1;
    load_lds_b32(second ? vb : kb, static_cast<std::uint32_t>(line * kLine), sink);
  }
}

template <int DS, int WAVES, int CT>
__device__ __forceinline__ void decode_mfma_combine(const DecodeMfmaShared<DS, WAVES, CT> &sh, int h,
                                                    int d, float &m_out, float &l_out,
                                                    float &a_out) {
  float mm = -INFINITY;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) mm = fmaxf(mm, sh.m[w][h]);
  float l = 0.f, acc = 0.f;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) {
    const float wgt = fast_exp2(sh.m[w][h] - mm);
    l = fmaf(sh.l[w][h], wgt, l);
    acc = fmaf(sh.acc[w][h][d], wgt, acc);
  }
  m_out = mm;
  l_out = l;
  a_out = acc;
}

// Maps a block id to (unit, dims slice) so the DS slices of one unit share
// an XCD: unit t's slices are blocks ((t/8)*DS + dq)*8 + t%8.
template <int DS>
__device__ __forceinline__ void xcd_unit(unsigned b, std::size_t &unit, int &dq) {
  const unsigned j = b >> 3;
  unit = static_cast<std::size_t>(j / DS) * 8 + (b & 7);
  dq = static_cast<int>(j % DS);
}

template <int DS> inline unsigned xcd_grid(std::size_t units) {
  return static_cast<unsigned>(((units + 7) / 8) * 8 * DS);
}

} // namespace raftinfer::amd
