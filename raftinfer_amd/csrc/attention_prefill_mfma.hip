// Causal gated GQA prefill attention for the Qwen3.5 signature (16 query
// heads, 4 KV heads, head_dim 256) on gfx950 bf16 MFMA.
//
// Work split.  A workgroup owns one KV head and 8 query tokens.  The 4 query
// heads of the GQA group x the 8 tokens are the 32 columns of one MFMA
// operand (column c = head_in_group * 8 + token), so every K/V element read
// serves all four heads.  The 4 waves split the key range: wave w takes the
// 32-key tiles w, w+4, ...; at PP512 that is 256 workgroups, and the longest
// query tile's 16 key tiles run four at a time on the CU's four SIMDs.
//
// Per tile and wave:
//   staging     K and V rows go from the cache straight into the wave's own
//               LDS tile (global_load_lds_dwordx4, no VGPRs), stored as two
//               halves of the head dims (4 half-rows of 256 bytes per
//               instruction); the next tile's K goes out after the QK chain
//               (first half) and after the softmax (second half), its V after
//               the PV (PP512 13.12 -> ~12.8 us against whole-tile issue
//               straight after each tile's reads).
//               Half-rows are stored as 16 16-byte chunks with chunk c at
//               c ^ swz(row) (see swz for the bank conflicts this leaves);
//   S^T = K Q^T 16 x v_mfma_f32_32x32x16_bf16, K and Q rows read from LDS
//               with ds_read_b128 four MFMAs ahead (the Q tile is staged once
//               per workgroup, in the K tile's chunk order);
//   softmax     online in the exp2 domain; lane l owns column l % 32 and 16
//               of the tile's keys; the reference max moves only when a
//               column max grows by more than 2^8 (lazy rescaling);
//   O^T += V^T P^T  16 x v_mfma_f32_32x32x16_bf16; P^T stays in VGPRs in the
//               S^T accumulator's key order, and the V^T operand is read in
//               that order straight from the row-major V tile with
//               ds_read_b64_tr_b16 (lane i of a 16-lane group receives 4 keys
//               of one dim), eight MFMAs' operands at a time.  The O^T
//               accumulators stay in AGPRs (inline-asm MFMA).
// The waves' partial (max, sum, O) are merged through LDS at the end; wave w
// finishes dims [64w, 64w+64) and applies the sigmoid gate.  Each wave loads
// the gate of its quarter at the start as whole 128-byte lines and stores its
// output the same way, both staged in its own part of the merge area, so
// neither goes out as scattered 8-byte pieces and only one barrier follows
// the loop.  With past == 0 the keys come from the key/value
// inputs and each workgroup also writes its 8 tokens' cache rows (the append).
#include "decode_scan.hpp"
#include "norm_rope.hpp"
#include "prefill_mfma.hpp"

namespace raftinfer::amd {
namespace {

constexpr int kQTok = 8;             // query tokens per workgroup
constexpr int kKTile = 32;           // keys per tile
constexpr int kWaves = 4;            // key-split waves per workgroup
constexpr int kThreads = kWaves * kWave;
constexpr float kLazyRescale = 8.0f; // log2 units
constexpr int kPvBatch = 8;          // PV MFMAs whose operands are read together
constexpr int kHalfElems = kKTile * kHeadDim / 2; // one half of a K / V tile (128 dims)

typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4v;

struct WaveTile {
  bf16_bits k[kKTile * kHeadDim];
  bf16_bits v[kKTile * kHeadDim];
};
struct PrefillShared {
  union {
    WaveTile tile[kWaves];                  // 128 KiB
    // merge: [source wave][finishing wave][block][register quad][lane]; o[w][w]
    // holds wave w's gate / output stage
    float4 o[kWaves][kWaves][2][4][kWave];
  };
  bf16_bits q[32 * kHeadDim]; // Q^T operand rows (one per column), swizzled like K
  float m[kWaves][kWave];
  float l[kWaves][kWave];
};

// The q producer fused into the prefill kernel (NormQ).
struct PrefillNormRope {
  const void *weight; // q norm weight [256], bf16 or f32
  bool weight_f32;
  int pairs;    // rotary_dim / 2 (rotary_dim a multiple of 8)
  double ratio; // rope_base^(-2 / rotary_dim)
  float epsilon;
};
struct alignas(16) NormQShared {
  float weight[kHeadDim];        // the staged norm weight (bf16 uses the first half)
  float rot[kQTok][kHeadDim];    // per token slot: cos[pairs] then sin[pairs]
};

// Physical 16-byte chunk of logical chunk c in tile row r: c ^ (r & 7).  The
// LDS bank-conflict counter, calibrated on these access patterns alone, shows
// this leaves 2-way conflicts on the K/Q ds_read_b128 (16 rows per pass) and
// 4-way on the V ds_read_b64_tr_b16; c ^ (4 (r % 4) + (r / 4) % 4) is free of
// both, but measured PP512 13.2 -> 13.1 us, PP2048 80 -> 78, PP128 7.13 ->
// 7.3 (more lane bases held across the loop), so the loop is not bound by
// these reads and the simpler swizzle stays.
__device__ __forceinline__ int swz(int r) { return r & 7; }

__device__ __forceinline__ int chunk_offset(int r, int c) { // in bf16 elements
  return r * kHeadDim + ((c ^ swz(r)) << 3);
}

__device__ __forceinline__ bf16x8 lds_b128(const bf16_bits *p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(p));
}

__device__ __forceinline__ u32x2 lds_tr16(const bf16_bits *p) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v *)(p)));
}



__host__ __device__ constexpr std::size_t ceil_div_u(std::size_t n, std::size_t d) {
  return (n + d - 1) / d;
}

// o += a * b (v_mfma_f32_32x32x16_bf16) with the accumulator pinned to AGPRs.
// The compiler would otherwise move all 128 accumulator registers between
// AGPRs and VGPRs around every tile because of the (rare) rescale code.  The
// s_nop covers the VALU-write -> MFMA-read hazard of the operands, which the
// hazard recognizer does not see through asm.  For the same reason the
// compiler does not know the MFMA's result latency: a register copy of `o`
// placed right after this statement would read it before it is written.  The
// build (raftinfer_amd/asm_check.py) scans this file's assembly and fails on
// any such read; the drain below covers the reads the kernel itself makes.
__device__ __forceinline__ void mfma_acc_agpr(floatx16 &o, bf16x8 a, bf16x8 b) {
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(o) : "v"(a), "v"(b));
}
// o *= s for an AGPR-resident accumulator.  The empty asm statements pin the
// copy to VGPRs inside this (rare) rescale path; without them the compiler
// hoists the AGPR -> VGPR copies of all accumulators onto every tile.
__device__ __forceinline__ void scale_agpr(floatx16 &o, float s) {
  floatx16 x = o;
  asm volatile("" : "+v"(x));
#pragma unroll
  for (int i = 0; i < 16; ++i) x[i] *= s;
  asm volatile("" : "+v"(x));
  o = x;
}
// Wait states after the last such MFMA before VALU code reads its result.
__device__ __forceinline__ void mfma_drain() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" ::: "memory"); }

__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

// The q producer's RMSNorm + RoPE applied in place to the staged Q rows, bit
// for bit.  Sliced form (rotary pairs a multiple of 32; norm_rope_256_slice):
// eight lanes per row, so a wave finishes its 8 rows at once with one LDS
// round trip.
__device__ __forceinline__ void norm_rope_rows_sliced(bf16_bits *q, int r, int g, const float *weight,
                                                      bool weight_f32, int pairs, const float *rot,
                                                      float epsilon) {
  bf16_bits *row = q + r * kHeadDim;
  u32x4 raw[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) raw[j] = *reinterpret_cast<const u32x4 *>(row + (((4 * g + j) ^ swz(r)) << 3));
  float x[32], w[32], v[32];
  unpack_bf16x32(raw, x);
  load_slice_weights(weight, weight_f32, g, w);
  norm_rope_256_slice(x, w, g, pairs, rot, epsilon, v);
  u32x4 out[4];
  pack_bf16x32(v, out);
#pragma unroll
  for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x4 *>(row + (((4 * g + j) ^ swz(r)) << 3)) = out[j];
}

// Lane-wise form (any rotary width): rows 8w .. 8w+7 one at a time, lane l
// owning dims 4l .. 4l+3 (8 bytes of logical chunk l / 2).
__device__ __forceinline__ void norm_rope_rows_lanewise(bf16_bits *q, int wave, int lane, const float *weight,
                                                        bool weight_f32, int pairs, const float (*rot)[kHeadDim],
                                                        float epsilon) {
  float w[4];
  if (weight_f32) {
    const float4 x = reinterpret_cast<const float4 *>(weight)[lane];
    w[0] = x.x; w[1] = x.y; w[2] = x.z; w[3] = x.w;
  } else {
    const u32x2 x = reinterpret_cast<const u32x2 *>(weight)[lane];
    w[0] = bf16_lo(x[0]); w[1] = bf16_hi(x[0]); w[2] = bf16_lo(x[1]); w[3] = bf16_hi(x[1]);
  }
#pragma unroll
  for (int rr = 0; rr < 8; ++rr) {
    const int r = 8 * wave + rr;
    u32x2 *slot = reinterpret_cast<u32x2 *>(q + chunk_offset(r, lane >> 1) + 4 * (lane & 1));
    const u32x2 raw = *slot;
    const float x[4] = {bf16_lo(raw[0]), bf16_hi(raw[0]), bf16_lo(raw[1]), bf16_hi(raw[1])};
    float v[4];
    norm_rope_256_lane(x, w, lane, pairs, rot[r & (kQTok - 1)], epsilon, v);
    *slot = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  }
}

// FromInput: past == 0 and every key is read from the key/value inputs
// ([tokens][4][256]); the workgroup also writes its own tokens' rows into the
// cache (the append), so no separate append kernel runs.  Otherwise keys are
// read from the cache, which already holds them.
//
// key_in, value_in and gate are deliberately not __restrict__: the plain append
// and gate loads must stay where they are issued, between the LDS-direct
// loads whose hand-written vmcnt waits count them.  With __restrict__ the
// compiler may sink them past the asm loads (it knows the asm cannot reach
// restrict-only memory), and the waits would then release K/V tiles that have
// not landed.
//
// NormQ: `query` is the raw q projection [tokens][16][2][256]; its query half
// is staged like Q and normalised + rotated in LDS (the producer
// qwen35_split_query_gate_norm_rope fused in), and the gate is its second half.
template <bool HeadMajor, bool FromInput, bool NormQ = false>
__global__ __launch_bounds__(kThreads) void prefill_mfma_kernel(
    const bf16_bits *__restrict__ query, const bf16_bits *key_in,
    const bf16_bits *value_in, const bf16_bits *gate,
    bf16_bits *__restrict__ output, bf16_bits *__restrict__ cache, std::size_t tokens,
    std::size_t max_ctx, std::size_t past, PrefillNormRope nq) {
  constexpr bool head_major = HeadMajor;
  static_assert(!(NormQ && FromInput), "the fused producer path reads K/V from the cache");
  __shared__ PrefillShared sh;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int col = lane & 31;  // MFMA column: head_in_group * 8 + token
  const int half = lane >> 5; // k-half of the MFMA operands
  // XCD-aware map: the hardware deals workgroup b to XCD b % 8, and XCDs 2h,
  // 2h+1 take KV head h, so each XCD's L2 holds one head's K/V.  Slots are
  // dealt longest query tile first.
  const std::size_t n_qtiles = ceil_div_u(tokens, kQTok);
  const unsigned xcd = blockIdx.x & 7u;
  const std::size_t slot = 2 * (blockIdx.x >> 3) + (xcd & 1u);
  if (slot >= n_qtiles) return; // padding of an odd tile count
  const std::size_t qtile = n_qtiles - 1 - slot;
  const std::size_t kv_head = xcd >> 1;
  const std::size_t t0 = qtile * kQTok;
  const std::size_t q_rows = tokens - t0 < kQTok ? tokens - t0 : kQTok;
  const std::size_t key_end = past + t0 + q_rows;
  const std::size_t n_tiles = (key_end + kKTile - 1) / kKTile;
  const std::size_t plane = max_ctx * kKvHeads * kHeadDim;
  const float scale = kLog2e / 16.0f;
  const int col_tok = col & (kQTok - 1);
  const std::size_t col_row = static_cast<std::size_t>(col_tok) < q_rows ? col_tok : q_rows - 1;
  const std::size_t col_pos = past + t0 + col_row;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave); // wave index as a scalar
  // Element offset of column c's row (head c / 8, token c % 8, clamped to the
  // tile's tokens) in the query / gate / output layout [T][16][256].
  auto io_row = [&](int c) {
    const std::size_t tt = static_cast<std::size_t>(c & 7) < q_rows ? static_cast<std::size_t>(c & 7) : q_rows - 1;
    return ((t0 + tt) * kQueryHeads + kv_head * kGroup + (c >> 3)) * kHeadDim;
  };
  // Row of column c's gate: the gate input, or the second half of its q
  // projection row.
  const bf16_bits *gate_src = NormQ ? query + kHeadDim : gate;
  auto gate_row = [&](int c) { return NormQ ? 2 * io_row(c) : io_row(c); };
  constexpr std::size_t q_row_elems = NormQ ? 2 * kHeadDim : kHeadDim; // elements between Q rows
  WaveTile &tile = sh.tile[wave_u];
  constexpr int kLateLoads = 4 + (FromInput ? 2 : 0); // gate (+ append) loads per thread

  floatx16 o[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) o[nb] = floatx16{};
  float m_run = -INFINITY; // reference max of column `col` (exp2 domain)
  float l_run = 0.f;       // sum over this lane's keys, relative to m_run

  // Staging: load instruction i fills tile rows 2i, 2i+1 (1 KiB of LDS, lane
  // -> row 2i + half, physical chunk `col`) straight from the cache, so the
  // lane reads logical chunk col ^ swz(row) of its key.  Keys past key_end
  // read row key_end - 1 (in bounds); their scores are masked.
  constexpr std::uint32_t row_bytes = head_major && !FromInput ? kHeadDim * 2 : kKvHeads * kHeadDim * 2;
  // Row 0 of this KV head in the K and V sources.
  const bf16_bits *k_src = FromInput ? key_in + kv_head * kHeadDim
                                     : cache + cache_row(head_major, 0, kv_head, max_ctx);
  const bf16_bits *v_src = FromInput ? value_in + kv_head * kHeadDim : k_src + plane;
  const unsigned lds_k = lds_address(tile.k), lds_v = lds_address(tile.v);
  // A tile is stored as two halves of the head dims ([half][32 rows][256 B],
  // 16-byte chunk c of a half-row at c ^ swz(row)), so that each half is
  // filled by 8 load instructions of 1 KiB (4 half-rows each) and the next
  // tile's first half can go out once the current tile's dims 0-127 are read.
  // Instruction i of half hh: lane -> row 4i + lane / 16, physical chunk
  // lane % 16; swz(row) depends on i only through its parity, so two per-lane
  // offsets serve all 8.
  const int hrow = lane >> 4, hpc = lane & 15;
  std::uint32_t voff_half[2];
#pragma unroll
  for (int p = 0; p < 2; ++p)
    voff_half[p] = (4 * p + hrow) * row_bytes + 16u * (hpc ^ swz(4 * p + hrow));
  auto issue_half = [&](const bf16_bits *plane_base, unsigned lds, std::size_t k0, int hh) {
    const bf16_bits *base = plane_base + k0 * (row_bytes / 2);
    const std::size_t rows_left = key_end - k0;
    if (rows_left >= kKTile) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        load_lds_b128(base, voff_half[i & 1] + 8 * (i >> 1) * row_bytes + 256u * hh,
                      lds + 8192u * hh + 1024u * i);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = 4 * i + hrow;
        const int last = static_cast<int>(rows_left) - 1;
        const std::uint32_t rr = r < last ? r : last;
        load_lds_b128(base, rr * row_bytes + 256u * hh + 16u * (hpc ^ swz(r)), lds + 8192u * hh + 1024u * i);
      }
    }
  };
  auto issue = [&](const bf16_bits *plane_base, unsigned lds, std::size_t k0) {
    issue_half(plane_base, lds, k0, 0);
    issue_half(plane_base, lds, k0, 1);
  };
  // Element offsets: k_base into the Q stage (whole 256-dim rows), kt_base
  // into a K tile half (128-dim rows), v_base into a V tile half.
  int k_base[4], kt_base[4], v_base[2];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    k_base[j] = chunk_offset(col, 2 * j + half);
    kt_base[j] = col * (kHeadDim / 2) + (((2 * j + half) ^ swz(col)) << 3);
  }
  {
    const int g = lane >> 4, r = lane & 15;
    const int trow = 4 * half + (r >> 2);
    const int dsub = 16 * (g & 1) + 4 * (r & 3); // dim offset inside a 32-dim block
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int d = 32 * j + dsub;
      v_base[j] = trow * (kHeadDim / 2) + (((d >> 3) ^ swz(trow)) << 3) + (d & 7);
    }
  }
  // Q tile -> LDS, row = column c (token c % 8 of head 4 kv + c / 8), in the
  // K tile's chunk order; wave w loads rows 8w .. 8w+7 (4 instructions).
  {
    const unsigned lq = lds_address(sh.q);
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int i = 4 * wave_u + ii;
      const int r = 2 * i + half; // column of this lane's row
      const int rt = r & (kQTok - 1);
      const std::size_t rrow = static_cast<std::size_t>(rt) < q_rows ? rt : q_rows - 1;
      const std::uint32_t voff = static_cast<std::uint32_t>(rrow * kQueryHeads + (r >> 3)) * (q_row_elems * 2) +
                                 16u * (col ^ swz(r));
      load_lds_b128(query + (t0 * kQueryHeads + kv_head * kGroup) * q_row_elems, voff, lq + 1024u * i);
    }
  }
  [[maybe_unused]] NormQShared *nqs = nullptr;
  if constexpr (NormQ) {
    // The q norm weight (512 B bf16 or 1 KiB f32) into LDS by wave 0, issued
    // before K/V so the Q wait below covers it; lanes past the weight re-read
    // its last piece.
    __shared__ NormQShared nq_sh;
    nqs = &nq_sh;
    if (wave_u == 0) {
      const std::uint32_t bytes = nq.weight_f32 ? 1024u : 512u;
      const std::uint32_t off = 16u * lane < bytes ? 16u * lane : bytes - 16u;
      load_lds_b128(nq.weight, off, lds_address(nq_sh.weight));
    }
  }
  std::size_t t = wave_u;
  // Issue order: Q, K(t0), V(t0), then the append and gate loads (kLateLoads,
  // needed only at the end) | K(t+4) V(t+4) per tile t, so 16 loads (plus
  // kLateLoads on the first tile) follow K(t) when it is waited for, and 16
  // (or none on the last tile, plus kLateLoads on the first) follow V(t).
  if (t < n_tiles) {
    issue(k_src, lds_k, t * kKTile);
    issue(v_src, lds_v, t * kKTile);
  }
  // Append (FromInput): thread -> two 16-byte pieces of this workgroup's K/V
  // rows (2 planes x 8 tokens x 32 pieces); loaded now, stored at the end.
  u32x4 app[2];
  if constexpr (FromInput) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int idx = tid + kThreads * j; // 0 .. 511
      const int pl = idx >> 8, tok = (idx >> 5) & 7, piece = idx & 31;
      const std::size_t tt = static_cast<std::size_t>(tok) < q_rows ? tok : q_rows - 1;
      const bf16_bits *src = (pl ? value_in : key_in) + ((t0 + tt) * kKvHeads + kv_head) * kHeadDim;
      app[j] = *reinterpret_cast<const u32x4 *>(src + 8 * piece);
    }
  }
  // Gate of this wave's output quarter (dims 64w .. 64w+63), held in registers
  // until the epilogue.  Column c (head c / 8, token c % 8) of the quarter is
  // one 128-byte line; load n covers columns 8n .. 8n+7 (lane -> column
  // 8n + lane / 8, 16-byte chunk lane % 8), whole lines per instruction.
  // Tokens past q_rows read token q_rows - 1 (never stored), so every thread
  // issues exactly kLateLoads loads here, which the waits below count.
  u32x4 gc[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const int c = 8 * n + (lane >> 3), k = lane & 7;
    gc[n] = *reinterpret_cast<const u32x4 *>(gate_src + gate_row(c) + 64 * wave_u + 8 * k);
  }

  if constexpr (NormQ) {
    // Rotation tables of the tile's (up to 8) positions, while Q is in flight.
    for (int i = tid; i < kQTok * nq.pairs; i += kThreads) {
      const int slot = i / nq.pairs, pp = i - slot * nq.pairs;
      const std::size_t tt = static_cast<std::size_t>(slot) < q_rows ? slot : q_rows - 1;
      float cs, sn;
      rope_cos_sin(pp, past + t0 + tt, nq.ratio, cs, sn);
      nqs->rot[slot][pp] = cs;
      nqs->rot[slot][nq.pairs + pp] = sn;
    }
  }
  if (t < n_tiles) wait_vm<32 + kLateLoads>(); else wait_vm<0>(); // this wave's Q rows have landed
  __syncthreads(); // ... and every other wave's
  if constexpr (NormQ) {
    if (nq.pairs % 32 == 0)
      norm_rope_rows_sliced(sh.q, 8 * wave_u + (lane >> 3), lane & 7, nqs->weight, nq.weight_f32, nq.pairs,
                            nqs->rot[(lane >> 3) & (kQTok - 1)], nq.epsilon);
    else
      norm_rope_rows_lanewise(sh.q, wave_u, lane, nqs->weight, nq.weight_f32, nq.pairs, nqs->rot, nq.epsilon);
    __syncthreads(); // every row is normalised
  }
  for (; t < n_tiles; t += kWaves) {
    const std::size_t k0 = t * kKTile;
    const bool more = t + kWaves < n_tiles;
    const std::size_t k0_next = k0 + kWaves * kKTile;
    const bool first = t == static_cast<std::size_t>(wave_u);
    if (first) wait_vm<16 + kLateLoads>(); else wait_vm<16>(); // K(t) has landed; V(t) may still be in flight
    // S^T = K Q^T: A row = key `col` of the tile (lane & 31), k-half `half`.
    // Chunk 2 kb + half of row `col` sits at (2 (kb & 3) + half) ^ (col & 7)
    // + 8 (kb >> 2): four lane bases plus constant offsets.
    // Operands are read four MFMAs ahead (one batch per k_base group).
    floatx16 s = floatx16{};
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) {
      bf16x8 ka[4], qa[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ka[j] = lds_b128(tile.k + kt_base[j] + 64 * (k4 & 1) + kHalfElems * (k4 >> 1));
        qa[j] = lds_b128(sh.q + k_base[j] + 64 * k4);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka[j], qa[j], s, 0, 0, 0);
    }
    wait_lgkm0(); // the K tile has been read
    if (more) issue_half(k_src, lds_k, k0_next, 0);

    // Key of accumulator register i: k0 + 8 (i / 4) + 4 half + i % 4.  Only
    // a tile that reaches past the tile's first query position is masked.
    float mx = -INFINITY;
    if (k0 + kKTile - 1 > past + t0) {
      const std::ptrdiff_t rel_pos = static_cast<std::ptrdiff_t>(col_pos - k0) - 4 * half;
      const int lim = rel_pos < -1 ? -1 : (rel_pos > kKTile ? kKTile : static_cast<int>(rel_pos));
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        s[i] = (i >> 2) * 8 + (i & 3) > lim ? -INFINITY : s[i] * scale;
        mx = fmaxf(mx, s[i]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        s[i] *= scale;
        mx = fmaxf(mx, s[i]);
      }
    }
    mx = max_xor32(mx);
    const bool grow = mx > m_run + kLazyRescale;
    if (first) {
      // A wave's first tile: nothing is accumulated yet (m = -inf, l = 0,
      // o = 0), so the new max needs no rescale of the accumulators (the
      // rescale moves all 128 of them through VGPRs; PP128 7.24 -> 6.86 us).
      m_run = grow ? mx : m_run;
    } else if (__builtin_amdgcn_ballot_w64(grow) != 0) {
      // Lanes that do not grow keep their scale (1, also when m is still -inf).
      const float m_new = grow ? mx : m_run;
      const float sc = grow ? fexp2(m_run - mx) : 1.0f; // -inf -> 0 on a first tile
      l_run *= sc;
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) scale_agpr(o[nb], sc);
      m_run = m_new;
    }
    // A column whose keys so far are all masked keeps m = -inf; its
    // probabilities are exp2(-inf - 0) = 0 rather than exp2(-inf + inf).
    const float m_ref = m_run == -INFINITY ? 0.f : m_run;
    bf16x8 pw[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      float p[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) p[j] = fexp2(s[8 * kb + j] - m_ref);
      const u32x4 pk{pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(p[4], p[5]),
                     pack_bf16x2(p[6], p[7])};
      // The sum takes the same bf16 probabilities the PV product uses, so the
      // output is an exact convex combination of the V rows with those weights
      // (a key that holds all the weight gives its V row exactly).
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const std::uint32_t w = pk[j];
        l_run += bf16_lo(w) + bf16_hi(w);
      }
      pw[kb] = __builtin_bit_cast(bf16x8, pk);
    }

    if (more) issue_half(k_src, lds_k, k0_next, 1); // after the softmax
    if (first) {
      if (more) wait_vm<16 + kLateLoads>(); else wait_vm<kLateLoads>(); // V(t) has landed
    } else {
      if (more) wait_vm<16>(); else wait_vm<0>();
    }
    // O^T += V^T P^T.  k-slot (kb, half, j) <-> key 16 kb + 4 half + j (j < 4)
    // and 16 kb + 8 + 4 half + (j - 4) (j >= 4), the P^T register order.  A
    // row (dim) 32 nb + 16 (g & 1) + r of 16-lane group g: source lane r of
    // the transposed read supplies dims 4 (r & 3) .. +3 of key (r >> 2).
    // Row 16 kb + trow (+ 8) and dim 32 nb + dsub: the swizzle key is trow & 7
    // for every row read, so two lane bases (nb & 1) plus constant offsets
    // (rows 16 kb (+8), chunk 8 (nb >> 1)) cover all 32 reads.
    // The operands of kPvBatch MFMAs are read before any of them is issued, so
    // the LDS latency is paid once per batch rather than once per MFMA.
    {
      constexpr int kBatch = kPvBatch;
#pragma unroll
      for (int b0 = 0; b0 < 16; b0 += kBatch) {
        bf16x8 av[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          const int nb = (b0 + j) >> 1, kb = (b0 + j) & 1;
          const bf16_bits *v0 =
              tile.v + v_base[nb & 1] + 64 * ((nb >> 1) & 1) + kHalfElems * (nb >> 2) + (kHeadDim / 2) * 16 * kb;
          const u32x2 lo = lds_tr16(v0);
          const u32x2 hi = lds_tr16(v0 + (kHeadDim / 2) * 8);
          av[j] = __builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          const int nb = (b0 + j) >> 1, kb = (b0 + j) & 1;
          mfma_acc_agpr(o[nb], av[j], pw[kb]);
        }
      }
      mfma_drain(); // the accumulators may be read by VALU code below
    }
    wait_lgkm0(); // the V tile has been read
    if (more) issue(v_src, lds_v, k0_next);
  }


  // Append (FromInput): every wave has waited for all of its loads by now, so
  // the cache rows go out here and drain under the merge and the epilogue.
  if constexpr (FromInput) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int idx = tid + kThreads * j;
      const int pl = idx >> 8, tok = (idx >> 5) & 7, piece = idx & 31;
      if (static_cast<std::size_t>(tok) < q_rows)
        *reinterpret_cast<u32x4 *>(cache + pl * plane + cache_row(head_major, t0 + tok, kv_head, max_ctx) +
                                   8 * piece) = app[j];
    }
  }
  // Wave w finishes O^T blocks 2w, 2w+1 (dims 64w .. 64w+63).  As soon as its
  // loop ends it writes the other three quarters into its own tile region
  // (o[w][q] for finisher q; only wave w reads that region before this point),
  // so early waves export while late ones still compute, and it stages its
  // gate quarter in its own slot o[w][w].  One barrier, then each wave merges
  // its quarter and finishes it without further workgroup synchronisation.
  // (The quarter loop is unrolled so that every register index is a
  // compile-time constant.)
#pragma unroll
  for (int q = 0; q < kWaves; ++q) {
    if (q == wave) continue;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const floatx16 &x = o[2 * q + j];
        sh.o[wave][q][j][i4][lane] = make_float4(x[4 * i4], x[4 * i4 + 1], x[4 * i4 + 2], x[4 * i4 + 3]);
      }
  }
  // Gate / output staging: [32 columns][64 dims] bf16 in the wave's own slot,
  // 16-byte chunk k of column c at k ^ ((c / 4) % 8), so the epilogue's 8-byte
  // reads (32 columns, one chunk) and the 16-byte row writes hit distinct banks.
  bf16_bits *stage = reinterpret_cast<bf16_bits *>(&sh.o[wave][wave][0][0][0]);
  auto stage_at = [](int c, int k) { return c * 64 + ((k ^ ((c >> 2) & 7)) << 3); };
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const int c = 8 * n + (lane >> 3), k = lane & 7;
    *reinterpret_cast<u32x4 *>(stage + stage_at(c, k)) = gc[n];
  }
  sh.m[wave][lane] = m_run;
  sh.l[wave][lane] = l_run;
  __syncthreads(); // every wave's exports, m and l are written

  // The other waves' quarters are read first; the gate's sigmoids (which do
  // not depend on the merge) are computed while those reads are in flight.
  float4 xo[kWaves][2][4];
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    if (w == wave) continue;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) xo[w][j][i4] = sh.o[w][wave][j][i4][lane];
  }
  float mw[kWaves], lw[kWaves];
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    mw[w] = sh.m[w][lane];
    lw[w] = sh.l[w][lane];
  }
  // Sigmoid of the gate pieces this lane finishes: column col, dims
  // 32 j + 8 i4 + 4 half .. +3 of the quarter.
  float sg[2][16];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const u32x2 g = *reinterpret_cast<const u32x2 *>(stage + stage_at(col, 4 * j + i4) + 4 * half);
      sg[j][4 * i4] = sigmoid_gate(bf16_lo(g[0]));
      sg[j][4 * i4 + 1] = sigmoid_gate(bf16_hi(g[0]));
      sg[j][4 * i4 + 2] = sigmoid_gate(bf16_lo(g[1]));
      sg[j][4 * i4 + 3] = sigmoid_gate(bf16_hi(g[1]));
    }
  // A wave that saw no key has m = -inf and weight 0; some wave saw key 0.
  float mm = -INFINITY;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) mm = fmaxf(mm, mw[w]);
  float lsum = 0.f;
  floatx16 f[2];
#pragma unroll
  for (int q = 0; q < kWaves; ++q) {
    if (q != wave) continue;
    const float a = fexp2(m_run - mm);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 16; ++i) f[j][i] = a * o[2 * q + j][i];
  }
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const float a = fexp2(mw[w] - mm);
    lsum += a * lw[w];
    if (w == wave) continue;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const float4 x = xo[w][j][i4];
        f[j][4 * i4] += a * x.x;
        f[j][4 * i4 + 1] += a * x.y;
        f[j][4 * i4 + 2] += a * x.z;
        f[j][4 * i4 + 3] += a * x.w;
      }
  }
  const float inv = 1.0f / (lsum + xor32(lsum));
  // Gated outputs replace the gate in the stage (each lane rewrites exactly
  // the 8-byte pieces it read), then leave as whole 128-byte lines.
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      auto *slot = reinterpret_cast<u32x2 *>(stage + stage_at(col, 4 * j + i4) + 4 * half);
      const floatx16 &x = f[j];
      *slot = u32x2{pack_bf16x2(x[4 * i4] * inv * sg[j][4 * i4], x[4 * i4 + 1] * inv * sg[j][4 * i4 + 1]),
                    pack_bf16x2(x[4 * i4 + 2] * inv * sg[j][4 * i4 + 2], x[4 * i4 + 3] * inv * sg[j][4 * i4 + 3])};
    }
  wave_lds_order(); // the stage is rewritten by other lanes of this wave
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const int c = 8 * n + (lane >> 3), k = lane & 7;
    if (static_cast<std::size_t>(c & 7) < q_rows)
      *reinterpret_cast<u32x4 *>(output + io_row(c) + 64 * wave_u + 8 * k) =
          *reinterpret_cast<const u32x4 *>(stage + stage_at(c, k));
  }
}

} // namespace

void launch_prefill_mfma(const bf16_bits *q, const bf16_bits *key, const bf16_bits *value,
                         const bf16_bits *gate, bf16_bits *out, bf16_bits *cache,
                         std::size_t tokens, std::size_t max_ctx, std::size_t past,
                         bool head_major, bool fused_append, hipStream_t stream) {
  // 8 workgroups (one per XCD) per pair of query tiles.
  const unsigned grid = static_cast<unsigned>(8 * ceil_div_unchecked(ceil_div_unchecked(tokens, kQTok), 2));
  const PrefillNormRope none{};
  if (fused_append) {
    if (head_major)
      prefill_mfma_kernel<true, true><<<grid, kThreads, 0, stream>>>(q, key, value, gate, out, cache,
                                                                     tokens, max_ctx, past, none);
    else
      prefill_mfma_kernel<false, true><<<grid, kThreads, 0, stream>>>(q, key, value, gate, out, cache,
                                                                      tokens, max_ctx, past, none);
  } else if (head_major) {
    prefill_mfma_kernel<true, false><<<grid, kThreads, 0, stream>>>(q, key, value, gate, out, cache,
                                                                    tokens, max_ctx, past, none);
  } else {
    prefill_mfma_kernel<false, false><<<grid, kThreads, 0, stream>>>(q, key, value, gate, out, cache,
                                                                     tokens, max_ctx, past, none);
  }
}

namespace {
// The k producer fused with the cache append: block = token, wave h = KV
// head h.  RMSNorm + RoPE of the raw key row (the arithmetic of
// qwen35_qk_norm_rope) stored at position past + t of the K plane, and the
// value row copied to the V plane.
__global__ __launch_bounds__(256) void key_norm_rope_append_kernel(
    const bf16_bits *__restrict__ key, const bf16_bits *__restrict__ value, const void *weight,
    bool weight_f32, int pairs, double ratio, float epsilon, bf16_bits *__restrict__ cache,
    std::size_t max_ctx, std::size_t past, bool head_major) {
  __shared__ float rot[kHeadDim];
  const std::size_t t = blockIdx.x;
  const int lane = threadIdx.x & 63, h = threadIdx.x >> 6;
  const std::size_t src = (t * kKvHeads + h) * kHeadDim + 4 * lane;
  const u32x2 raw = *reinterpret_cast<const u32x2 *>(key + src);
  const u32x2 vv = *reinterpret_cast<const u32x2 *>(value + src);
  float w[4];
  if (weight_f32) {
    const float4 x = reinterpret_cast<const float4 *>(weight)[lane];
    w[0] = x.x; w[1] = x.y; w[2] = x.z; w[3] = x.w;
  } else {
    const u32x2 x = reinterpret_cast<const u32x2 *>(weight)[lane];
    w[0] = bf16_lo(x[0]); w[1] = bf16_hi(x[0]); w[2] = bf16_lo(x[1]); w[3] = bf16_hi(x[1]);
  }
  if (static_cast<int>(threadIdx.x) < pairs) {
    float cs, sn;
    rope_cos_sin(threadIdx.x, past + t, ratio, cs, sn);
    rot[threadIdx.x] = cs;
    rot[pairs + threadIdx.x] = sn;
  }
  __syncthreads();
  const float x[4] = {bf16_lo(raw[0]), bf16_hi(raw[0]), bf16_lo(raw[1]), bf16_hi(raw[1])};
  float v[4];
  norm_rope_256_lane(x, w, lane, pairs, rot, epsilon, v);
  const std::size_t row = cache_row(head_major, past + t, h, max_ctx) + 4 * lane;
  *reinterpret_cast<u32x2 *>(cache + row) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  *reinterpret_cast<u32x2 *>(cache + max_ctx * kKvHeads * kHeadDim + row) = vv;
}
} // namespace

void launch_prefill_mfma_fused(const bf16_bits *query_gate, const bf16_bits *key,
                               const bf16_bits *value, bf16_bits *out, bf16_bits *cache,
                               std::size_t tokens, std::size_t max_ctx, std::size_t past,
                               bool head_major, const void *q_weight, const void *k_weight,
                               bool weight_f32, int pairs, double ratio, float epsilon,
                               hipStream_t stream) {
  key_norm_rope_append_kernel<<<static_cast<unsigned>(tokens), 256, 0, stream>>>(
      key, value, k_weight, weight_f32, pairs, ratio, epsilon, cache, max_ctx, past, head_major);
  const unsigned grid = static_cast<unsigned>(8 * ceil_div_unchecked(ceil_div_unchecked(tokens, kQTok), 2));
  const PrefillNormRope nq{q_weight, weight_f32, pairs, ratio, epsilon};
  if (head_major)
    prefill_mfma_kernel<true, false, true><<<grid, kThreads, 0, stream>>>(
        query_gate, key, value, nullptr, out, cache, tokens, max_ctx, past, nq);
  else
    prefill_mfma_kernel<false, false, true><<<grid, kThreads, 0, stream>>>(
        query_gate, key, value, nullptr, out, cache, tokens, max_ctx, past, nq);
}

} // namespace raftinfer::amd
