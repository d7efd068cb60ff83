// Causal gated GQA prefill attention for the Qwen3.5 signature (16 query
// heads, 4 KV heads, head_dim 256) on gfx950 bf16 MFMA.
//
// Workgroup = 4 waves = one KV head x a 32-token query tile; wave w computes
// query head 4*kv_head + w, so every K/V tile staged in LDS serves the four
// heads of the GQA group.  Per 32-key tile:
//   S  = Q K^T       16 x v_mfma_f32_32x32x16_bf16 (Q in VGPRs, K row-major in LDS)
//   online softmax   fp32 running max per row (exp2 domain), per-lane partial sums
//   O += P V         16 x v_mfma_f32_32x32x16_bf16 (P re-laid out through LDS,
//                    V stored transposed in LDS so the key axis is contiguous)
// The sigmoid gate is applied in the epilogue.  Tiles past the causal
// diagonal are skipped; the diagonal tile is masked per element.
#include "decode_scan.hpp"
#include "prefill_mfma.hpp"

namespace raftinfer::amd {
namespace {

constexpr int kQTile = 32;
constexpr int kKTile = 32;
constexpr int kKStride = kHeadDim + 8; // bf16 elements per K row in LDS (528 B)
constexpr int kVStride = kKTile + 8;   // bf16 elements per transposed V row (80 B)
constexpr int kPStride = kKTile + 8;

struct PrefillShared {
  bf16_bits k[kKTile][kKStride];
  bf16_bits vt[kHeadDim][kVStride];
  bf16_bits p[4][kQTile][kPStride];
};

__device__ __forceinline__ bf16x8 lds_b128(const bf16_bits *p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(p));
}

__global__ __launch_bounds__(256) void prefill_mfma_kernel(
    const bf16_bits *__restrict__ query, const bf16_bits *__restrict__ gate,
    bf16_bits *__restrict__ output, const bf16_bits *__restrict__ cache, std::size_t tokens,
    std::size_t max_ctx, std::size_t past, bool head_major) {
  __shared__ PrefillShared sh;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int col = lane & 31;  // MFMA column / A-operand row
  const int half = lane >> 5; // k-half of the A/B operands
  // Largest (most keys) query tiles are dispatched first.
  const std::size_t qtile = gridDim.x - 1 - blockIdx.x;
  const std::size_t kv_head = blockIdx.y;
  const std::size_t head = kv_head * kGroup + wave;
  const std::size_t t0 = qtile * kQTile;
  const std::size_t q_rows = tokens - t0 < kQTile ? tokens - t0 : kQTile;
  const std::size_t key_end = past + t0 + q_rows;
  const std::size_t plane = max_ctx * kKvHeads * kHeadDim;
  const float scale = kLog2e / 16.0f;

  // Q as the A operand: lane holds row `col`, dims kb*16 + half*8 .. +8.
  bf16x8 qa[16];
  {
    const bool valid = static_cast<std::size_t>(col) < q_rows;
    const bf16_bits *qrow = query + ((t0 + col) * kQueryHeads + head) * kHeadDim + half * 8;
#pragma unroll
    for (int kb = 0; kb < 16; ++kb) {
      u32x4 w = valid ? *reinterpret_cast<const u32x4 *>(qrow + kb * 16) : u32x4{0u, 0u, 0u, 0u};
      qa[kb] = __builtin_bit_cast(bf16x8, w);
    }
  }

  floatx16 o[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) o[nb] = floatx16{};
  float m_run[16], l_run[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    m_run[i] = -INFINITY;
    l_run[i] = 0.f;
  }

  // Staging assignment: thread -> keys 4*kg..4*kg+3, dims 8*db..8*db+7.
  const int kg = tid >> 5;
  const int db = tid & 31;

  for (std::size_t k0 = 0; k0 < key_end; k0 += kKTile) {
    u32x4 kc[4], vc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const std::size_t key = k0 + 4 * kg + j;
      if (key < key_end) {
        const std::size_t row = cache_row(head_major, key, kv_head, max_ctx) + 8 * db;
        kc[j] = *reinterpret_cast<const u32x4 *>(cache + row);
        vc[j] = *reinterpret_cast<const u32x4 *>(cache + plane + row);
      } else {
        kc[j] = u32x4{0u, 0u, 0u, 0u};
        vc[j] = u32x4{0u, 0u, 0u, 0u};
      }
    }
    __syncthreads(); // previous tile fully consumed
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<u32x4 *>(&sh.k[4 * kg + j][8 * db]) = kc[j];
    // Transpose V: for each of the 8 dims pack the 4 keys' bf16 into 8 bytes.
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int word = e >> 1;
      const bool hi = e & 1;
      auto pick = [&](int j) -> std::uint32_t {
        return hi ? (vc[j][word] >> 16) : (vc[j][word] & 0xFFFFu);
      };
      u32x2 packed{pick(0) | (pick(1) << 16), pick(2) | (pick(3) << 16)};
      *reinterpret_cast<u32x2 *>(&sh.vt[8 * db + e][4 * kg]) = packed;
    }
    __syncthreads();

    // S = Q K^T for this wave's head.
    floatx16 s = floatx16{};
#pragma unroll
    for (int kb = 0; kb < 16; ++kb) {
      const bf16x8 b = lds_b128(&sh.k[col][kb * 16 + half * 8]);
      s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa[kb], b, s, 0, 0, 0);
    }

    // Online softmax on rows (i/4)*8 + half*4 + i%4, column = key k0 + col.
    const std::size_t key = k0 + col;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = (i >> 2) * 8 + half * 4 + (i & 3);
      const std::size_t qpos = past + t0 + row;
      float v = s[i] * scale;
      if (key > qpos || key >= key_end) v = -INFINITY;
      float mx = row16_max(v);
      mx = fmaxf(mx, xor16(mx));
      const float mnew = fmaxf(m_run[i], mx);
      const float sc = exp2f(m_run[i] - mnew);
      const float p = exp2f(v - mnew);
      l_run[i] = l_run[i] * sc + p;
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) o[nb][i] *= sc;
      m_run[i] = mnew;
      sh.p[wave][row][col] = f32_to_bf16(p);
    }
    __syncthreads();
    bf16x8 pa[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) pa[kb] = lds_b128(&sh.p[wave][col][kb * 16 + half * 8]);
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bf16x8 b = lds_b128(&sh.vt[nb * 32 + col][kb * 16 + half * 8]);
        o[nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pa[kb], b, o[nb], 0, 0, 0);
      }
    }
  }

  // Epilogue: row sums, normalise, gate, store.
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    float l = row16_sum(l_run[i]);
    l += xor16(l);
    const int row = (i >> 2) * 8 + half * 4 + (i & 3);
    if (static_cast<std::size_t>(row) >= q_rows) continue;
    const float inv = 1.0f / l;
    const std::size_t base = ((t0 + row) * kQueryHeads + head) * kHeadDim;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      const std::size_t idx = base + nb * 32 + col;
      const float gv = bf16_to_f32(gate[idx]);
      output[idx] = f32_to_bf16(o[nb][i] * inv * sigmoid_gate(gv));
    }
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
