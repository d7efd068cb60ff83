// Shared host/device helpers for the gfx950 attention and gated-delta kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <limits>
#include <stdexcept>
#include <string>
#include <type_traits>

namespace raftinfer::amd {

// ---------------------------------------------------------------- types
using bf16_bits = std::uint16_t;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ------------------------------------------------------- bf16 conversion
// Round-to-nearest-even with quiet-NaN preservation, the rounding of
// cpp/reference/bf16.hpp:16-32 (and of CUDA's __float2bfloat16_rn that the
// reference kernels use for cache stores).
__host__ __device__ __forceinline__ bf16_bits f32_to_bf16(float value) {
  std::uint32_t bits;
#if defined(__HIP_DEVICE_COMPILE__)
  bits = __float_as_uint(value);
#else
  __builtin_memcpy(&bits, &value, sizeof bits);
#endif
  // Branch-free: the compiler turns both selects into v_cndmask.
  const std::uint32_t hi = bits >> 16;
  const std::uint32_t rounded = (bits + 0x7FFFu + (hi & 1u)) >> 16;
  const bool nan_without_payload = (bits & 0x007FFFFFu) != 0 && (hi & 0x7Fu) == 0;
  const std::uint32_t special = nan_without_payload ? (hi | 1u) : hi;
  const bool inf_or_nan = (bits & 0x7F800000u) == 0x7F800000u;
  return static_cast<bf16_bits>(inf_or_nan ? special : rounded);
}

__host__ __device__ __forceinline__ float bf16_to_f32(bf16_bits b) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __uint_as_float(static_cast<std::uint32_t>(b) << 16);
#else
  const std::uint32_t bits = static_cast<std::uint32_t>(b) << 16;
  float f;
  __builtin_memcpy(&f, &bits, sizeof f);
  return f;
#endif
}

// Low / high bf16 of a packed dword as float.
__device__ __forceinline__ float bf16_lo(std::uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(std::uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
// Two floats -> a packed bf16 pair by the hardware conversion
// (v_cvt_pk_bf16_f32, round to nearest even).  Finite values and infinities
// get exactly the bits of f32_to_bf16; a NaN stays a NaN but its payload bits
// may differ, so cache appends (compared bit for bit) keep f32_to_bf16.
__device__ __forceinline__ std::uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16_pair __attribute__((ext_vector_type(2)));
  const bf16_pair v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(std::uint32_t, v);
}

// Element loads / stores from f32 or bf16 storage.
template <typename T> struct Elem;
template <> struct Elem<float> {
  static __device__ __forceinline__ float load(const float *p, std::size_t i) { return p[i]; }
  static __device__ __forceinline__ void store(float *p, std::size_t i, float v) { p[i] = v; }
};
template <> struct Elem<bf16_bits> {
  static __device__ __forceinline__ float load(const bf16_bits *p, std::size_t i) {
    return bf16_to_f32(p[i]);
  }
  static __device__ __forceinline__ void store(bf16_bits *p, std::size_t i, float v) {
    p[i] = f32_to_bf16(v);
  }
};
template <> struct Elem<_Float16> {
  static __device__ __forceinline__ float load(const _Float16 *p, std::size_t i) {
    return static_cast<float>(p[i]);
  }
  static __device__ __forceinline__ void store(_Float16 *p, std::size_t i, float v) {
    p[i] = static_cast<_Float16>(v);
  }
};

// ------------------------------------------------- wavefront reductions
// DPP row (16-lane) butterflies: quad_perm xor1 / xor2, row_half_mirror,
// row_mirror.  After the four steps every lane of a 16-lane row holds the
// row's total.
template <int Ctrl> __device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), Ctrl, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // row_half_mirror
constexpr int kDppMirror = 0x140;     // row_mirror
constexpr int kDppRor12 = 0x12C;      // row_ror:12 (lane i reads lane (i + 4) % 16 of its row)

__device__ __forceinline__ float row16_sum(float x) {
  x += dpp<kDppXor1>(x);
  x += dpp<kDppXor2>(x);
  x += dpp<kDppHalfMirror>(x);
  x += dpp<kDppMirror>(x);
  return x;
}
__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, dpp<kDppXor1>(x));
  x = fmaxf(x, dpp<kDppXor2>(x));
  x = fmaxf(x, dpp<kDppHalfMirror>(x));
  x = fmaxf(x, dpp<kDppMirror>(x));
  return x;
}
// Exchange with lane ^ 16 / ^ 32 inside the wavefront (LDS crossbar, no
// memory traffic).
__device__ __forceinline__ float xor16(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), 0x401F));
}
__device__ __forceinline__ float xor32(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_ds_bpermute(((threadIdx.x ^ 32) & 63) << 2, __builtin_bit_cast(int, x)));
}
// Reduce-scatter step over lane halves / row pairs without the LDS crossbar.
// v_permlane32_swap exchanges the upper 32 lanes of `a` with the lower 32 of
// `b`; summing the two registers after it gives lanes 0..31 a[l] + a[l^32]
// and lanes 32..63 b[l] + b[l^32].  v_permlane16_swap does the same for
// odd/even 16-lane rows: even rows get a[l] + a[l^16], odd rows b[l] + b[l^16].
// Written as inline asm: the compiler builtin's two results are folded into
// one when both are used in the same expression.  The s_nop covers the
// VALU-write -> permlane-read hazard of the operands.
__device__ __forceinline__ float swap_sum32(float a, float b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return a + b;
}
__device__ __forceinline__ float swap_sum16(float a, float b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return a + b;
}
// x op x[lane ^ 16] and x op x[lane ^ 32] (op = max or +) in every lane, by a
// swap of two copies of x.
__device__ __forceinline__ float max_xor16(float x) {
  float a = x, b = x;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return fmaxf(a, b);
}
__device__ __forceinline__ float max_xor32(float x) {
  float a = x, b = x;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return fmaxf(a, b);
}
__device__ __forceinline__ float sum_xor16(float x) { return swap_sum16(x, x); }
__device__ __forceinline__ float sum_xor32(float x) { return swap_sum32(x, x); }

// x + x[lane ^ 8] (row_ror:8 reads lane ^ 8 of the row).
__device__ __forceinline__ float sum_xor8(float x) { return x + dpp<0x128>(x); }

__device__ __forceinline__ float wave_sum(float x) {
  x = row16_sum(x);
  x += xor16(x);
  x += xor32(x);
  return x;
}
__device__ __forceinline__ float wave_max(float x) {
  x = row16_max(x);
  x = fmaxf(x, xor16(x));
  x = fmaxf(x, xor32(x));
  return x;
}

// c + a.lo * b.lo + a.hi * b.hi for packed bf16 pairs (v_dot2_f32_bf16).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot2_bf16(std::uint32_t a, std::uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b),
                                         c, false);
}

// Orders a wave's own LDS writes before its later LDS reads by other lanes.
// The LDS unit executes one wave's instructions in order, so only compiler
// reordering must be prevented; a memory fence here would also wait for every
// outstanding global store of the wave.
__device__ __forceinline__ void wave_lds_order() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_wave_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// ------------------------------------------------ LDS-direct loads
// LDS byte address of a __shared__ object.
template <typename T> __device__ __forceinline__ unsigned lds_address(T *p) {
  return static_cast<unsigned>(reinterpret_cast<std::uintptr_t>(
      (__attribute__((address_space(3))) char *)(p)));
}

// 16 bytes from base + voff (per lane) into LDS at lds + 16 * lane
// (global_load_lds_dwordx4).  base and lds must be wave-uniform; they are
// moved to scalar registers here (readfirstlane), so the instruction's scalar
// operands never depend on the compiler proving that uniformity.  Written as
// asm, with the waits below issued by hand: the compiler cannot tell which
// LDS region such a load writes and would otherwise wait for every
// outstanding one before each LDS read.  The kernels that use it issue no
// other instruction that reads M0.
__device__ __forceinline__ void load_lds_b128(const void *base, std::uint32_t voff, unsigned lds) {
  // readfirstlane returns int: each half goes back to uint32 before it is
  // widened, so a low word with bit 31 set is not sign-extended into the
  // high word.
  const auto b = reinterpret_cast<std::uintptr_t>(base);
  const auto hi = static_cast<std::uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<std::uint32_t>(b >> 32)));
  const auto lo = static_cast<std::uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<std::uint32_t>(b)));
  const std::uint64_t sbase = (static_cast<std::uint64_t>(hi) << 32) | lo;
  const auto slds = static_cast<unsigned>(__builtin_amdgcn_readfirstlane(lds));
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(slds), "v"(voff), "s"(sbase)
               : "memory", "m0");
#pragma clang diagnostic pop
}
// 4 bytes from base + voff (per lane) into LDS at lds + 4 * lane
// (global_load_lds_dword); the same conventions as load_lds_b128.
__device__ __forceinline__ void load_lds_b32(const void *base, std::uint32_t voff, unsigned lds) {
  const auto b = reinterpret_cast<std::uintptr_t>(base);
  const auto hi = static_cast<std::uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<std::uint32_t>(b >> 32)));
  const auto lo = static_cast<std::uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<std::uint32_t>(b)));
  const std::uint64_t sbase = (static_cast<std::uint64_t>(hi) << 32) | lo;
  const auto slds = static_cast<unsigned>(__builtin_amdgcn_readfirstlane(lds));
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2"
               :
               : "s"(slds), "v"(voff), "s"(sbase)
               : "memory", "m0");
#pragma clang diagnostic pop
}
template <int N> __device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}
__device__ __forceinline__ void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory"); }

// ------------------------------------------------------ host utilities
template <typename Error> inline void require(bool condition, const char *message) {
  if (!condition) throw Error(message);
}

template <typename Error>
inline std::size_t checked_mul(std::size_t a, std::size_t b, const char *message) {
  require<Error>(a == 0 || b <= std::numeric_limits<std::size_t>::max() / a, message);
  return a * b;
}

template <typename Error>
inline std::size_t checked_add(std::size_t a, std::size_t b, const char *message) {
  require<Error>(b <= std::numeric_limits<std::size_t>::max() - a, message);
  return a + b;
}

inline std::size_t ceil_div_unchecked(std::size_t n, std::size_t d) {
  return n / d + (n % d == 0 ? 0 : 1);
}

template <typename Error> inline void check_launch(const char *name) {
  const hipError_t error = hipGetLastError();
  if (error != hipSuccess) {
    throw Error(std::string{name} + " launch failed: " + hipGetErrorString(error));
  }
}

} // namespace raftinfer::amd
