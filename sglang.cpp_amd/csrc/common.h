// Shared device helpers for the gfx950 attention kernels.
//
// bf16 values are carried as raw uint16_t in memory and widened to fp32 in
// registers; narrowing uses the hardware v_cvt_pk_bf16_f32 (round to
// nearest even), reached through clang's __bf16 conversion.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/sgl_attn.h"

namespace sgl {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// f(integral_constant<int, i>) for i = I .. N-1, unrolled at compile time.
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Low / high bf16 of a packed 32-bit word, widened to fp32.
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float x) {
  __bf16 b = (__bf16)x;
  return (uint32_t)__builtin_bit_cast(uint16_t, b);
}

// Pack two fp32 into one word of two bf16 (a in the low half).
// One v_cvt_pk_bf16_f32 (round to nearest even, as the scalar conversion).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

// Round-trip through bf16 (the value a bf16 store then load would give).
__device__ __forceinline__ float round_bf16(float x) {
  return bf16_bits_to_f32(f32_to_bf16_bits(x));
}

// 16 bytes (8 bf16) unpacked to fp32.
__device__ __forceinline__ void unpack8(const u32x4_t& v, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_lo(v[i]);
    f[2 * i + 1] = bf16_hi(v[i]);
  }
}

__device__ __forceinline__ u32x4_t pack8(const float* f) {
  u32x4_t v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
  return v;
}

// 16-bit element types carried as bit patterns: DT = SGL_DTYPE_BF16 or
// SGL_DTYPE_F16 (fp32 arithmetic, one round-to-nearest-even per store).
typedef _Float16 f16_t;

template <int DT>
__device__ __forceinline__ float to_f32(uint32_t bits16) {
  if constexpr (DT == SGL_DTYPE_BF16) return __uint_as_float(bits16 << 16);
  else return static_cast<float>(__builtin_bit_cast(f16_t, static_cast<uint16_t>(bits16)));
}
template <int DT>
__device__ __forceinline__ uint32_t from_f32(float x) {
  // Round to nearest even in both cases (v_cvt_f16_f32 / the bf16 cast).
  if constexpr (DT == SGL_DTYPE_BF16) return f32_to_bf16_bits(x);
  else return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<f16_t>(x)));
}
template <int DT>
__device__ __forceinline__ float round_t(float x) {
  return to_f32<DT>(from_f32<DT>(x));
}
// Two values packed into one word (a in the low half), exact when both are
// DT-representable.
template <int DT>
__device__ __forceinline__ uint32_t pack2_t(float a, float b) {
  if constexpr (DT == SGL_DTYPE_BF16) return pack_bf16x2(a, b);
  else return from_f32<DT>(a) | (from_f32<DT>(b) << 16);
}
template <int DT>
__device__ __forceinline__ void unpack8_t(const u32x4_t& v, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = to_f32<DT>(v[i] & 0xffffu);
    f[2 * i + 1] = to_f32<DT>(v[i] >> 16);
  }
}
template <int DT>
__device__ __forceinline__ u32x4_t pack8_t(const float (&f)[8]) {
  u32x4_t v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = pack2_t<DT>(f[2 * i], f[2 * i + 1]);
  return v;
}

__device__ __forceinline__ u32x4_t ldg128(const void* p) {
  return *reinterpret_cast<const u32x4_t*>(p);
}
__device__ __forceinline__ void stg128(void* p, const u32x4_t& v) {
  *reinterpret_cast<u32x4_t*>(p) = v;
}
// 16-byte load / store, non-temporal when NT (streams read or written once).
template <bool NT>
__device__ __forceinline__ u32x4_t ldg128_nt(const void* p) {
  if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  else return ldg128(p);
}
template <bool NT>
__device__ __forceinline__ void stg128_nt(void* p, const u32x4_t& v) {
  if constexpr (NT) __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(p));
  else stg128(p, v);
}

// Combine each lane with lane ^ 16 / lane ^ 32 through gfx950's
// v_permlane16_swap / v_permlane32_swap (register to register; a generic
// __shfl_xor is an LDS ds_bpermute). Swapping a value with a copy of itself
// leaves the two partners' values in the two registers, in the same order in
// both lanes, so the combined value is bitwise equal across partners. Inline
// asm: the compiler's builtin folds the two results of a self-swap into one.
// The s_nop covers the VALU-write -> permlane-read hazard.
template <bool kHalf32>
__device__ __forceinline__ void swap_pair(float x, float& lo, float& hi) {
  uint32_t a = __builtin_bit_cast(uint32_t, x), b = a;
  if constexpr (kHalf32)
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  else
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  lo = __builtin_bit_cast(float, a);
  hi = __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float max_xor16(float x) {
  float a, b;
  swap_pair<false>(x, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float max_xor32(float x) {
  float a, b;
  swap_pair<true>(x, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float sum_xor16(float x) {
  float a, b;
  swap_pair<false>(x, a, b);
  return a + b;
}
__device__ __forceinline__ float sum_xor32(float x) {
  float a, b;
  swap_pair<true>(x, a, b);
  return a + b;
}

// Sum over aligned groups of `width` lanes (width a power of two <= 64).
// DPP lane exchange inside rows of 16 lanes (no LDS round trip, unlike the
// ds_bpermute a generic __shfl_xor becomes). CTRL: 0xB1 = quad_perm
// [1,0,3,2] (lane ^ 1), 0x4E = quad_perm [2,3,0,1] (lane ^ 2), 0x141 =
// row_half_mirror (i -> 7 - i in each 8), 0x140 = row_mirror (i -> 15 - i),
// 0x128 = row_ror:8 (i -> i ^ 8 in each 16).
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(x), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __builtin_bit_cast(float, dpp_u32<CTRL>(__builtin_bit_cast(uint32_t, x)));
}

// Sum over aligned groups of `width` lanes (width a power of two <= 64); the
// result is bitwise the same in every lane of a group.
template <int width>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (width == 16) {
    // Pairings whose two partners add the same two values (commutative), so
    // all 16 lanes end with identical bits.
    x += dpp_f32<0xB1>(x);
    x += dpp_f32<0x4E>(x);
    x += dpp_f32<0x141>(x);
    x += dpp_f32<0x140>(x);
    return x;
  } else {
#pragma unroll
    for (int off = width / 2; off > 0; off >>= 1) x += __shfl_xor(x, off, kWave);
    return x;
  }
}

template <int width>
__device__ __forceinline__ float group_max(float x) {
#pragma unroll
  for (int off = width / 2; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, kWave));
  return x;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Launch-status helper: converts the last HIP error into a status code.
inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? SGL_OK : static_cast<int>(e);
}

}  // namespace sgl
