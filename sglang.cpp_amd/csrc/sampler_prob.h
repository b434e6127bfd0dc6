// The Sampler's probabilities from logits, shared by the temperature-softmax
// kernel (softmax.hip) and the draws that read logits directly
// (sampling.hip), so both compute every probability with the same
// operations and get the same bits. With a = log2(e) / t (one division per
// row) the exponent of a raw logit x is x a - M a, M the row's largest raw
// logit, formed by one fused multiply-add with the row constant nb = -(M a):
//   per statistics lane v < kStatLanes, a running max mx of its raw logits
//   and sum of 2^(x a - mx a) over its chunks c = v + kStatLanes k
//   (elements [P c, P c + P)), then the elements past the whole chunks one
//   by one; the lanes folded in a fixed order (a butterfly within each group
//   of 64 lanes, then the 16 group values in order) into M and
//   s = sum 2^(x a - M a); p = 2^(fma(x, a, nb)) * (1 / s).
// A temperature that is not positive gives a = NaN, so that row's
// probabilities are NaN (and its draws the last index).
// Floating-point contraction is off in these functions: the one fused
// multiply-add is explicit, and another one chosen differently in the two
// kernels would change low bits.
#pragma once

#include "common.h"

namespace sgl {
namespace sp {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kStatLanes = 1024;  // lanes that compute a row's statistics
constexpr int kStatWaves = kStatLanes / kWave;

template <int DT>
struct Elem;
template <>
struct Elem<SGL_DTYPE_BF16> {
  static constexpr int kPer = 8;  // elements per 16-byte chunk
  __device__ static float at(const u32x4_t& v, int j) {
    const uint32_t w = v[j >> 1];
    return (j & 1) ? bf16_hi(w) : bf16_lo(w);
  }
  __device__ static float load1(const void* p, int64_t i) {
    return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  }
};
template <>
struct Elem<SGL_DTYPE_F16> {
  static constexpr int kPer = 8;
  __device__ static float at(const u32x4_t& v, int j) {
    const uint32_t w = v[j >> 1];
    return static_cast<float>(__builtin_bit_cast(f16_t, static_cast<uint16_t>((j & 1) ? w >> 16 : w)));
  }
  __device__ static float load1(const void* p, int64_t i) {
    return static_cast<float>(__builtin_bit_cast(f16_t, static_cast<const uint16_t*>(p)[i]));
  }
};
template <>
struct Elem<SGL_DTYPE_F32> {
  static constexpr int kPer = 4;
  __device__ static float at(const u32x4_t& v, int j) { return __uint_as_float(v[j]); }
  __device__ static float load1(const void* p, int64_t i) { return static_cast<const float*>(p)[i]; }
};

// The exp2 scale of a raw logit: log2(e) / t, NaN unless t > 0.
__device__ __forceinline__ float exp2_scale(float t) {
#pragma clang fp contract(off)
  return t > 0.f ? kLog2e / t : __builtin_nanf("");
}

// The row constant of the exponent fma(x, a, nb) given the row max M.
__device__ __forceinline__ float exp2_offset(float m, float a) {
#pragma clang fp contract(off)
  return -(m * a);
}

// A lane's running state: max mx of its raw logits, nb = exp2_offset(mx, a)
// and the sum s of 2^(fma(x, a, nb)). Starts at (-inf, 0, 0).
struct LaneStats {
  float mx = -INFINITY, nb = 0.f, s = 0.f;
};

// LaneStats updated by N raw logits.
template <int N>
__device__ __forceinline__ void online_update(const float (&x)[N], float a, LaneStats& st) {
#pragma clang fp contract(off)
  float cm = x[0];
#pragma unroll
  for (int j = 1; j < N; ++j) cm = fmaxf(cm, x[j]);
  if (cm > st.mx) {
    const float nb = exp2_offset(cm, a);
    st.s *= __builtin_amdgcn_exp2f(__builtin_fmaf(st.mx, a, nb));  // 0 while mx = -inf
    st.mx = cm;
    st.nb = nb;
  }
#pragma unroll
  for (int j = 0; j < N; ++j) st.s += __builtin_amdgcn_exp2f(__builtin_fmaf(x[j], a, st.nb));
}

template <int DT>
__device__ __forceinline__ void unpack(const u32x4_t& v, float (&x)[Elem<DT>::kPer]) {
#pragma unroll
  for (int j = 0; j < Elem<DT>::kPer; ++j) x[j] = Elem<DT>::at(v, j);
}

// The probability of raw logit x given a, nb = exp2_offset(M, a) and 1 / s.
__device__ __forceinline__ float prob(float x, float a, float nb, float inv_s) {
#pragma clang fp contract(off)
  return __builtin_amdgcn_exp2f(__builtin_fmaf(x, a, nb)) * inv_s;
}

// A lane's sum relative to the row max M (a lane with no element adds 0).
__device__ __forceinline__ float lane_sum_at(const LaneStats& st, float m, float a) {
#pragma clang fp contract(off)
  return st.mx == -INFINITY ? 0.f
                            : st.s * __builtin_amdgcn_exp2f(__builtin_fmaf(st.mx, a, exp2_offset(m, a)));
}

// Fixed-order reductions over the kStatWaves groups of 64 statistics lanes:
// a butterfly within each group, then every wave folds the group values in
// order. One value per thread (1024 threads: group = wave) ...
template <int kWaves>
__device__ __forceinline__ float block_max(float x, float* sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, kWave));
  __syncthreads();  // earlier readers of sh are done
  if (lane == 0) sh[wave] = x;
  __syncthreads();
  float m = sh[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) m = fmaxf(m, sh[w]);
  return m;
}

template <int kWaves>
__device__ __forceinline__ float block_sum(float x, float* sh) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, kWave);
  __syncthreads();
  if (lane == 0) sh[wave] = x;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) s += sh[w];
  return s;
}

// ... or two per thread (512 threads: x0 for lane t = group w, x1 for lane
// t + 512 = group w + 8), the same butterflies and the same fold.
template <int kWaves>
__device__ __forceinline__ float block_max2(float x0, float x1, float* sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    x0 = fmaxf(x0, __shfl_xor(x0, o, kWave));
    x1 = fmaxf(x1, __shfl_xor(x1, o, kWave));
  }
  __syncthreads();
  if (lane == 0) {
    sh[wave] = x0;
    sh[kWaves + wave] = x1;
  }
  __syncthreads();
  float m = sh[0];
#pragma unroll
  for (int w = 1; w < 2 * kWaves; ++w) m = fmaxf(m, sh[w]);
  return m;
}

template <int kWaves>
__device__ __forceinline__ float block_sum2(float x0, float x1, float* sh) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    x0 += __shfl_xor(x0, o, kWave);
    x1 += __shfl_xor(x1, o, kWave);
  }
  __syncthreads();
  if (lane == 0) {
    sh[wave] = x0;
    sh[kWaves + wave] = x1;
  }
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < 2 * kWaves; ++w) s += sh[w];
  return s;
}

// Statistics lane `lane`'s state over a row read from memory: chunks
// c = lane + kStatLanes k below nfull (aligned rows), then the elements from
// nfull * P one by one.
template <int DT>
__device__ __forceinline__ LaneStats lane_stats(const char* row, int d, bool vec, int lane, float a) {
  constexpr int P = Elem<DT>::kPer;
  LaneStats st;
  const int nfull = vec ? d / P : 0;
  auto chunk = [&](int c) {
    return *reinterpret_cast<const u32x4_t*>(row + static_cast<int64_t>(c) * 16);
  };
  // Eight chunks' loads in flight, then processed in chunk order (the
  // order, and so the bits, of the one-at-a-time loop).
  constexpr int kAhead = 8;
  int c = lane;
  for (; c + (kAhead - 1) * kStatLanes < nfull; c += kAhead * kStatLanes) {
    u32x4_t v[kAhead];
#pragma unroll
    for (int k = 0; k < kAhead; ++k) v[k] = chunk(c + k * kStatLanes);
#pragma unroll
    for (int k = 0; k < kAhead; ++k) {
      float x[P];
      unpack<DT>(v[k], x);
      online_update(x, a, st);
    }
  }
  for (; c < nfull; c += kStatLanes) {
    float x[P];
    unpack<DT>(chunk(c), x);
    online_update(x, a, st);
  }
  for (int e = nfull * P + lane; e < d; e += kStatLanes) {
    const float x[1] = {Elem<DT>::load1(row, e)};
    online_update(x, a, st);
  }
  return st;
}

}  // namespace sp
}  // namespace sgl
