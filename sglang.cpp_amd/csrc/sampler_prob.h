// The Sampler's probabilities from logits, shared by the temperature-softmax
// kernel (softmax.hip) and the draws that read logits directly
// (sampling.hip), so both compute every probability with the same
// operations and get the same bits:
//   y = x * (1 / t); per statistics lane v < kStatLanes, a running max m and
//   sum of 2^((y - m) log2e) over its chunks c = v + kStatLanes k
//   (elements [P c, P c + P)), then the elements past the whole chunks one
//   by one; folded in a fixed order (a butterfly within each group of 64
//   lanes, then the 16 group values in order); p = 2^((y - m) log2e) *
//   (1 / sum). A 1024-thread workgroup runs one lane per thread; a 512-thread
//   workgroup runs lanes t and t + 512 on thread t.
// Floating-point contraction is off in these functions: a fused multiply-add
// chosen differently in the two kernels would change low bits.
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

// Running (max, sum of 2^((y - max) log2e)) of a lane, updated by N values.
template <int N>
__device__ __forceinline__ void online_update(const float (&y)[N], float& mx, float& s) {
#pragma clang fp contract(off)
  float cm = y[0];
#pragma unroll
  for (int j = 1; j < N; ++j) cm = fmaxf(cm, y[j]);
  if (cm > mx) {
    s *= __builtin_amdgcn_exp2f((mx - cm) * kLog2e);  // 0 while mx = -inf
    mx = cm;
  }
#pragma unroll
  for (int j = 0; j < N; ++j) s += __builtin_amdgcn_exp2f((y[j] - mx) * kLog2e);
}

template <int DT>
__device__ __forceinline__ void scaled(const u32x4_t& v, float inv_t, float (&y)[Elem<DT>::kPer]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int j = 0; j < Elem<DT>::kPer; ++j) y[j] = Elem<DT>::at(v, j) * inv_t;
}

__device__ __forceinline__ float scaled1(float x, float inv_t) {
#pragma clang fp contract(off)
  return x * inv_t;
}

// The probability of logit x given the row's max m and 1 / sum.
__device__ __forceinline__ float prob(float x, float inv_t, float m, float inv_s) {
#pragma clang fp contract(off)
  return __builtin_amdgcn_exp2f((x * inv_t - m) * kLog2e) * inv_s;
}

// A lane's sum relative to the row max (a lane with no element adds 0).
__device__ __forceinline__ float lane_sum_at(float mx, float s, float m) {
#pragma clang fp contract(off)
  return mx == -INFINITY ? 0.f : s * __builtin_amdgcn_exp2f((mx - m) * kLog2e);
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

// Statistics lane `lane`'s max and sum over a row read from memory: chunks
// c = lane + kStatLanes k below nfull (aligned rows), then the elements from
// nfull * P one by one.
template <int DT>
__device__ __forceinline__ void lane_stats(const char* row, int d, bool vec, int lane, float inv_t,
                                           float& mx, float& s) {
  constexpr int P = Elem<DT>::kPer;
  mx = -INFINITY;
  s = 0.f;
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
      float y[P];
      scaled<DT>(v[k], inv_t, y);
      online_update(y, mx, s);
    }
  }
  for (; c < nfull; c += kStatLanes) {
    float y[P];
    scaled<DT>(chunk(c), inv_t, y);
    online_update(y, mx, s);
  }
  for (int e = nfull * P + lane; e < d; e += kStatLanes) {
    const float y[1] = {scaled1(Elem<DT>::load1(row, e), inv_t)};
    online_update(y, mx, s);
  }
}

}  // namespace sp
}  // namespace sgl
