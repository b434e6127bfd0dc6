// Temperature softmax of logits rows, the probabilities the Sampler hands to
// the sampling kernels: the reference builds them with three LibTorch
// operations (src/engine/engine.cc:306-308: logits.to(float32), division by
// the per-row temperature, torch::softmax over the vocabulary), i.e. a
// widening copy, an elementwise pass and a softmax that reads its input
// again for the max, the sum and the output.
//
// Here one 512-thread workgroup takes one row: y_i = float(x_i) * (1 / t),
// m = max_i y_i, s = sum_i 2^((y_i - m) log2 e), p_i = 2^((y_i - m) log2 e)
// * (1 / s), the max and the sum taken together (online) as the row streams
// in. For 16-bit logits rows of up to kMaxRegChunks * 4096 elements
// (Qwen3's 151,936 included) the raw row stays in registers for the output
// phase, so HBM sees one read of the logits and one write of the
// probabilities; fp32 logits and longer rows read the row again for the
// output (mostly from the last-level cache).
//
// Accuracy against the exact softmax of float(x) / t (float64): y carries
// half an ulp of |y| from the reciprocal-multiply (about 6e-8 |y|), the exp2
// argument a few ulp of |y - m|, so a probability is within ~1e-5 relative
// for logits up to ~100 in magnitude; the fp32 sum adds below ~1e-5 for rows
// of this length.
#include <math.h>

#include "common.h"

namespace sgl {
namespace {

// 512 threads (two waves per SIMD, up to 256 VGPRs each): a 16-bit row of
// 151,936 logits is 38 16-byte chunks (152 VGPRs) per lane.
constexpr int kSmThreads = 512;
constexpr int kSmWaves = kSmThreads / kWave;
constexpr int kMaxRegChunks = 40;  // 16-byte chunks a lane holds (160 VGPRs)
// Word 3 of a raw buffer resource on gfx950 (32-bit data format, no
// swizzle, unit stride): plain byte-addressed loads with a range check.
constexpr int kRawBufferWord3 = 0x00020000;

struct SoftmaxArgs {
  float* probs;
  const void* logits;
  const float* temps;  // [batch] or null
  float temp;          // used when temps is null
  int64_t batch, d, p_st, x_st;  // strides in elements
  bool vec;            // 16-byte aligned rows (base and stride of both)
};

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

// Fixed-order workgroup reductions: wave reduction, then every wave folds
// the 8 wave values in order.
__device__ __forceinline__ float block_max(float x, float* sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, kWave));
  __syncthreads();  // earlier readers of sh are done
  if (lane == 0) sh[wave] = x;
  __syncthreads();
  float m = sh[0];
#pragma unroll
  for (int w = 1; w < kSmWaves; ++w) m = fmaxf(m, sh[w]);
  return m;
}

__device__ __forceinline__ float block_sum(float x, float* sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, kWave);
  __syncthreads();
  if (lane == 0) sh[wave] = x;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < kSmWaves; ++w) s += sh[w];
  return s;
}

constexpr float kLog2e = 1.4426950408889634f;

// Running (max, sum of 2^((y - max) log2e)) of a lane, updated by n values.
template <int N>
__device__ __forceinline__ void online_update(const float (&y)[N], float& mx, float& s) {
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

// Chunk c (elements [P c, P c + P), whole and inside the row) through
// 16-byte global loads: the streaming path.
template <int DT>
__device__ __forceinline__ u32x4_t load_chunk(const char* row, int c) {
  return *reinterpret_cast<const u32x4_t*>(row + static_cast<int64_t>(c) * 16);
}

// The elements of a chunk as fp32 scaled by 1 / t.
template <int DT>
__device__ __forceinline__ void scaled(const u32x4_t& v, float inv_t, float (&y)[Elem<DT>::kPer]) {
#pragma unroll
  for (int j = 0; j < Elem<DT>::kPer; ++j) y[j] = Elem<DT>::at(v, j) * inv_t;
}

// NC > 0 (16-byte aligned rows): the lane's whole chunks c = tid + T k,
// k < NC, stay in registers (buffer loads: one lane offset, the chunk step
// as the scalar offset, reads past the row return 0); NC == 0: every phase
// streams the row (aligned rows by 16-byte loads, others element by
// element). The partial last chunk of a row (d % P elements) belongs to one
// lane, which takes it element by element.
template <int DT, int NC>
__global__ void __launch_bounds__(kSmThreads) softmax_temperature_kernel(SoftmaxArgs a) {
  __shared__ float red[kSmWaves];
  constexpr int P = Elem<DT>::kPer;
  constexpr int B = 16 / P;  // bytes per element
  const int r = blockIdx.x;
  const char* row = static_cast<const char*>(a.logits) + static_cast<int64_t>(r) * a.x_st * B;
  float* prow = a.probs + static_cast<int64_t>(r) * a.p_st;
  const int d = static_cast<int>(a.d);
  const int nfull = a.vec ? d / P : 0;      // chunks taken 16 bytes at a time
  const int e_tail = nfull * P;             // first element taken one by one
  const int tid = threadIdx.x;
  const float t = a.temps ? a.temps[r] : a.temp;
  const float inv_t = 1.0f / t;

  u32x4_t held[NC > 0 ? NC : 1];
  __amdgpu_buffer_rsrc_t prs;
  if constexpr (NC > 0) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(row), 0, d * B, kRawBufferWord3);
#pragma unroll
    for (int k = 0; k < NC; ++k)
      held[k] = __builtin_bit_cast(
          u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, tid * 16, k * kSmThreads * 16, 0));
    prs = __builtin_amdgcn_make_buffer_rsrc(prow, 0, d * 4, kRawBufferWord3);
  }

  // Phase 1: running max and sum as the row arrives.
  float mx = -INFINITY, s = 0.f;
  if constexpr (NC > 0) {
#pragma unroll
    for (int k = 0; k < NC; ++k)
      if (tid + k * kSmThreads < nfull) {
        float y[P];
        scaled<DT>(held[k], inv_t, y);
        online_update(y, mx, s);
      }
  } else {
    for (int c = tid; c < nfull; c += kSmThreads) {
      float y[P];
      scaled<DT>(load_chunk<DT>(row, c), inv_t, y);
      online_update(y, mx, s);
    }
  }
  // Elements past the whole chunks (the partial chunk, or every element of
  // an unaligned row), one by one.
  for (int e = e_tail + tid; e < d; e += kSmThreads) {
    const float y[1] = {Elem<DT>::load1(row, e) * inv_t};
    online_update(y, mx, s);
  }
  const float m = block_max(mx, red);
  // The lane's sum relative to the row max (a lane with no element adds 0).
  const float sl = mx == -INFINITY ? 0.f : s * __builtin_amdgcn_exp2f((mx - m) * kLog2e);
  const float inv_s = 1.0f / block_sum(sl, red);

  // Phase 2: the probabilities.
  auto prob = [&](float x) { return __builtin_amdgcn_exp2f((x * inv_t - m) * kLog2e) * inv_s; };
  if constexpr (NC > 0) {
    // Recompute y from the packed row: without this barrier the compiler
    // keeps phase 1's fp32 values alive instead (twice the registers).
#pragma unroll
    for (int k = 0; k < NC; ++k) asm volatile("" : "+v"(held[k]));
#pragma unroll
    for (int k = 0; k < NC; ++k)
      if (tid + k * kSmThreads < nfull) {
        float p[P];
#pragma unroll
        for (int j = 0; j < P; ++j) p[j] = prob(Elem<DT>::at(held[k], j));
#pragma unroll
        for (int q = 0; q < P / 4; ++q)
          __builtin_amdgcn_raw_buffer_store_b128(
              __builtin_bit_cast(u32x4_t, f32x4_t{p[4 * q], p[4 * q + 1], p[4 * q + 2], p[4 * q + 3]}),
              prs, tid * (4 * P) + 16 * q, k * kSmThreads * 4 * P, 0);
      }
  } else {
    for (int c = tid; c < nfull; c += kSmThreads) {
      const u32x4_t v = load_chunk<DT>(row, c);
      float p[P];
#pragma unroll
      for (int j = 0; j < P; ++j) p[j] = prob(Elem<DT>::at(v, j));
#pragma unroll
      for (int q = 0; q < P / 4; ++q)
        *reinterpret_cast<f32x4_t*>(prow + c * P + 4 * q) =
            f32x4_t{p[4 * q], p[4 * q + 1], p[4 * q + 2], p[4 * q + 3]};
    }
  }
  for (int e = e_tail + tid; e < d; e += kSmThreads) prow[e] = prob(Elem<DT>::load1(row, e));
}

template <int DT>
int launch_softmax(const SoftmaxArgs& a, hipStream_t s) {
  constexpr int P = Elem<DT>::kPer;
  const int64_t per_lane = (a.d / P + kSmThreads - 1) / kSmThreads;  // whole chunks per lane
  const dim3 grid(static_cast<uint32_t>(a.batch)), block(kSmThreads);
  // Registers hold aligned 16-bit rows of up to kMaxRegChunks chunks per
  // lane; fp32 logits, longer and unaligned rows stream.
  if constexpr (DT == SGL_DTYPE_F32) {
    hipLaunchKernelGGL((softmax_temperature_kernel<DT, 0>), grid, block, 0, s, a);
    return launch_status();
  }
  if (per_lane > kMaxRegChunks || !a.vec)
    hipLaunchKernelGGL((softmax_temperature_kernel<DT, 0>), grid, block, 0, s, a);
  else if (per_lane <= 8)
    hipLaunchKernelGGL((softmax_temperature_kernel<DT, 8>), grid, block, 0, s, a);
  else if (per_lane <= 16)
    hipLaunchKernelGGL((softmax_temperature_kernel<DT, 16>), grid, block, 0, s, a);
  else if (per_lane <= 24)
    hipLaunchKernelGGL((softmax_temperature_kernel<DT, 24>), grid, block, 0, s, a);
  else if (per_lane <= 32)
    hipLaunchKernelGGL((softmax_temperature_kernel<DT, 32>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((softmax_temperature_kernel<DT, kMaxRegChunks>), grid, block, 0, s, a);
  return launch_status();
}

}  // namespace
}  // namespace sgl

using namespace sgl;

extern "C" int sgl_softmax_temperature(float* probs, int64_t probs_stride_row, const void* logits,
                                       int64_t logits_stride_row, int logits_dtype,
                                       const float* temperatures, float temperature,
                                       int64_t batch, int64_t vocab, void* stream) {
  if (batch < 0 || vocab <= 0 || probs_stride_row < vocab || logits_stride_row < vocab)
    return SGL_ERR_INVALID_ARG;
  if (batch == 0) return SGL_OK;
  if (!probs || !logits) return SGL_ERR_INVALID_ARG;
  // 32-bit element and byte offsets within a row (buffer ranges).
  if (batch > 0x7fffffff || vocab > (0x7fffffff / 4)) return SGL_ERR_UNSUPPORTED;
  if (!temperatures && !(temperature > 0.f)) return SGL_ERR_INVALID_ARG;
  int esize;
  if (logits_dtype == SGL_DTYPE_BF16 || logits_dtype == SGL_DTYPE_F16) esize = 2;
  else if (logits_dtype == SGL_DTYPE_F32) esize = 4;
  else return SGL_ERR_UNSUPPORTED;
  SoftmaxArgs a;
  a.probs = probs;
  a.logits = logits;
  a.temps = temperatures;
  a.temp = temperature;
  a.batch = batch;
  a.d = vocab;
  a.p_st = probs_stride_row;
  a.x_st = logits_stride_row;
  a.vec = aligned16(probs) && aligned16(logits) && (probs_stride_row * 4) % 16 == 0 &&
          (logits_stride_row * esize) % 16 == 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (logits_dtype == SGL_DTYPE_BF16) return launch_softmax<SGL_DTYPE_BF16>(a, s);
  if (logits_dtype == SGL_DTYPE_F16) return launch_softmax<SGL_DTYPE_F16>(a, s);
  return launch_softmax<SGL_DTYPE_F32>(a, s);
}
