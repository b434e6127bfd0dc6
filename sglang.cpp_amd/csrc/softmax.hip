// Temperature softmax of logits rows, the probabilities the Sampler hands to
// the sampling kernels: the reference builds them with three LibTorch
// operations (src/engine/engine.cc:306-308: logits.to(float32), division by
// the per-row temperature, torch::softmax over the vocabulary), i.e. a
// widening copy, an elementwise pass and a softmax that reads its input
// again for the max, the sum and the output.
//
// Here one workgroup takes one row: with a = log2(e) / t and M the row's
// largest logit, s = sum_i 2^(x_i a - M a) and p_i = 2^(fma(x_i, a, -(M a)))
// * (1 / s), the max and the sum taken together (online) as the row streams
// in. For aligned 16-bit logits rows of up to kMaxRegChunks * 8192 elements
// (Qwen3's 151,936 included) a 1024-thread workgroup keeps the raw row in
// registers for the output phase, so HBM sees one read of the logits and one
// write of the probabilities; fp32 logits, longer and unaligned rows go to a
// 512-thread workgroup that reads the row again for the output (mostly from
// the last-level cache).
//
// Accuracy against the exact softmax of float(x) / t (float64): the exp2
// argument x a - M a carries the rounding of a (half an ulp, times |x a|)
// and of M a (half an ulp of |M a|), and one more rounding in the fma, so a
// probability is within ~1e-5 relative for scaled logits |x / t| up to
// ~100; the fp32 sum adds below ~1e-5 for rows of this length. (The
// exponent as one fma of the raw logit is two vector operations per element
// fewer than scaling, subtracting and multiplying by log2 e.)
#include <math.h>

#include "common.h"
#include "sampler_prob.h"

namespace sgl {
namespace {

using sp::Elem;

// Streaming rows: 512 threads, thread t runs the statistics lanes t and
// t + 512 of sampler_prob.h.
constexpr int kSmThreads = sp::kStatLanes / 2;
constexpr int kSmWaves = kSmThreads / kWave;
// Register-held rows: 1024 threads (four waves per SIMD, up to 128 VGPRs
// each), at most kMaxRegChunks 16-byte chunks (80 VGPRs) per lane. Measured
// against 512 threads holding twice the chunks (two waves per SIMD): 53.8 ->
// 50.9 us on HBM-resident Qwen3 rows, 42.9 -> 40.1 us cache-resident.
constexpr int kMaxRegChunks = 20;
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

// The row read twice (statistics, then output) in sp::lane_stats' order for
// lanes tid and tid + 512, so the statistics are the same bits as the
// register-held kernel's and the draws from logits'.
template <int DT>
__global__ void __launch_bounds__(kSmThreads) softmax_temperature_stream(SoftmaxArgs a) {
  __shared__ float red[2 * kSmWaves];
  constexpr int P = Elem<DT>::kPer;
  constexpr int B = 16 / P;  // bytes per element
  const int r = blockIdx.x;
  const char* row = static_cast<const char*>(a.logits) + static_cast<int64_t>(r) * a.x_st * B;
  float* prow = a.probs + static_cast<int64_t>(r) * a.p_st;
  const int d = static_cast<int>(a.d);
  const int nfull = a.vec ? d / P : 0;  // chunks taken 16 bytes at a time
  const int e_tail = nfull * P;         // first element taken one by one
  const int tid = threadIdx.x;
  const float t = a.temps ? a.temps[r] : a.temp;
  const float sc = sp::exp2_scale(t);

  const sp::LaneStats st0 = sp::lane_stats<DT>(row, d, a.vec, tid, sc);
  const sp::LaneStats st1 = sp::lane_stats<DT>(row, d, a.vec, tid + kSmThreads, sc);
  const float m = sp::block_max2<kSmWaves>(st0.mx, st1.mx, red);
  const float inv_s = 1.0f / sp::block_sum2<kSmWaves>(sp::lane_sum_at(st0, m, sc),
                                                      sp::lane_sum_at(st1, m, sc), red);
  const float nb = sp::exp2_offset(m, sc);

  // The probabilities.
  for (int c = tid; c < nfull; c += kSmThreads) {
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(row + static_cast<int64_t>(c) * 16);
    float p[P];
#pragma unroll
    for (int j = 0; j < P; ++j) p[j] = sp::prob(Elem<DT>::at(v, j), sc, nb, inv_s);
#pragma unroll
    for (int q = 0; q < P / 4; ++q)
      *reinterpret_cast<f32x4_t*>(prow + c * P + 4 * q) =
          f32x4_t{p[4 * q], p[4 * q + 1], p[4 * q + 2], p[4 * q + 3]};
  }
  for (int e = e_tail + tid; e < d; e += kSmThreads)
    prow[e] = sp::prob(Elem<DT>::load1(row, e), sc, nb, inv_s);
}

// Register-held rows (aligned 16-bit logits): thread t is the statistics
// lane t and holds its chunks c = t + 1024 k, k < NC (a row of 151,936
// logits is 19 chunks, 76 VGPRs, per lane), loaded with buffer loads (one
// lane offset, the chunk step as the scalar offset, reads past the row
// return 0). Same statistics order, so the same bits, as the streaming
// kernel and the draws from logits.
template <int DT, int NC>
__global__ void __launch_bounds__(sp::kStatLanes) softmax_temperature_held(SoftmaxArgs a) {
  __shared__ float red[sp::kStatWaves];
  constexpr int T = sp::kStatLanes;
  constexpr int P = Elem<DT>::kPer;
  constexpr int B = 16 / P;  // bytes per element
  const int r = blockIdx.x;
  const char* row = static_cast<const char*>(a.logits) + static_cast<int64_t>(r) * a.x_st * B;
  float* prow = a.probs + static_cast<int64_t>(r) * a.p_st;
  const int d = static_cast<int>(a.d);
  const int nfull = d / P;          // aligned rows only
  const int e_tail = nfull * P;
  const int tid = threadIdx.x;
  const float t = a.temps ? a.temps[r] : a.temp;
  const float sc = sp::exp2_scale(t);

  u32x4_t held[NC];
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(row), 0, d * B, kRawBufferWord3);
#pragma unroll
  for (int k = 0; k < NC; ++k)
    held[k] = __builtin_bit_cast(
        u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, tid * 16, k * T * 16, 0));
  const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(prow, 0, d * 4, kRawBufferWord3);
  sp::LaneStats st;
#pragma unroll
  for (int k = 0; k < NC; ++k)
    if (tid + k * T < nfull) {
      float x[P];
      sp::unpack<DT>(held[k], x);
      sp::online_update(x, sc, st);
    }
  for (int e = e_tail + tid; e < d; e += T) {
    const float x[1] = {Elem<DT>::load1(row, e)};
    sp::online_update(x, sc, st);
  }
  const float m = sp::block_max<sp::kStatWaves>(st.mx, red);
  const float inv_s = 1.0f / sp::block_sum<sp::kStatWaves>(sp::lane_sum_at(st, m, sc), red);
  const float nb = sp::exp2_offset(m, sc);

  // The probabilities, recomputed from the packed row: without this barrier
  // the compiler keeps the fp32 values of the statistics pass alive instead
  // (twice the registers).
#pragma unroll
  for (int k = 0; k < NC; ++k) asm volatile("" : "+v"(held[k]));
#pragma unroll
  for (int k = 0; k < NC; ++k)
    if (tid + k * T < nfull) {
      float p[P];
#pragma unroll
      for (int j = 0; j < P; ++j) p[j] = sp::prob(Elem<DT>::at(held[k], j), sc, nb, inv_s);
#pragma unroll
      for (int q = 0; q < P / 4; ++q)
        __builtin_amdgcn_raw_buffer_store_b128(
            __builtin_bit_cast(u32x4_t, f32x4_t{p[4 * q], p[4 * q + 1], p[4 * q + 2], p[4 * q + 3]}),
            prs, tid * (4 * P) + 16 * q, k * T * 4 * P, 0);
    }
  for (int e = e_tail + tid; e < d; e += T)
    prow[e] = sp::prob(Elem<DT>::load1(row, e), sc, nb, inv_s);
}

template <int DT>
int launch_softmax(const SoftmaxArgs& a, hipStream_t s) {
  constexpr int P = Elem<DT>::kPer;
  const int64_t per_lane = (a.d / P + sp::kStatLanes - 1) / sp::kStatLanes;  // chunks per lane
  const dim3 grid(static_cast<uint32_t>(a.batch));
  const dim3 held(sp::kStatLanes);
  if constexpr (DT == SGL_DTYPE_F32) {
    hipLaunchKernelGGL((softmax_temperature_stream<DT>), grid, dim3(kSmThreads), 0, s, a);
    return launch_status();
  }
  if (!a.vec || per_lane > kMaxRegChunks)
    hipLaunchKernelGGL((softmax_temperature_stream<DT>), grid, dim3(kSmThreads), 0, s, a);
  else if (per_lane <= 4)
    hipLaunchKernelGGL((softmax_temperature_held<DT, 4>), grid, held, 0, s, a);
  else if (per_lane <= 8)
    hipLaunchKernelGGL((softmax_temperature_held<DT, 8>), grid, held, 0, s, a);
  else if (per_lane <= 12)
    hipLaunchKernelGGL((softmax_temperature_held<DT, 12>), grid, held, 0, s, a);
  else if (per_lane <= 16)
    hipLaunchKernelGGL((softmax_temperature_held<DT, 16>), grid, held, 0, s, a);
  else
    hipLaunchKernelGGL((softmax_temperature_held<DT, kMaxRegChunks>), grid, held, 0, s, a);
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
