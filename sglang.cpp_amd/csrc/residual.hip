// Residual-path kernels around the attention layer: RMSNorm over hidden
// rows, fused residual add + RMSNorm, and the gated activations of the MLP
// (SiLU / tanh-GELU and multiply). All are one pass over HBM: each row or
// element pair is read once and written once, 16 bytes per lane.
//
// Reference semantics (allen-shaw/sglang.cpp, values computed by FlashInfer
// v0.2.0.post1's norm and activation kernels):
//   RMSNorm::forward / forward_inplace (src/layers/normalization.cu:236-269):
//     out = T(x * rsqrt(mean(x^2) + eps) * w), fp32 math.
//   RMSNorm::fused_add_forward_inplace (src/layers/normalization.cu:386-416):
//     s = x + residual (fp32); residual <- T(s); x <- T(s * rsqrt(mean(s^2)
//     + eps) * w).
//   silu_and_mul / gelu_and_mul (src/layers/activation.cu:8-14, 15-77):
//     out[t, i] = T(act(in[t, i]) * in[t, d + i]) with silu(x) = x / (1 +
//     e^-x) and gelu(x) = 0.5 x (1 + tanh(0.7978845608 (x + 0.044715 x^3))).
// T is bf16 or fp16 (both are built, as in the reference).
#include <math.h>

#include "common.h"

namespace sgl {
namespace {

// Eight consecutive elements starting at e0 of a row of d elements: one
// 16-byte access when the row allows it (VEC), element by element with a
// bound check otherwise (elements past d read as 0 and are not written).
template <int DT, bool VEC, bool NT = false>
__device__ __forceinline__ void load8(const uint16_t* row, int64_t e0, int64_t d, float (&f)[8]) {
  if constexpr (VEC) {
    if constexpr (NT)
      unpack8_t<DT>(__builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(row + e0)), f);
    else
      unpack8_t<DT>(ldg128(row + e0), f);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = e0 + i < d ? to_f32<DT>(row[e0 + i]) : 0.f;
  }
}
template <int DT, bool VEC, bool NT = false>
__device__ __forceinline__ void store8(uint16_t* row, int64_t e0, int64_t d, const float (&f)[8]) {
  if constexpr (VEC) {
    if constexpr (NT)
      __builtin_nontemporal_store(pack8_t<DT>(f), reinterpret_cast<u32x4_t*>(row + e0));
    else
      stg128(row + e0, pack8_t<DT>(f));
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (e0 + i < d) row[e0 + i] = static_cast<uint16_t>(from_f32<DT>(f[i]));
  }
}

// Sum over the 64 lanes of a wave, the same bits in every lane.
__device__ __forceinline__ float wave_sum(float x) { return sum_xor32(sum_xor16(group_sum<16>(x))); }

struct NormArgs {
  uint16_t* x;         // normalised in place unless out is set
  uint16_t* out;       // plain RMSNorm output (may equal x)
  uint16_t* residual;  // fused add: updated in place
  const uint16_t* w;
  int64_t rows, d, x_st, out_st, r_st;
  float eps;
};

constexpr int kRowsPerBlock = 4;  // one wave per row
// Rows are read once and written once: non-temporal loads and stores.
// Measured at the Qwen3-8B shape (fused add, T 8192, hidden 4096) on
// buffers rotated past the 256 MB last-level cache: 4.62 -> 5.38 TB/s; the
// same rows re-run back to back from the cache lose 6.5 -> 5.6 TB/s.
constexpr bool kNormNt = true;

// One wave per row. NV > 0: the row (<= 512 NV elements) stays in registers
// between the sum of squares and the scaling, so HBM sees one read and one
// write. NV == 0: rows longer than 8192 elements take a second pass that
// re-reads the row (for the fused add, the rounded sum it wrote to residual).
template <int DT, int NV, bool VEC, bool ADD>
__global__ void __launch_bounds__(kWave * kRowsPerBlock) rmsnorm_kernel(NormArgs a) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const int lane = threadIdx.x & 63;
  const int64_t d = a.d;
  const uint16_t* xr = a.x + row * a.x_st;
  uint16_t* rr = ADD ? a.residual + row * a.r_st : nullptr;
  uint16_t* outr = ADD ? a.x + row * a.x_st : a.out + row * a.out_st;
  // Chunk j of the row: elements [(64 j + lane) 8, +8).
  auto first = [&](int j, float (&f)[8]) {
    const int64_t e0 = (static_cast<int64_t>(j) * kWave + lane) * 8;
    if (e0 < d) {
      load8<DT, VEC, kNormNt>(xr, e0, d, f);
      if constexpr (ADD) {
        float r[8];
        load8<DT, VEC, kNormNt>(rr, e0, d, r);
#pragma unroll
        for (int i = 0; i < 8; ++i) f[i] += r[i];
        store8<DT, VEC, kNormNt>(rr, e0, d, f);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] = 0.f;
    }
  };
  auto second = [&](int j, float (&f)[8], float scale) {
    const int64_t e0 = (static_cast<int64_t>(j) * kWave + lane) * 8;
    if (e0 >= d) return;
    float w[8];
    load8<DT, VEC>(a.w, e0, d, w);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (f[i] * scale) * w[i];
    store8<DT, VEC, kNormNt>(outr, e0, d, f);
  };
  float ss = 0.f;
  if constexpr (NV > 0) {
    float held[NV][8];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      first(j, held[j]);
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += held[j][i] * held[j][i];
    }
    ss = wave_sum(ss);
    const float scale = 1.0f / sqrtf(ss / static_cast<float>(d) + a.eps);
#pragma unroll
    for (int j = 0; j < NV; ++j) second(j, held[j], scale);
  } else {
    const int nchunks = static_cast<int>((d + 511) / 512);
    for (int j = 0; j < nchunks; ++j) {
      float f[8];
      first(j, f);
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += f[i] * f[i];
    }
    ss = wave_sum(ss);
    const float scale = 1.0f / sqrtf(ss / static_cast<float>(d) + a.eps);
    for (int j = 0; j < nchunks; ++j) {
      const int64_t e0 = (static_cast<int64_t>(j) * kWave + lane) * 8;
      if (e0 >= d) break;
      float f[8];
      load8<DT, VEC>(ADD ? rr : xr, e0, d, f);
      second(j, f, scale);
    }
  }
}

struct ActArgs {
  uint16_t* out;
  const uint16_t* in;
  int64_t tokens, d, in_st, out_st;
  uint32_t chunks_per_row;  // ceil(d / 8)
  int64_t total_chunks;
};

// act(x) * y with act(x) = x * sigmoid(k x): k = 1 is SiLU; for the tanh
// GELU, 0.5 (1 + tanh(u)) = sigmoid(2 u), so gelu(x) = x * sigmoid(2 u) with
// u = 0.7978845608 (x + 0.044715 x^3). sigmoid(z) = 1 / (1 + 2^(-z log2 e))
// on the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32: about one fp32
// ulp each, far below the output's bf16/fp16 rounding; a correctly rounded
// division would make this HBM-bound kernel VALU-bound).
template <int ACT>
__device__ __forceinline__ float act_mul(float x, float y) {
  float z = x;
  if constexpr (ACT == 1) z = 2.0f * 0.7978845608f * (x + 0.044715f * x * x * x);
  const float e = __builtin_amdgcn_exp2f(-z * 1.4426950408889634f);
  return x * __builtin_amdgcn_rcpf(1.0f + e) * y;
}

// Input and output are streamed non-temporally: each element is read or
// written once, and at Qwen3-8B's shape (8192 tokens x 12288) the 604 MB
// pass is larger than the last-level cache, which cached accesses only
// thrash (measured 103.4 -> 92.1 us). The norm kernels keep cached accesses:
// their passes fit that cache and non-temporal ones measured slower there.
template <int DT, int ACT, bool VEC>
__global__ void __launch_bounds__(256) act_and_mul_kernel(ActArgs a) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; c < a.total_chunks;
       c += stride) {
    int64_t t, e0;
    if (a.total_chunks <= 0xffffffffll) {  // 32-bit division, the common case
      const uint32_t cu = static_cast<uint32_t>(c);
      const uint32_t tu = cu / a.chunks_per_row;
      t = tu;
      e0 = static_cast<int64_t>(cu - tu * a.chunks_per_row) * 8;
    } else {
      t = c / a.chunks_per_row;
      e0 = (c - t * a.chunks_per_row) * 8;
    }
    const uint16_t* xr = a.in + t * a.in_st;
    float x[8], y[8];
    load8<DT, VEC, true>(xr, e0, a.d, x);
    load8<DT, VEC, true>(xr + a.d, e0, a.d, y);
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = act_mul<ACT>(x[i], y[i]);
    store8<DT, VEC, true>(a.out + t * a.out_st, e0, a.d, x);
  }
}

// Workgroups for a grid-stride elementwise launch: one 16-byte chunk per
// thread up to 2^28 chunks (measured on MI355X at 8192 x 12288: one chunk per
// thread 5.9 TB/s, six per thread 5.5, 24 per thread 5.2), then a loop.
int64_t elementwise_blocks(int64_t items) {
  int64_t b = (items + 255) / 256;
  return b < 1 ? 1 : (b > (1 << 20) ? (1 << 20) : b);
}

bool dtype_ok(int dtype) { return dtype == SGL_DTYPE_BF16 || dtype == SGL_DTYPE_F16; }

template <int DT, int NV, bool ADD>
void launch_norm_vec(bool vec, const NormArgs& a, hipStream_t s) {
  const dim3 grid(static_cast<uint32_t>((a.rows + kRowsPerBlock - 1) / kRowsPerBlock));
  if (vec)
    hipLaunchKernelGGL((rmsnorm_kernel<DT, NV, true, ADD>), grid, dim3(kWave * kRowsPerBlock), 0, s, a);
  else
    hipLaunchKernelGGL((rmsnorm_kernel<DT, NV, false, ADD>), grid, dim3(kWave * kRowsPerBlock), 0, s, a);
}

template <int DT, bool ADD>
void launch_norm(bool vec, const NormArgs& a, hipStream_t s) {
  const int64_t chunks = (a.d + 511) / 512;
  if (chunks <= 1) launch_norm_vec<DT, 1, ADD>(vec, a, s);
  else if (chunks <= 2) launch_norm_vec<DT, 2, ADD>(vec, a, s);
  else if (chunks <= 4) launch_norm_vec<DT, 4, ADD>(vec, a, s);
  else if (chunks <= 8) launch_norm_vec<DT, 8, ADD>(vec, a, s);
  else if (chunks <= 16) launch_norm_vec<DT, 16, ADD>(vec, a, s);
  else launch_norm_vec<DT, 0, ADD>(vec, a, s);
}

bool vec_ok(const void* p, int64_t stride) { return aligned16(p) && stride % 8 == 0; }

}  // namespace
}  // namespace sgl

using namespace sgl;

extern "C" int sgl_rmsnorm(void* out, const void* x, const void* weight, int64_t rows, int64_t d,
                           int64_t x_stride_row, int64_t out_stride_row, int dtype, float eps,
                           void* stream) {
  if (rows < 0 || d <= 0 || !dtype_ok(dtype)) return rows < 0 || d <= 0 ? SGL_ERR_INVALID_ARG : SGL_ERR_UNSUPPORTED;
  if (rows == 0) return SGL_OK;
  if (!out || !x || !weight || x_stride_row < d || out_stride_row < d) return SGL_ERR_INVALID_ARG;
  if (rows > static_cast<int64_t>(0x7fffffff) * kRowsPerBlock) return SGL_ERR_INVALID_ARG;
  NormArgs a{};
  a.x = static_cast<uint16_t*>(const_cast<void*>(x));
  a.out = static_cast<uint16_t*>(out);
  a.w = static_cast<const uint16_t*>(weight);
  a.rows = rows;
  a.d = d;
  a.x_st = x_stride_row;
  a.out_st = out_stride_row;
  a.eps = eps;
  const bool vec = d % 8 == 0 && vec_ok(x, x_stride_row) && vec_ok(out, out_stride_row) &&
                   aligned16(weight);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == SGL_DTYPE_BF16) launch_norm<SGL_DTYPE_BF16, false>(vec, a, s);
  else launch_norm<SGL_DTYPE_F16, false>(vec, a, s);
  return launch_status();
}

extern "C" int sgl_fused_add_rmsnorm(void* x, void* residual, const void* weight, int64_t rows,
                                     int64_t d, int64_t x_stride_row, int64_t residual_stride_row,
                                     int dtype, float eps, void* stream) {
  if (rows < 0 || d <= 0 || !dtype_ok(dtype)) return rows < 0 || d <= 0 ? SGL_ERR_INVALID_ARG : SGL_ERR_UNSUPPORTED;
  if (rows == 0) return SGL_OK;
  if (!x || !residual || !weight || x_stride_row < d || residual_stride_row < d)
    return SGL_ERR_INVALID_ARG;
  if (rows > static_cast<int64_t>(0x7fffffff) * kRowsPerBlock) return SGL_ERR_INVALID_ARG;
  NormArgs a{};
  a.x = static_cast<uint16_t*>(x);
  a.residual = static_cast<uint16_t*>(residual);
  a.w = static_cast<const uint16_t*>(weight);
  a.rows = rows;
  a.d = d;
  a.x_st = x_stride_row;
  a.r_st = residual_stride_row;
  a.eps = eps;
  const bool vec = d % 8 == 0 && vec_ok(x, x_stride_row) && vec_ok(residual, residual_stride_row) &&
                   aligned16(weight);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == SGL_DTYPE_BF16) launch_norm<SGL_DTYPE_BF16, true>(vec, a, s);
  else launch_norm<SGL_DTYPE_F16, true>(vec, a, s);
  return launch_status();
}

static int act_and_mul(int act, void* out, const void* input, int64_t tokens, int64_t d,
                       int64_t in_stride_row, int64_t out_stride_row, int dtype, void* stream) {
  if (tokens < 0 || d <= 0) return SGL_ERR_INVALID_ARG;
  if (!dtype_ok(dtype)) return SGL_ERR_UNSUPPORTED;
  if (tokens == 0) return SGL_OK;
  if (!out || !input || in_stride_row < 2 * d || out_stride_row < d) return SGL_ERR_INVALID_ARG;
  const int64_t cpr = (d + 7) / 8;
  if (cpr > 0xffffffffll) return SGL_ERR_INVALID_ARG;
  ActArgs a;
  a.out = static_cast<uint16_t*>(out);
  a.in = static_cast<const uint16_t*>(input);
  a.tokens = tokens;
  a.d = d;
  a.in_st = in_stride_row;
  a.out_st = out_stride_row;
  a.chunks_per_row = static_cast<uint32_t>(cpr);
  a.total_chunks = tokens * cpr;
  const bool vec = d % 8 == 0 && vec_ok(input, in_stride_row) && vec_ok(out, out_stride_row);
  const dim3 grid(static_cast<uint32_t>(elementwise_blocks(a.total_chunks)));
  const hipStream_t s = static_cast<hipStream_t>(stream);
#define SGL_ACT_LAUNCH(DT, ACT)                                                               \
  do {                                                                                        \
    if (vec) hipLaunchKernelGGL((act_and_mul_kernel<DT, ACT, true>), grid, dim3(256), 0, s, a); \
    else hipLaunchKernelGGL((act_and_mul_kernel<DT, ACT, false>), grid, dim3(256), 0, s, a);    \
  } while (0)
  if (dtype == SGL_DTYPE_BF16) {
    if (act == 0) SGL_ACT_LAUNCH(SGL_DTYPE_BF16, 0);
    else SGL_ACT_LAUNCH(SGL_DTYPE_BF16, 1);
  } else {
    if (act == 0) SGL_ACT_LAUNCH(SGL_DTYPE_F16, 0);
    else SGL_ACT_LAUNCH(SGL_DTYPE_F16, 1);
  }
#undef SGL_ACT_LAUNCH
  return launch_status();
}

extern "C" int sgl_silu_and_mul(void* out, const void* input, int64_t tokens, int64_t d,
                                int64_t in_stride_row, int64_t out_stride_row, int dtype,
                                void* stream) {
  return act_and_mul(0, out, input, tokens, d, in_stride_row, out_stride_row, dtype, stream);
}

extern "C" int sgl_gelu_and_mul(void* out, const void* input, int64_t tokens, int64_t d,
                                int64_t in_stride_row, int64_t out_stride_row, int dtype,
                                void* stream) {
  return act_and_mul(1, out, input, tokens, d, in_stride_row, out_stride_row, dtype, stream);
}
