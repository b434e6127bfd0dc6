// q/k RMSNorm, NeoX RoPE, and the fused RoPE + qk-norm + KV-store pass.
//
// Reference semantics:
//   RMSNorm per (token, head) row: fused_qk_rmsnorm_3d_strided_vec_kernel
//     (src/layers/normalization.cu:99-170): s = sum(x^2) in fp32,
//     scale = rsqrt(s / d + eps), x <- T((x * scale) * w), T = bf16 or fp16
//     for the standalone norm and RoPE (the reference dispatches both); the
//     fused pass below writes the bf16 pool and is bf16.
//   RoPE: rotate-half with a half-width fp32 cos/sin cache
//     (src/layers/rotary_embedding.cu:50-66): for i < h = rotary_dim / 2,
//     x'[i] = x[i] c_i - x[i+h] s_i, x'[i+h] = x[i+h] c_i + x[i] s_i.
//   Order inside AttentionLayer::forward (src/layers/attention_layer.cc:27-47):
//     norm (bf16 written back) -> RoPE (bf16 written back) -> store_kv.
//
// Layout on gfx950: a row of D bf16 is spread over D/8 lanes (16 bytes per
// lane, one 128-bit load), so a wave64 holds 64*8/D rows. The RoPE partner
// element i +/- D/2 lives in the lane D/16 positions away in the same row
// group and is fetched with one cross-lane exchange per 32-bit word. The
// fused pass reads every qkv byte once and writes q, k, the K-cache row and
// the V-cache row once, which is the minimum traffic for the three
// reference kernels together.
#include <math.h>

#include "common.h"

namespace sgl {
namespace {

// --- per-row building blocks (LPR = lanes per row = D / 8) ------------------

// DT: the 16-bit element type of the rows (SGL_DTYPE_BF16 / SGL_DTYPE_F16),
// as the reference dispatches both (normalization.cu:346-372,
// rotary_embedding.cu:124-168).
template <int LPR, int DT>
__device__ __forceinline__ void rmsnorm8(float (&x)[8], const uint16_t* __restrict__ w,
                                         int lane_in_row, float inv_d, float eps) {
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss += x[i] * x[i];
  ss = group_sum<LPR>(ss);
  const float scale = rsqrtf(ss * inv_d + eps);
  float wf[8];
  unpack8_t<DT>(ldg128(w + lane_in_row * 8), wf);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = round_t<DT>((x[i] * scale) * wf[i]);
}

// One rotated value: x c + p' s, p' the partner with its sign flipped on
// the first half (x c - p s there: negation is exact), as one multiply and
// one fused multiply-add wherever RoPE is applied, so every path rounds
// alike.
__device__ __forceinline__ float rope_one(float x, float p_signed, float c, float s) {
  return fmaf(p_signed, s, x * c);
}

// Sign bits of both 16-bit halves of a packed word (bf16 and fp16 alike).
constexpr uint32_t kSign2 = 0x80008000u;

// Rotate-half RoPE of the 8 values this lane holds; x must hold DT values.
template <int LPR, int DT>
__device__ __forceinline__ void rope8(float (&x)[8], const float* __restrict__ cos_row,
                                      const float* __restrict__ sin_row, int lane_in_row) {
  constexpr int HALF = LPR / 2;
  const bool first = lane_in_row < HALF;
  const int j = first ? lane_in_row : lane_in_row - HALF;
  // Partner values: exchange packed 16-bit words (exact, x is DT-valued).
  float p[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w = pack2_t<DT>(x[2 * i], x[2 * i + 1]);
    uint32_t pw;
    if constexpr (HALF == 8) {
      pw = dpp_u32<0x128>(w);  // lane ^ 8 inside the 16-lane row
    } else {
      pw = static_cast<uint32_t>(__shfl_xor(static_cast<int>(w), HALF, kWave));
    }
    pw ^= first ? kSign2 : 0u;
    p[2 * i] = to_f32<DT>(pw & 0xffffu);
    p[2 * i + 1] = to_f32<DT>(pw >> 16);
  }
  const f32x4_t c0 = *reinterpret_cast<const f32x4_t*>(cos_row + j * 8);
  const f32x4_t c1 = *reinterpret_cast<const f32x4_t*>(cos_row + j * 8 + 4);
  const f32x4_t s0 = *reinterpret_cast<const f32x4_t*>(sin_row + j * 8);
  const f32x4_t s1 = *reinterpret_cast<const f32x4_t*>(sin_row + j * 8 + 4);
  const float c[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
  const float s[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = rope_one(x[i], p[i], c[i], s[i]);
}

// --- cos/sin cache ----------------------------------------------------------

// inv_freq is computed once on the host (64 values for head_dim 128) with the
// reference constructor's fp32 statements, so every device builds the
// identical table: inv_freq = 1 / base^(float(2k) / float(rotary_dim)).
constexpr int kMaxHalfRotary = 256;
struct InvFreq {
  float v[kMaxHalfRotary];
};

__global__ void __launch_bounds__(256) cos_sin_cache_kernel(float* __restrict__ cos_cache,
                                                            float* __restrict__ sin_cache,
                                                            int64_t max_pos, int half,
                                                            InvFreq inv) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= max_pos * half) return;
  const int64_t pos = i / half;
  const int k = static_cast<int>(i - pos * half);
  const float f = static_cast<float>(pos) * inv.v[k];  // freqs = outer(t, inv_freq)
  cos_cache[i] = cosf(f);
  sin_cache[i] = sinf(f);
}

// --- standalone qk RMSNorm --------------------------------------------------

template <int LPR, int DT>
__global__ void __launch_bounds__(256) qk_rmsnorm_kernel(
    uint16_t* __restrict__ q, uint16_t* __restrict__ k, const uint16_t* __restrict__ qw,
    const uint16_t* __restrict__ kw, int64_t tokens, int64_t q_heads, int64_t k_heads,
    int64_t q_st, int64_t q_sh, int64_t k_st, int64_t k_sh, float inv_d, float eps) {
  constexpr int ROWS = 256 / LPR;
  const int lane_in_row = threadIdx.x % LPR;
  const int64_t q_rows = tokens * q_heads;
  const int64_t total = q_rows + tokens * k_heads;
  const int64_t job = static_cast<int64_t>(blockIdx.x) * ROWS + threadIdx.x / LPR;
  // Whole row groups exit together, so the group reductions stay well formed.
  if (job >= total) return;
  uint16_t* row;
  const uint16_t* w;
  if (job < q_rows) {
    const int64_t t = job / q_heads;
    row = q + t * q_st + (job - t * q_heads) * q_sh;
    w = qw;
  } else {
    const int64_t kj = job - q_rows;
    const int64_t t = kj / k_heads;
    row = k + t * k_st + (kj - t * k_heads) * k_sh;
    w = kw;
  }
  float x[8];
  unpack8_t<DT>(ldg128(row + lane_in_row * 8), x);
  rmsnorm8<LPR, DT>(x, w, lane_in_row, inv_d, eps);
  stg128(row + lane_in_row * 8, pack8_t<DT>(x));
}

// Any d: one wave per row, scalar element loop.
template <int DT>
__global__ void __launch_bounds__(256) qk_rmsnorm_generic_kernel(
    uint16_t* __restrict__ q, uint16_t* __restrict__ k, const uint16_t* __restrict__ qw,
    const uint16_t* __restrict__ kw, int64_t tokens, int64_t q_heads, int64_t k_heads,
    int64_t d, int64_t q_st, int64_t q_sh, int64_t k_st, int64_t k_sh, float eps) {
  const int lane = threadIdx.x % kWave;
  const int64_t q_rows = tokens * q_heads;
  const int64_t total = q_rows + tokens * k_heads;
  const int64_t job = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
  if (job >= total) return;
  uint16_t* row;
  const uint16_t* w;
  if (job < q_rows) {
    const int64_t t = job / q_heads;
    row = q + t * q_st + (job - t * q_heads) * q_sh;
    w = qw;
  } else {
    const int64_t kj = job - q_rows;
    const int64_t t = kj / k_heads;
    row = k + t * k_st + (kj - t * k_heads) * k_sh;
    w = kw;
  }
  float ss = 0.f;
  for (int64_t i = lane; i < d; i += kWave) {
    const float v = to_f32<DT>(row[i]);
    ss += v * v;
  }
  ss = group_sum<kWave>(ss);
  const float scale = rsqrtf(ss / static_cast<float>(d) + eps);
  for (int64_t i = lane; i < d; i += kWave) {
    const float v = to_f32<DT>(row[i]);
    row[i] = static_cast<uint16_t>(from_f32<DT>((v * scale) * to_f32<DT>(w[i])));
  }
}

// --- standalone RoPE --------------------------------------------------------

template <int LPR, int DT>
__global__ void __launch_bounds__(256) rope_kernel(
    uint16_t* __restrict__ q, uint16_t* __restrict__ k, const float* __restrict__ cos_cache,
    const float* __restrict__ sin_cache, const int32_t* __restrict__ positions, int64_t nnz,
    int64_t q_heads, int64_t kv_heads, int64_t q_st, int64_t q_sh, int64_t k_st, int64_t k_sh) {
  constexpr int ROWS = 256 / LPR;
  constexpr int D = LPR * 8;
  const int lane_in_row = threadIdx.x % LPR;
  const int64_t q_rows = nnz * q_heads;
  const int64_t total = q_rows + nnz * kv_heads;
  const int64_t job = static_cast<int64_t>(blockIdx.x) * ROWS + threadIdx.x / LPR;
  if (job >= total) return;
  uint16_t* row;
  int64_t t;
  if (job < q_rows) {
    t = job / q_heads;
    row = q + t * q_st + (job - t * q_heads) * q_sh;
  } else {
    const int64_t kj = job - q_rows;
    t = kj / kv_heads;
    row = k + t * k_st + (kj - t * kv_heads) * k_sh;
  }
  const int64_t pos = positions[t];
  float x[8];
  unpack8_t<DT>(ldg128(row + lane_in_row * 8), x);
  rope8<LPR, DT>(x, cos_cache + pos * (D / 2), sin_cache + pos * (D / 2), lane_in_row);
  stg128(row + lane_in_row * 8, pack8_t<DT>(x));
}

// Any head_dim / rotary_dim / cache width: one workgroup per row, as the
// reference fallback kernel (src/layers/rotary_embedding.cu:9-67). All reads
// of the row finish before any write (barrier), so the update is in place.
template <int DT>
__global__ void __launch_bounds__(128) rope_generic_kernel(
    uint16_t* __restrict__ q, uint16_t* __restrict__ k, const float* __restrict__ cos_cache,
    const float* __restrict__ sin_cache, const int32_t* __restrict__ positions, int64_t nnz,
    int64_t q_heads, int64_t kv_heads, int64_t rotary_dim, int64_t head_dim,
    int64_t cos_width, int64_t q_st, int64_t q_sh, int64_t k_st, int64_t k_sh) {
  const int64_t row_id = blockIdx.x;
  const int64_t q_rows = nnz * q_heads;
  uint16_t* row;
  int64_t t;
  if (row_id < q_rows) {
    t = row_id / q_heads;
    row = q + t * q_st + (row_id - t * q_heads) * q_sh;
  } else {
    const int64_t kj = row_id - q_rows;
    t = kj / kv_heads;
    row = k + t * k_st + (kj - t * kv_heads) * k_sh;
  }
  const int64_t pos = positions[t];
  const int64_t half = rotary_dim / 2;
  constexpr int kMaxPerThread = 8;  // head_dim <= 1024 with 128 threads
  float out[kMaxPerThread];
  int n = 0;
  for (int64_t i = threadIdx.x; i < rotary_dim && n < kMaxPerThread; i += blockDim.x, ++n) {
    const bool first = i < half;
    const int64_t pair = first ? i : i - half;
    const int64_t other = first ? i + half : i - half;
    const int64_t ci = cos_width == rotary_dim ? i : pair;
    const float v = to_f32<DT>(row[i]);
    const float o = to_f32<DT>(row[other]);
    const float c = cos_cache[pos * cos_width + ci];
    const float s = sin_cache[pos * cos_width + ci];
    out[n] = rope_one(v, first ? -o : o, c, s);
  }
  __syncthreads();
  n = 0;
  for (int64_t i = threadIdx.x; i < rotary_dim && n < kMaxPerThread; i += blockDim.x, ++n) {
    row[i] = static_cast<uint16_t>(from_f32<DT>(out[n]));
  }
}

// --- fused qk-norm + RoPE + KV store ---------------------------------------

// Row jobs per token: [0, Hq) q rows, [Hq, Hq+Hkv) k rows, [Hq+Hkv, Hq+2Hkv) v rows.
// blocks_per_token consecutive blocks cover the rows of kFusedTokensPerBlock
// consecutive tokens (the last block's spare rows idle), so the token index
// is one scalar division; a thread takes the same row of each of those
// tokens. Loads go out in two waves before any math: every token's row,
// slot and position, then (once the positions are in) the weight and the
// cos/sin rows, so a lane waits for two memory latencies for all its rows
// (measured at config 3: 28.0 -> 26.7 us for the two waves, 25.9 -> 24.9 us
// for the scalar token index and one rounding per pair, 24.9 -> 23.3 us for
// two tokens per thread; four measured slower).
constexpr int kFusedTokensPerBlock = 2;
// The qkv rows are read once and the q rows and the K/V pool rows written
// once: non-temporal loads and stores. Measured at config 3 on buffers
// rotated past the 256 MB last-level cache (HBM-resident): 4.46 -> 5.20
// TB/s (1, 3 and 4 tokens per thread: 5.03, 5.13, 5.01); the same buffers
// re-run back to back from the cache lose 5.5-5.9 -> 5.3 TB/s.
constexpr bool kFusedNtLoad = true;
constexpr bool kFusedNtStore = true;

template <int LPR>
__global__ void __launch_bounds__(256) fused_qknorm_rope_store_kernel(
    uint16_t* __restrict__ qkv, int64_t qkv_st, uint16_t* __restrict__ k_cache,
    uint16_t* __restrict__ v_cache, const uint16_t* __restrict__ qw,
    const uint16_t* __restrict__ kw, const float* __restrict__ cos_cache,
    const float* __restrict__ sin_cache, const int32_t* __restrict__ positions,
    const int32_t* __restrict__ out_loc, int hq, int hkv, int blocks_per_token, float eps,
    bool k_back, int64_t num_tokens) {
  constexpr int ROWS = 256 / LPR;
  constexpr int D = LPR * 8;
  constexpr int HALF = LPR / 2;
  constexpr int NT = kFusedTokensPerBlock;
  const int lane_in_row = threadIdx.x % LPR;
  const int rows_per_token = hq + 2 * hkv;
  const int64_t tb = blockIdx.x / static_cast<uint32_t>(blocks_per_token);
  const int r = static_cast<int>(blockIdx.x - tb * blocks_per_token) * ROWS + threadIdx.x / LPR;
  if (r >= rows_per_token) return;
  const bool is_v = r >= hq + hkv;
  const bool is_q = r < hq;
  const uint16_t* w = is_q ? qw : kw;
  // Addresses are a workgroup-uniform 64-bit row base (the token is uniform)
  // plus a 32-bit lane offset, so each access is one scalar-base
  // instruction and no per-lane 64-bit address is held.
  const uint32_t lane_off = static_cast<uint32_t>(r * D + lane_in_row * 8);
  u32x4_t raw[NT];
  int64_t slot[NT], pos[NT];
  uint16_t* rowb[NT];
#pragma unroll
  for (int k = 0; k < NT; ++k) {
    const int64_t t = min(tb * NT + k, num_tokens - 1);
    rowb[k] = qkv + t * qkv_st;
    raw[k] = ldg128_nt<kFusedNtLoad>(rowb[k] + lane_off);
    slot[k] = out_loc[t];
    pos[k] = positions[t];
  }
  const uint32_t head_off = static_cast<uint32_t>(lane_in_row * 8);
  if (is_v) {  // v row: raw copy into the cache
    const uint32_t h_off = static_cast<uint32_t>((r - hq - hkv) * D) + head_off;
#pragma unroll
    for (int k = 0; k < NT; ++k)
      if (tb * NT + k < num_tokens) stg128_nt<kFusedNtStore>(v_cache + slot[k] * hkv * D + h_off, raw[k]);
    return;
  }
  float wf[8];
  if (w != nullptr) unpack8(ldg128(w + lane_in_row * 8), wf);
  const bool first = lane_in_row < HALF;
  const uint32_t psign = first ? kSign2 : 0u;
  const int jj = first ? lane_in_row : lane_in_row - HALF;
  f32x4_t c0[NT], c1[NT], s0[NT], s1[NT];
#pragma unroll
  for (int k = 0; k < NT; ++k) {
    const float* cr = cos_cache + pos[k] * (D / 2) + jj * 8;
    const float* sr = sin_cache + pos[k] * (D / 2) + jj * 8;
    c0[k] = *reinterpret_cast<const f32x4_t*>(cr);
    c1[k] = *reinterpret_cast<const f32x4_t*>(cr + 4);
    s0[k] = *reinterpret_cast<const f32x4_t*>(sr);
    s1[k] = *reinterpret_cast<const f32x4_t*>(sr + 4);
  }
#pragma unroll
  for (int k = 0; k < NT; ++k) {
    float x[8];
    unpack8(raw[k], x);
    u32x4_t words = raw[k];
    if (w != nullptr) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += x[i] * x[i];
      ss = group_sum<LPR>(ss);
      const float scale = rsqrtf(ss * (1.0f / D) + eps);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        words[i] = pack_bf16x2((x[2 * i] * scale) * wf[2 * i], (x[2 * i + 1] * scale) * wf[2 * i + 1]);
      unpack8(words, x);
    }
    float p[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t wd = words[i];
      uint32_t pw;
      if constexpr (HALF == 8) pw = dpp_u32<0x128>(wd);
      else pw = static_cast<uint32_t>(__shfl_xor(static_cast<int>(wd), HALF, kWave));
      pw ^= psign;
      p[2 * i] = bf16_lo(pw);
      p[2 * i + 1] = bf16_hi(pw);
    }
    const float c[8] = {c0[k][0], c0[k][1], c0[k][2], c0[k][3], c1[k][0], c1[k][1], c1[k][2], c1[k][3]};
    const float sn[8] = {s0[k][0], s0[k][1], s0[k][2], s0[k][3], s1[k][0], s1[k][1], s1[k][2], s1[k][3]};
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = rope_one(x[i], p[i], c[i], sn[i]);
    const u32x4_t packed = pack8(x);
    if (tb * NT + k < num_tokens) {
      if (is_q || k_back) stg128_nt<kFusedNtStore>(rowb[k] + lane_off, packed);
      if (!is_q) stg128_nt<kFusedNtStore>(k_cache + slot[k] * hkv * D + (static_cast<uint32_t>((r - hq) * D) + head_off), packed);
    }
  }
}

inline int64_t blocks_for(int64_t jobs, int rows_per_block) {
  return (jobs + rows_per_block - 1) / rows_per_block;
}

}  // namespace
}  // namespace sgl

using namespace sgl;

extern "C" int sgl_rope_cos_sin_cache(float* cos_cache, float* sin_cache, int64_t max_pos,
                                      int rotary_dim, float base, void* stream) {
  if (!cos_cache || !sin_cache || max_pos <= 0 || rotary_dim <= 0 || (rotary_dim & 1))
    return SGL_ERR_INVALID_ARG;
  const int half = rotary_dim / 2;
  if (half > kMaxHalfRotary) return SGL_ERR_UNSUPPORTED;
  InvFreq inv;
  for (int k = 0; k < half; ++k) {
    const float expo = static_cast<float>(2 * k) / static_cast<float>(rotary_dim);
    inv.v[k] = 1.0f / powf(base, expo);
  }
  const int64_t n = max_pos * half;
  hipLaunchKernelGGL(cos_sin_cache_kernel, dim3((n + 255) / 256), dim3(256), 0,
                     static_cast<hipStream_t>(stream), cos_cache, sin_cache, max_pos, half, inv);
  return launch_status();
}

extern "C" int sgl_qk_rmsnorm(void* q, void* k, const void* q_weight, const void* k_weight,
                              int64_t tokens, int64_t q_heads, int64_t k_heads, int64_t d,
                              int64_t q_st, int64_t q_sh, int64_t k_st, int64_t k_sh, float eps,
                              int dtype, void* stream) {
  if (tokens < 0 || q_heads < 0 || k_heads < 0 || d <= 0) return SGL_ERR_INVALID_ARG;
  if (dtype != SGL_DTYPE_BF16 && dtype != SGL_DTYPE_F16) return SGL_ERR_UNSUPPORTED;
  if (k == nullptr) k_heads = 0;
  const int64_t total = tokens * (q_heads + k_heads);
  if (total == 0) return SGL_OK;
  if ((q_heads > 0 && (!q || !q_weight)) || (k_heads > 0 && !k_weight))
    return SGL_ERR_INVALID_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto* qp = static_cast<uint16_t*>(q);
  auto* kp = static_cast<uint16_t*>(k);
  auto* qw = static_cast<const uint16_t*>(q_weight);
  auto* kw = static_cast<const uint16_t*>(k_weight);
  const bool vec_ok = (q_st % 8 == 0) && (q_sh % 8 == 0) && (k_st % 8 == 0) && (k_sh % 8 == 0) &&
                      aligned16(q) && (k == nullptr || aligned16(k)) &&
                      (qw == nullptr || aligned16(qw)) && (kw == nullptr || aligned16(kw));
  const float inv_d = 1.0f / static_cast<float>(d);
#define SGL_NORM_CASE(LPR_)                                                                  \
  if (dtype == SGL_DTYPE_BF16)                                                               \
    hipLaunchKernelGGL((qk_rmsnorm_kernel<LPR_, SGL_DTYPE_BF16>),                            \
                       dim3(blocks_for(total, 256 / LPR_)), dim3(256), 0, s, qp, kp, qw, kw, \
                       tokens, q_heads, k_heads, q_st, q_sh, k_st, k_sh, inv_d, eps);        \
  else                                                                                       \
    hipLaunchKernelGGL((qk_rmsnorm_kernel<LPR_, SGL_DTYPE_F16>),                             \
                       dim3(blocks_for(total, 256 / LPR_)), dim3(256), 0, s, qp, kp, qw, kw, \
                       tokens, q_heads, k_heads, q_st, q_sh, k_st, k_sh, inv_d, eps);        \
  return launch_status();
  if (vec_ok) {
    switch (d) {
      case 64: SGL_NORM_CASE(8)
      case 128: SGL_NORM_CASE(16)
      case 256: SGL_NORM_CASE(32)
      case 512: SGL_NORM_CASE(64)
      default: break;
    }
  }
#undef SGL_NORM_CASE
  if (dtype == SGL_DTYPE_BF16)
    hipLaunchKernelGGL(qk_rmsnorm_generic_kernel<SGL_DTYPE_BF16>, dim3(blocks_for(total, 4)),
                       dim3(256), 0, s, qp, kp, qw, kw, tokens, q_heads, k_heads, d, q_st, q_sh,
                       k_st, k_sh, eps);
  else
    hipLaunchKernelGGL(qk_rmsnorm_generic_kernel<SGL_DTYPE_F16>, dim3(blocks_for(total, 4)),
                       dim3(256), 0, s, qp, kp, qw, kw, tokens, q_heads, k_heads, d, q_st, q_sh,
                       k_st, k_sh, eps);
  return launch_status();
}

extern "C" int sgl_rope(void* q, void* k, const float* cos_cache, const float* sin_cache,
                        const int32_t* positions, int64_t nnz, int64_t q_heads, int64_t kv_heads,
                        int64_t rotary_dim, int64_t head_dim, int64_t cos_width, int64_t q_st,
                        int64_t q_sh, int64_t k_st, int64_t k_sh, int dtype, void* stream) {
  if (nnz < 0 || q_heads < 0 || kv_heads < 0 || head_dim <= 0) return SGL_ERR_INVALID_ARG;
  if (dtype != SGL_DTYPE_BF16 && dtype != SGL_DTYPE_F16) return SGL_ERR_UNSUPPORTED;
  if (rotary_dim <= 0 || (rotary_dim & 1) || rotary_dim > head_dim) return SGL_ERR_INVALID_ARG;
  if (cos_width != rotary_dim && cos_width != rotary_dim / 2) return SGL_ERR_INVALID_ARG;
  const int64_t total = nnz * (q_heads + kv_heads);
  if (total == 0) return SGL_OK;
  if (!cos_cache || !sin_cache || !positions || (q_heads && !q) || (kv_heads && !k))
    return SGL_ERR_INVALID_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto* qp = static_cast<uint16_t*>(q);
  auto* kp = static_cast<uint16_t*>(k);
  const bool vec_ok = rotary_dim == head_dim && cos_width == head_dim / 2 && (q_st % 8 == 0) &&
                      (q_sh % 8 == 0) && (k_st % 8 == 0) && (k_sh % 8 == 0) &&
                      (q == nullptr || aligned16(q)) && (k == nullptr || aligned16(k)) &&
                      aligned16(cos_cache) && aligned16(sin_cache);
#define SGL_ROPE_CASE(LPR_)                                                                   \
  if (dtype == SGL_DTYPE_BF16)                                                                \
    hipLaunchKernelGGL((rope_kernel<LPR_, SGL_DTYPE_BF16>), dim3(blocks_for(total, 256 / LPR_)), \
                       dim3(256), 0, s, qp, kp, cos_cache, sin_cache, positions, nnz, q_heads, \
                       kv_heads, q_st, q_sh, k_st, k_sh);                                     \
  else                                                                                        \
    hipLaunchKernelGGL((rope_kernel<LPR_, SGL_DTYPE_F16>), dim3(blocks_for(total, 256 / LPR_)), \
                       dim3(256), 0, s, qp, kp, cos_cache, sin_cache, positions, nnz, q_heads, \
                       kv_heads, q_st, q_sh, k_st, k_sh);                                     \
  return launch_status();
  if (vec_ok) {
    switch (head_dim) {
      case 64: SGL_ROPE_CASE(8)
      case 128: SGL_ROPE_CASE(16)
      case 256: SGL_ROPE_CASE(32)
      case 512: SGL_ROPE_CASE(64)
      default: break;
    }
  }
#undef SGL_ROPE_CASE
  if (rotary_dim > 128 * 8) return SGL_ERR_UNSUPPORTED;
  if (dtype == SGL_DTYPE_BF16)
    hipLaunchKernelGGL(rope_generic_kernel<SGL_DTYPE_BF16>, dim3(total), dim3(128), 0, s, qp, kp,
                       cos_cache, sin_cache, positions, nnz, q_heads, kv_heads, rotary_dim,
                       head_dim, cos_width, q_st, q_sh, k_st, k_sh);
  else
    hipLaunchKernelGGL(rope_generic_kernel<SGL_DTYPE_F16>, dim3(total), dim3(128), 0, s, qp, kp,
                       cos_cache, sin_cache, positions, nnz, q_heads, kv_heads, rotary_dim,
                       head_dim, cos_width, q_st, q_sh, k_st, k_sh);
  return launch_status();
}

extern "C" int sgl_fused_qknorm_rope_store(void* qkv, int64_t qkv_stride_token, void* k_cache,
                                           void* v_cache, const void* q_weight,
                                           const void* k_weight, const float* cos_cache,
                                           const float* sin_cache, const int32_t* positions,
                                           const int32_t* out_loc, int64_t num_tokens,
                                           int num_qo_heads, int num_kv_heads, int head_dim,
                                           float eps, int flags, void* stream) {
  if (num_tokens < 0 || num_qo_heads <= 0 || num_kv_heads <= 0) return SGL_ERR_INVALID_ARG;
  if (flags & ~SGL_FUSED_NO_K_WRITEBACK) return SGL_ERR_INVALID_ARG;
  if (num_tokens == 0) return SGL_OK;
  if (!qkv || !k_cache || !v_cache || !cos_cache || !sin_cache || !positions || !out_loc)
    return SGL_ERR_INVALID_ARG;
  if ((q_weight == nullptr) != (k_weight == nullptr)) return SGL_ERR_INVALID_ARG;
  const int64_t rows = static_cast<int64_t>(num_qo_heads + 2 * num_kv_heads);
  if (qkv_stride_token < rows * head_dim) return SGL_ERR_INVALID_ARG;
  if (qkv_stride_token % 8 != 0 || !aligned16(qkv) || !aligned16(k_cache) ||
      !aligned16(v_cache) || !aligned16(cos_cache) || !aligned16(sin_cache) ||
      (q_weight && (!aligned16(q_weight) || !aligned16(k_weight))))
    return SGL_ERR_ALIGNMENT;
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto* base = static_cast<uint16_t*>(qkv);
  auto* kc = static_cast<uint16_t*>(k_cache);
  auto* vc = static_cast<uint16_t*>(v_cache);
  auto* qw = static_cast<const uint16_t*>(q_weight);
  auto* kw = static_cast<const uint16_t*>(k_weight);
#define SGL_FUSED_CASE(LPR_)                                                                   \
  {                                                                                            \
    const int64_t bpt = blocks_for(rows, 256 / LPR_);                                          \
    if (num_tokens * bpt > 0x7fffffff) return SGL_ERR_UNSUPPORTED;                             \
    hipLaunchKernelGGL(fused_qknorm_rope_store_kernel<LPR_>, dim3((num_tokens + kFusedTokensPerBlock - 1) / kFusedTokensPerBlock * bpt), \
                       dim3(256), \
                       0, s, base, qkv_stride_token, kc, vc, qw, kw, cos_cache, sin_cache,      \
                       positions, out_loc, num_qo_heads, num_kv_heads, static_cast<int>(bpt),   \
                       eps, (flags & SGL_FUSED_NO_K_WRITEBACK) == 0, num_tokens);               \
    return launch_status();                                                                    \
  }
  switch (head_dim) {
    case 64: SGL_FUSED_CASE(8)
    case 128: SGL_FUSED_CASE(16)
    case 256: SGL_FUSED_CASE(32)
    case 512: SGL_FUSED_CASE(64)
    default: break;
  }
#undef SGL_FUSED_CASE
  return SGL_ERR_UNSUPPORTED;
}
