// Split-KV paged decode on gfx950 matrix cores.
//
// Reference semantics: FlashInferBackend::forward, decode branch
// (src/attention/flashinfer_backend.cu:553-595): for request r and q head h,
//   o[r, h] = softmax_j(q[r, h] . K[indices[kv_indptr[r] + j], h / G] * sm_scale)
//             . V[indices[kv_indptr[r] + j], h / G]
// with the page table token-granular (page_size 1), no window, no soft-cap.
//
// Work decomposition: one workgroup (4 waves) per (request, kv head, KV
// chunk). All G query heads of the kv head ride in one 16-wide MFMA operand,
// so every K/V byte is read from HBM exactly once per step. Each wave walks
// 32-token tiles of the chunk (tile w, w+4, ...), keeps an online softmax,
// and the 4 wave states are merged through LDS. A request longer than one
// chunk writes fp32 partials plus a log2-sum-exp, merged by a second kernel.
//
// Matrix formulation (v_mfma_f32_16x16x32_bf16, lane l, n = l % 16, j = l / 16):
//   S^T[tok, head] = K[tok, :] . Q[head, :]   A = K rows, B = Q^T
//   O^T[d, head]  += V^T[d, tok] . P^T[tok, head]
// Both products put the query head on the lane's column n, so the softmax
// max/sum and the rescale of O are lane-local apart from one 4-way exchange.
// The k index of each product is a summation index: A and B only have to
// agree on which token (or d) sits in each lane's k slots, so the V operand
// uses the d-order d = 8 * m + nb (m = MFMA row, nb = which of 8 MFMAs). With
// that order a lane needs V[tok][8n .. 8n+7] for its 8 tokens — one 16-byte
// load per token, 16 lanes covering a whole 256-byte row — and an in-register
// 8x8 transpose of bf16 halves (v_perm) builds the operands.
#include <math.h>

#include "common.h"

namespace sgl {
namespace {

constexpr int kD = 128;
constexpr int kTile = 32;
constexpr int kWaves = 4;
constexpr int kMaxGroup = 16;

struct DecodeArgs {
  const uint16_t* q;
  int64_t q_st, q_sh;
  const uint16_t* kc;
  const uint16_t* vc;
  int64_t kv_ss, kv_sh;
  const int32_t* indices;
  const int32_t* kv_indptr;
  const int32_t* q_indptr;
  int hq, group;
  float scale_log2;  // sm_scale * log2(e)
  uint16_t* o;
  int64_t o_st, o_sh;
  float* part_o;    // [B, max_chunks, hq, D]
  float* part_lse;  // [B, max_chunks, hq]
  int chunk, max_chunks;
};

__device__ __forceinline__ bf16x8_t as_bf16x8(const u32x4_t& v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

// Operand for MFMA nb of O^T: slot e takes bf16 element nb of row vr[e].
template <int nb>
__device__ __forceinline__ bf16x8_t v_operand(const u32x4_t (&vr)[8]) {
  constexpr int w = nb / 2;
  constexpr uint32_t sel = (nb & 1) ? 0x07060302u : 0x05040100u;
  u32x4_t out;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    out[k] = __builtin_amdgcn_perm(vr[2 * k + 1][w], vr[2 * k][w], sel);
  }
  return as_bf16x8(out);
}

__global__ void __launch_bounds__(256) paged_decode_kernel(DecodeArgs a) {
  const int c = blockIdx.x;
  const int h = blockIdx.y;
  const int r = blockIdx.z;
  const int kv_beg = a.kv_indptr[r];
  const int kv_len = a.kv_indptr[r + 1] - kv_beg;
  const int nch = kv_len > a.chunk ? (kv_len + a.chunk - 1) / a.chunk : 1;
  if (c >= nch) return;
  const int t0 = c * a.chunk;
  const int t1 = min(kv_len, t0 + a.chunk);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n = lane & 15;
  const int j = lane >> 4;
  const int qrow = a.q_indptr ? a.q_indptr[r] : r;
  const bool head_ok = n < a.group;
  const int head = h * a.group + n;

  // Q^T operand: lane holds q[head][32 s + 8 j .. + 8] for s = 0..3.
  bf16x8_t qop[4];
  {
    const uint16_t* qp = a.q + static_cast<int64_t>(qrow) * a.q_st +
                         static_cast<int64_t>(head_ok ? head : 0) * a.q_sh + 8 * j;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u32x4_t v = head_ok ? ldg128(qp + 32 * s) : u32x4_t{0, 0, 0, 0};
      qop[s] = as_bf16x8(v);
    }
  }

  const uint16_t* kbase = a.kc + static_cast<int64_t>(h) * a.kv_sh;
  const uint16_t* vbase = a.vc + static_cast<int64_t>(h) * a.kv_sh;
  const int32_t* idx = a.indices + kv_beg;

  float m = -INFINITY;
  float l = 0.f;
  f32x4_t acc[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) acc[nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int tb = t0 + wave * kTile; tb < t1; tb += kWaves * kTile) {
    const int last = t1 - tb - 1;  // last valid token offset in this tile
    // K rows: tokens n and 16 + n; V rows: tokens 16 b + 4 j + i (slot e = 4 b + i).
    const int64_t sk0 = idx[tb + min(n, last)];
    const int64_t sk1 = idx[tb + min(16 + n, last)];
    int64_t sv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) sv[e] = idx[tb + min(16 * (e >> 2) + 4 * j + (e & 3), last)];

    u32x4_t kr0[4], kr1[4], vr[8];
    const uint16_t* k0 = kbase + sk0 * a.kv_ss + 8 * j;
    const uint16_t* k1 = kbase + sk1 * a.kv_ss + 8 * j;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      kr0[s] = ldg128(k0 + 32 * s);
      kr1[s] = ldg128(k1 + 32 * s);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) vr[e] = ldg128(vbase + sv[e] * a.kv_ss + 8 * n);

    f32x4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kr0[s]), qop[s], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kr1[s]), qop[s], s1, 0, 0, 0);
    }

    // Lane holds scores of tokens 16 b + 4 j + i for head n.
    float sc[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tok0 = 4 * j + i;
      sc[i] = tok0 <= last ? s0[i] * a.scale_log2 : -INFINITY;
      sc[4 + i] = tok0 + 16 <= last ? s1[i] * a.scale_log2 : -INFINITY;
    }
    float mt = sc[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) mt = fmaxf(mt, sc[e]);
    mt = fmaxf(mt, __shfl_xor(mt, 16, kWave));
    mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));
    const float mn = fmaxf(m, mt);
    const float alpha = exp2f(m - mn);
    float p[8];
    float ps = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      p[e] = exp2f(sc[e] - mn);
      ps += p[e];
    }
    l = l * alpha + ps;
    m = mn;
    u32x4_t pw;
#pragma unroll
    for (int k = 0; k < 4; ++k) pw[k] = pack_bf16x2(p[2 * k], p[2 * k + 1]);
    const bf16x8_t pop = as_bf16x8(pw);
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) acc[nb] *= alpha;
    acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v_operand<0>(vr), pop, acc[0], 0, 0, 0);
    acc[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v_operand<1>(vr), pop, acc[1], 0, 0, 0);
    acc[2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v_operand<2>(vr), pop, acc[2], 0, 0, 0);
    acc[3] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v_operand<3>(vr), pop, acc[3], 0, 0, 0);
    acc[4] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v_operand<4>(vr), pop, acc[4], 0, 0, 0);
    acc[5] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v_operand<5>(vr), pop, acc[5], 0, 0, 0);
    acc[6] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v_operand<6>(vr), pop, acc[6], 0, 0, 0);
    acc[7] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v_operand<7>(vr), pop, acc[7], 0, 0, 0);
  }
  l += __shfl_xor(l, 16, kWave);
  l += __shfl_xor(l, 32, kWave);

  // Merge the 4 wave states: waves 1..3 park theirs in LDS, wave 0 combines.
  __shared__ float sh_o[kWaves - 1][32][kWave];
  __shared__ float sh_m[kWaves][16];
  __shared__ float sh_l[kWaves][16];
  if (j == 0) {
    sh_m[wave][n] = m;
    sh_l[wave][n] = l;
  }
  if (wave > 0) {
#pragma unroll
    for (int nb = 0; nb < 8; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) sh_o[wave - 1][nb * 4 + i][lane] = acc[nb][i];
  }
  __syncthreads();
  if (wave != 0) return;
  float mw[kWaves];
  float mx = -INFINITY;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    mw[w] = sh_m[w][n];
    mx = fmaxf(mx, mw[w]);
  }
  float f[kWaves];
  float lt = 0.f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    f[w] = (mw[w] == -INFINITY) ? 0.f : exp2f(mw[w] - mx);
    lt += sh_l[w][n] * f[w];
  }
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = acc[nb][i] * f[0];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) v += sh_o[w - 1][nb * 4 + i][lane] * f[w];
      acc[nb][i] = v;
    }
  }
  if (!head_ok) return;
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  // Lane holds d = 32 j + 8 i + nb for head n.
  if (nch == 1) {
    uint16_t* op = a.o + static_cast<int64_t>(qrow) * a.o_st + static_cast<int64_t>(head) * a.o_sh;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v[8];
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) v[nb] = acc[nb][i] * inv;
      stg128(op + 32 * j + 8 * i, pack8(v));
    }
  } else {
    const int64_t pidx = (static_cast<int64_t>(r) * a.max_chunks + c) * a.hq + head;
    float* pp = a.part_o + pidx * kD;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4_t v0, v1;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        v0[nb] = acc[nb][i] * inv;
        v1[nb] = acc[nb + 4][i] * inv;
      }
      *reinterpret_cast<f32x4_t*>(pp + 32 * j + 8 * i) = v0;
      *reinterpret_cast<f32x4_t*>(pp + 32 * j + 8 * i + 4) = v1;
    }
    if (j == 0) a.part_lse[pidx] = lt > 0.f ? mx + log2f(lt) : -INFINITY;
  }
}

// Combines the chunk partials of every request that was split.
__global__ void __launch_bounds__(128) decode_merge_kernel(DecodeArgs a) {
  const int r = blockIdx.x;
  const int head = blockIdx.y;
  const int kv_len = a.kv_indptr[r + 1] - a.kv_indptr[r];
  const int nch = kv_len > a.chunk ? (kv_len + a.chunk - 1) / a.chunk : 1;
  if (nch <= 1) return;
  const int d = threadIdx.x;
  const int64_t base = static_cast<int64_t>(r) * a.max_chunks * a.hq + head;
  float mx = -INFINITY;
  for (int c = 0; c < nch; ++c) mx = fmaxf(mx, a.part_lse[base + static_cast<int64_t>(c) * a.hq]);
  float num = 0.f, den = 0.f;
  for (int c = 0; c < nch; ++c) {
    const int64_t pidx = base + static_cast<int64_t>(c) * a.hq;
    const float lse = a.part_lse[pidx];
    const float w = lse == -INFINITY ? 0.f : exp2f(lse - mx);
    num += w * a.part_o[pidx * kD + d];
    den += w;
  }
  const int qrow = a.q_indptr ? a.q_indptr[r] : r;
  const float v = den > 0.f ? num / den : 0.f;
  a.o[static_cast<int64_t>(qrow) * a.o_st + static_cast<int64_t>(head) * a.o_sh + d] =
      static_cast<uint16_t>(f32_to_bf16_bits(v));
}

}  // namespace
}  // namespace sgl

using namespace sgl;

extern "C" int sgl_decode_plan(const int32_t* kv_indptr_host, int batch_size, int num_qo_heads,
                               int num_kv_heads, int head_dim, sgl_decode_plan_t* plan) {
  if (!plan || !kv_indptr_host || batch_size < 0 || num_qo_heads <= 0 || num_kv_heads <= 0)
    return SGL_ERR_INVALID_ARG;
  if (num_qo_heads % num_kv_heads != 0) return SGL_ERR_INVALID_ARG;
  if (head_dim != kD || num_qo_heads / num_kv_heads > kMaxGroup) return SGL_ERR_UNSUPPORTED;
  int64_t total = 0;
  int max_len = 0;
  for (int r = 0; r < batch_size; ++r) {
    const int len = kv_indptr_host[r + 1] - kv_indptr_host[r];
    if (len < 0) return SGL_ERR_INVALID_ARG;
    total += len;
    max_len = len > max_len ? len : max_len;
  }
  // Aim for ~16 workgroups per CU on a 256-CU part; chunks are multiples of
  // 4 waves x 32 tokens so every wave of a full chunk gets whole tiles.
  constexpr int64_t kTargetBlocks = 4096;
  constexpr int kQuantum = kWaves * kTile;
  int64_t chunk = (total * num_kv_heads + kTargetBlocks - 1) / kTargetBlocks;
  chunk = (chunk + kQuantum - 1) / kQuantum * kQuantum;
  if (chunk < kQuantum) chunk = kQuantum;
  const int64_t cap = (static_cast<int64_t>(max_len) + kQuantum - 1) / kQuantum * kQuantum;
  if (cap > 0 && chunk > cap) chunk = cap;
  const int max_chunks = max_len > chunk ? static_cast<int>((max_len + chunk - 1) / chunk) : 1;
  plan->kv_chunk_size = static_cast<int32_t>(chunk);
  plan->max_chunks = max_chunks;
  plan->split_kv = max_chunks > 1 ? 1 : 0;
  plan->batch_size = batch_size;
  plan->num_qo_heads = num_qo_heads;
  plan->head_dim = head_dim;
  plan->workspace_bytes =
      plan->split_kv ? static_cast<int64_t>(batch_size) * max_chunks * num_qo_heads *
                           (head_dim + 1) * static_cast<int64_t>(sizeof(float))
                     : 0;
  return SGL_OK;
}

extern "C" int sgl_paged_decode(const sgl_decode_plan_t* plan, const void* q,
                                int64_t q_stride_token, int64_t q_stride_head,
                                const void* k_cache, const void* v_cache, int64_t kv_stride_slot,
                                int64_t kv_stride_head, const int32_t* indices,
                                const int32_t* kv_indptr, const int32_t* q_indptr,
                                int batch_size, int num_qo_heads, int num_kv_heads, int head_dim,
                                float sm_scale, void* o, int64_t o_stride_token,
                                int64_t o_stride_head, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  if (!plan || batch_size < 0 || num_qo_heads <= 0 || num_kv_heads <= 0)
    return SGL_ERR_INVALID_ARG;
  if (batch_size == 0) return SGL_OK;
  if (!q || !k_cache || !v_cache || !indices || !kv_indptr || !o) return SGL_ERR_INVALID_ARG;
  if (num_qo_heads % num_kv_heads != 0) return SGL_ERR_INVALID_ARG;
  const int group = num_qo_heads / num_kv_heads;
  if (head_dim != kD || group > kMaxGroup) return SGL_ERR_UNSUPPORTED;
  if (plan->kv_chunk_size <= 0 || plan->kv_chunk_size % kTile != 0 || plan->max_chunks <= 0)
    return SGL_ERR_INVALID_ARG;
  if (batch_size > plan->batch_size || num_qo_heads != plan->num_qo_heads)
    return SGL_ERR_CAPACITY;
  if (plan->split_kv && (workspace == nullptr || workspace_bytes < plan->workspace_bytes))
    return SGL_ERR_CAPACITY;
  if (q_stride_head % 8 || q_stride_token % 8 || kv_stride_slot % 8 || kv_stride_head % 8 ||
      o_stride_token % 8 || o_stride_head % 8 || !aligned16(q) || !aligned16(k_cache) ||
      !aligned16(v_cache) || !aligned16(o) || (workspace && !aligned16(workspace)))
    return SGL_ERR_ALIGNMENT;
  DecodeArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_st = q_stride_token;
  a.q_sh = q_stride_head;
  a.kc = static_cast<const uint16_t*>(k_cache);
  a.vc = static_cast<const uint16_t*>(v_cache);
  a.kv_ss = kv_stride_slot;
  a.kv_sh = kv_stride_head;
  a.indices = indices;
  a.kv_indptr = kv_indptr;
  a.q_indptr = q_indptr;
  a.hq = num_qo_heads;
  a.group = group;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.o = static_cast<uint16_t*>(o);
  a.o_st = o_stride_token;
  a.o_sh = o_stride_head;
  a.chunk = plan->kv_chunk_size;
  a.max_chunks = plan->max_chunks;
  const int64_t npart = static_cast<int64_t>(plan->batch_size) * plan->max_chunks * num_qo_heads;
  a.part_o = plan->split_kv ? static_cast<float*>(workspace) : nullptr;
  a.part_lse = plan->split_kv ? static_cast<float*>(workspace) + npart * kD : nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(paged_decode_kernel, dim3(plan->max_chunks, num_kv_heads, batch_size),
                     dim3(256), 0, s, a);
  int st = launch_status();
  if (st != SGL_OK || !plan->split_kv) return st;
  hipLaunchKernelGGL(decode_merge_kernel, dim3(batch_size, num_qo_heads), dim3(kD), 0, s, a);
  return launch_status();
}
