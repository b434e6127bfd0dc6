// Split-KV paged decode on gfx950 matrix cores.
//
// Reference semantics: FlashInferBackend::forward, decode branch
// (src/attention/flashinfer_backend.cu:553-595): for request r and q head h,
//   o[r, h] = softmax_j(q[r, h] . K[indices[kv_indptr[r] + j], h / G] * sm_scale)
//             . V[indices[kv_indptr[r] + j], h / G]
// with the page table token-granular (page_size 1), no window, no soft-cap.
//
// Work decomposition: one workgroup per (request, KV chunk) with one wave
// per kv head, so a workgroup reads whole [Hkv, D] slot rows (the pool
// layout) instead of one head segment per row. All G query heads of a kv head
// ride in one 16-wide MFMA operand, so every K/V byte is read from HBM exactly
// once per step. Each wave walks the chunk's 32-token tiles with a two-stage
// software pipeline: while tile t is on the matrix cores, the K/V rows of
// tile t+1 and the slot indices of tile t+2 are already in flight, so a wave
// always has 16 KiB of HBM reads outstanding.
// A request longer than one chunk writes fp32 partials plus a log2-sum-exp,
// combined by a second, short kernel. (Merging inside the decode launch
// would need an agent-scope release per workgroup, which on a multi-XCD part
// is an L2 write-back per workgroup; the kernel boundary is far cheaper.)
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
constexpr int kMaxWaves = 8;  // kv heads per workgroup (one wave each)
constexpr int kMaxGroup = 16;
constexpr int kMaxChunks = 128;  // bound on splits per request (LDS merge table)

struct DecodeArgs {
  const uint16_t* q;
  int64_t q_st, q_sh;
  const uint16_t* kc;
  const uint16_t* vc;
  int64_t kv_ss, kv_sh;
  const int32_t* indices;
  const int32_t* kv_indptr;
  const int32_t* q_indptr;
  int hq, hkv, group;
  float scale_log2;  // sm_scale * log2(e)
  uint16_t* o;
  int64_t o_st, o_sh;
  float* part_o;     // [B, max_chunks, hq, D]
  float* part_lse;   // [B, max_chunks, hq]
  int chunk, max_chunks;
};

// Workspace carve-up shared by the plan, the init call and the launch.
struct WorkspaceLayout {
  int64_t part_o_off, part_lse_off, total;
};

inline WorkspaceLayout workspace_layout(int batch, int max_chunks, int hq) {
  WorkspaceLayout w;
  const int64_t npart = static_cast<int64_t>(batch) * max_chunks * hq;
  auto align = [](int64_t x) { return (x + 255) / 256 * 256; };
  w.part_o_off = 0;
  w.part_lse_off = align(npart * kD * 4);
  w.total = w.part_lse_off + align(npart * 4);
  return w;
}

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

// Issue the 16 row loads of one 32-token tile. `slot_lane` holds, in lane
// l, the slot of token (l % 32) of the tile (clamped to the last valid one).
__device__ __forceinline__ void issue_tile_loads(const uint16_t* kbase, const uint16_t* vbase,
                                                 int64_t kv_ss, int slot_lane, int n, int j,
                                                 u32x4_t (&kr)[8], u32x4_t (&vr)[8]) {
  const int64_t sk0 = __shfl(slot_lane, n, kWave);
  const int64_t sk1 = __shfl(slot_lane, 16 + n, kWave);
  const uint16_t* k0 = kbase + sk0 * kv_ss + 8 * j;
  const uint16_t* k1 = kbase + sk1 * kv_ss + 8 * j;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    kr[s] = ldg128(k0 + 32 * s);
    kr[4 + s] = ldg128(k1 + 32 * s);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int64_t sv = __shfl(slot_lane, 16 * (e >> 2) + 4 * j + (e & 3), kWave);
    vr[e] = ldg128(vbase + sv * kv_ss + 8 * n);
  }
}

// Slot of token (lane % 32) of the tile starting at tb, clamped into
// [0, t1): tiles past the end re-read the last valid row (an L2 hit), which
// keeps every load in the pipelined loop unconditional.
__device__ __forceinline__ int load_slot(const int32_t* idx, int tb, int t1, int lane) {
  return idx[min(tb + (lane & 31), t1 - 1)];
}

struct HeadState {
  float m, l;
  f32x4_t acc[8];
};

// Online-softmax update of one 32-token tile starting at tb (rows in kr/vr).
__device__ __forceinline__ void consume_tile(const DecodeArgs& a, const bf16x8_t (&qop)[4],
                                             const u32x4_t (&kr)[8], const u32x4_t (&vr)[8],
                                             int tb, int t1, int j, HeadState& st) {
  const int last = t1 - tb - 1;  // last valid token offset in this tile
  f32x4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kr[s]), qop[s], s0, 0, 0, 0);
    s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kr[4 + s]), qop[s], s1, 0, 0, 0);
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
  const float mn = fmaxf(st.m, mt);
  const float alpha = exp2f(st.m - mn);
  float p[8];
  float ps = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    p[e] = exp2f(sc[e] - mn);
    ps += p[e];
  }
  st.l = st.l * alpha + ps;
  st.m = mn;
  u32x4_t pw;
#pragma unroll
  for (int k = 0; k < 4; ++k) pw[k] = pack_bf16x2(p[2 * k], p[2 * k + 1]);
  const bf16x8_t pop = as_bf16x8(pw);
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) st.acc[nb] *= alpha;
  st.acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v_operand<0>(vr), pop, st.acc[0], 0, 0, 0);
  st.acc[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v_operand<1>(vr), pop, st.acc[1], 0, 0, 0);
  st.acc[2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v_operand<2>(vr), pop, st.acc[2], 0, 0, 0);
  st.acc[3] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v_operand<3>(vr), pop, st.acc[3], 0, 0, 0);
  st.acc[4] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v_operand<4>(vr), pop, st.acc[4], 0, 0, 0);
  st.acc[5] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v_operand<5>(vr), pop, st.acc[5], 0, 0, 0);
  st.acc[6] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v_operand<6>(vr), pop, st.acc[6], 0, 0, 0);
  st.acc[7] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v_operand<7>(vr), pop, st.acc[7], 0, 0, 0);
}

// One wave: kv head h of request r over tokens [t0, t1) of chunk c (t0 < t1).
//
// Pipeline (all loads unconditional, so the compiler's in-order vmcnt waits
// stay partial): entering the step for tile t, the rows of t are in flight
// and the slots of t+1 have landed. The step issues the slot load of t+2,
// then the 16 row loads of t+1, then waits only for tile t's rows and
// consumes them. Two register sets ping-pong between "current" and "next".
__device__ __forceinline__ void decode_head(const DecodeArgs& a, int r, int c, int nch, int h,
                                            int t0, int t1, int qrow, int lane) {
  const int n = lane & 15;
  const int j = lane >> 4;
  const bool head_ok = n < a.group;
  const int head = h * a.group + n;
  const uint16_t* kbase = a.kc + static_cast<int64_t>(h) * a.kv_sh;
  const uint16_t* vbase = a.vc + static_cast<int64_t>(h) * a.kv_sh;
  const int32_t* idx = a.indices + a.kv_indptr[r];

  u32x4_t ka[8], va[8], kb[8], vb[8];
  int slot_a = load_slot(idx, t0, t1, lane);
  int slot_b = load_slot(idx, t0 + kTile, t1, lane);
  issue_tile_loads(kbase, vbase, a.kv_ss, slot_a, n, j, ka, va);

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

  HeadState st;
  st.m = -INFINITY;
  st.l = 0.f;
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) st.acc[nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  int tb = t0;
  while (true) {
    // tile tb in (ka, va); slots of tb + 32 in slot_b
    slot_a = load_slot(idx, tb + 2 * kTile, t1, lane);
    issue_tile_loads(kbase, vbase, a.kv_ss, slot_b, n, j, kb, vb);
    __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the consume
    consume_tile(a, qop, ka, va, tb, t1, j, st);
    __builtin_amdgcn_sched_barrier(0);
    tb += kTile;
    if (tb >= t1) break;
    // tile tb in (kb, vb); slots of tb + 32 in slot_a
    slot_b = load_slot(idx, tb + 2 * kTile, t1, lane);
    issue_tile_loads(kbase, vbase, a.kv_ss, slot_a, n, j, ka, va);
    __builtin_amdgcn_sched_barrier(0);
    consume_tile(a, qop, kb, vb, tb, t1, j, st);
    __builtin_amdgcn_sched_barrier(0);
    tb += kTile;
    if (tb >= t1) break;
  }
  float m = st.m;
  float l = st.l;
  l += __shfl_xor(l, 16, kWave);
  l += __shfl_xor(l, 32, kWave);
  if (!head_ok) return;
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  f32x4_t (&acc)[8] = st.acc;
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
    if (j == 0) a.part_lse[pidx] = l > 0.f ? m + log2f(l) : -INFINITY;
  }
}

// One workgroup per (KV chunk, request); its waves take the kv heads, so the
// workgroup streams whole [Hkv, D] slot rows (2 KiB at 8 kv heads) rather
// than one 256-byte head segment of each row.
__global__ void __launch_bounds__(kMaxWaves * kWave) paged_decode_kernel(DecodeArgs a) {
  const int c = blockIdx.x;
  const int r = blockIdx.y;
  const int kv_len = a.kv_indptr[r + 1] - a.kv_indptr[r];
  const int nch = kv_len > a.chunk ? (kv_len + a.chunk - 1) / a.chunk : 1;
  if (c >= nch) return;
  const int t0 = c * a.chunk;
  const int t1 = min(kv_len, t0 + a.chunk);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  const int qrow = a.q_indptr ? a.q_indptr[r] : r;
  if (t1 <= t0) {  // empty request: the output row is zero
    for (int e = threadIdx.x; e < a.hq * (kD / 8); e += blockDim.x) {
      const int hh = e / (kD / 8);
      stg128(a.o + static_cast<int64_t>(qrow) * a.o_st + static_cast<int64_t>(hh) * a.o_sh +
                 (e - hh * (kD / 8)) * 8,
             u32x4_t{0, 0, 0, 0});
    }
    return;
  }
  for (int h = wave; h < a.hkv; h += nwaves) decode_head(a, r, c, nch, h, t0, t1, qrow, lane);
}

// Combines the chunk partials of every split request: one workgroup per
// (request, kv head) handles its G heads. The chunk lse values are fetched
// in parallel into LDS and turned into weights; then each thread owns 4
// consecutive d of one head and streams the chunk partials (16-byte loads,
// several in flight).
__global__ void __launch_bounds__(256) decode_merge_kernel(DecodeArgs a) {
  const int h = blockIdx.x;
  const int r = blockIdx.y;
  const int kv_len = a.kv_indptr[r + 1] - a.kv_indptr[r];
  const int nch = kv_len > a.chunk ? (kv_len + a.chunk - 1) / a.chunk : 1;
  if (nch <= 1) return;
  __shared__ float sh_w[kMaxChunks][kMaxGroup];
  const int G = a.group;
  const int qrow = a.q_indptr ? a.q_indptr[r] : r;
  const int64_t base = static_cast<int64_t>(r) * a.max_chunks * a.hq + h * G;
  for (int e = threadIdx.x; e < nch * G; e += blockDim.x) {
    const int cc = e / G;
    const int g = e - cc * G;
    sh_w[cc][g] = a.part_lse[base + cc * a.hq + g];
  }
  __syncthreads();
  if (threadIdx.x < G) {
    const int g = threadIdx.x;
    float mx = -INFINITY;
    for (int cc = 0; cc < nch; ++cc) mx = fmaxf(mx, sh_w[cc][g]);
    float den = 0.f;
    for (int cc = 0; cc < nch; ++cc) {
      const float lse = sh_w[cc][g];
      const float w = lse == -INFINITY ? 0.f : exp2f(lse - mx);
      sh_w[cc][g] = w;
      den += w;
    }
    const float inv = den > 0.f ? 1.0f / den : 0.f;
    for (int cc = 0; cc < nch; ++cc) sh_w[cc][g] *= inv;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < G * (kD / 4); e += blockDim.x) {
    const int g = e / (kD / 4);
    const int d4 = (e - g * (kD / 4)) * 4;
    f32x4_t accm = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
    for (int cc = 0; cc < nch; ++cc) {
      const f32x4_t v =
          *reinterpret_cast<const f32x4_t*>(a.part_o + (base + cc * a.hq + g) * kD + d4);
      accm += v * sh_w[cc][g];
    }
    uint16_t* op = a.o + static_cast<int64_t>(qrow) * a.o_st +
                   static_cast<int64_t>(h * G + g) * a.o_sh + d4;
    u32x2_t packed = {pack_bf16x2(accm[0], accm[1]), pack_bf16x2(accm[2], accm[3])};
    *reinterpret_cast<u32x2_t*>(op) = packed;
  }
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
  // Aim for ~32 (request, kv head, chunk) waves per CU on a 256-CU part;
  // chunks are whole 32-token tiles, and no request splits into more than
  // kMaxChunks pieces.
  constexpr int64_t kTargetWaves = 8192;
  constexpr int kQuantum = kTile;
  int64_t chunk = (total * num_kv_heads + kTargetWaves - 1) / kTargetWaves;
  const int64_t min_chunk = (static_cast<int64_t>(max_len) + kMaxChunks - 1) / kMaxChunks;
  if (chunk < min_chunk) chunk = min_chunk;
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
  plan->num_kv_heads = num_kv_heads;
  plan->head_dim = head_dim;
  plan->workspace_bytes =
      plan->split_kv ? workspace_layout(batch_size, max_chunks, num_qo_heads).total : 0;
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
  if (plan->kv_chunk_size <= 0 || plan->kv_chunk_size % kTile != 0 || plan->max_chunks <= 0 ||
      plan->max_chunks > kMaxChunks)
    return SGL_ERR_INVALID_ARG;
  if (batch_size > plan->batch_size || num_qo_heads != plan->num_qo_heads ||
      num_kv_heads != plan->num_kv_heads)
    return SGL_ERR_CAPACITY;
  if (plan->split_kv && (workspace == nullptr || workspace_bytes < plan->workspace_bytes))
    return SGL_ERR_CAPACITY;
  if (q_stride_head % 8 || q_stride_token % 8 || kv_stride_slot % 8 || kv_stride_head % 8 ||
      o_stride_token % 8 || o_stride_head % 4 || !aligned16(q) || !aligned16(k_cache) ||
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
  a.hkv = num_kv_heads;
  a.group = group;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.o = static_cast<uint16_t*>(o);
  a.o_st = o_stride_token;
  a.o_sh = o_stride_head;
  a.chunk = plan->kv_chunk_size;
  a.max_chunks = plan->max_chunks;
  if (plan->split_kv) {
    const WorkspaceLayout w = workspace_layout(plan->batch_size, plan->max_chunks, num_qo_heads);
    char* base = static_cast<char*>(workspace);
    a.part_o = reinterpret_cast<float*>(base + w.part_o_off);
    a.part_lse = reinterpret_cast<float*>(base + w.part_lse_off);
  } else {
    a.part_o = nullptr;
    a.part_lse = nullptr;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int waves = num_kv_heads < kMaxWaves ? num_kv_heads : kMaxWaves;
  hipLaunchKernelGGL(paged_decode_kernel, dim3(plan->max_chunks, batch_size), dim3(waves * kWave),
                     0, s, a);
  int st = launch_status();
  if (st != SGL_OK || !plan->split_kv) return st;
  hipLaunchKernelGGL(decode_merge_kernel, dim3(num_kv_heads, batch_size), dim3(256), 0, s, a);
  return launch_status();
}
