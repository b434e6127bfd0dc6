// Paged causal prefill (ragged, prefix-cache aware) on gfx950 matrix cores.
//
// Reference semantics: FlashInferBackend::forward, prefill branch
// (src/attention/flashinfer_backend.cu:596-679) with MaskMode::kCausal:
// query i of request r (qo_len q_r, kv_len k_r) attends kv token j iff
// j <= i + (k_r - q_r) (bottom-right alignment, so cached prefix tokens are
// visible to every new token), kv slots taken from the token-granular
// indices[kv_indptr[r] + j].
//
// Work decomposition: one workgroup (4 waves) per (request, kv head, tile of
// 128 packed query rows). The G query heads that share a kv head are packed
// row-wise (packed row p -> token p / G, head h G + p % G), so each K/V tile
// staged in LDS feeds G heads. K/V tiles of 64 tokens are gathered from the
// pool (one 16-byte chunk per lane, slots from the index list) into a
// double-buffered LDS ring; the global loads of tile t+1 are in flight
// while tile t is on the matrix cores.
//
// Matrix formulation (v_mfma_f32_32x32x16_bf16, lane l, c = l % 32, hl = l / 32):
//   S^T[tok, row] = K[tok, :] . Q[row, :]      (A = K from LDS, B = Q^T in VGPRs)
//   O^T[d, row]  += V^T[d, tok] . P^T[tok, row] (A = V^T via in-register transpose)
// The query row sits on the lane's column c in both products, so the online
// softmax (max, sum, rescale of O) is lane-local apart from one exchange with
// lane l ^ 32. The V operand uses the d-order d = 4 m + db (m = MFMA row,
// db = which of 4 MFMAs), so a lane reads V[tok][4c .. 4c+3] — 8 bytes —
// per token and v_perm builds the operands.
#include <math.h>

#include "common.h"

namespace sgl {
namespace {

constexpr int kD = 128;
constexpr int kBM = 128;   // packed query rows per workgroup (32 per wave)
constexpr int kBN = 64;    // kv tokens per LDS tile
constexpr int kPitch = kD + 8;  // LDS row pitch in bf16 (272 B: rotates banks per row)
constexpr int kThreads = 256;
constexpr float kRescaleSlack = 8.f;  // log2 units: p <= 256 between rescales

struct PrefillArgs {
  const uint16_t* q;
  int64_t q_st, q_sh;
  const uint16_t* kc;
  const uint16_t* vc;
  int64_t kv_ss, kv_sh;
  const int32_t* indices;
  const int32_t* qo_indptr;
  const int32_t* kv_indptr;
  const int32_t* q_start;  // optional first query row per request
  int group;
  float scale_log2;
  uint16_t* o;
  int64_t o_st, o_sh;
  int tiles_per_req;  // gridDim.x
};

// ds_read_b64_tr_b16: within each group of 16 lanes, lane i receives
// element i % 4 of the 4-element (8-byte) pieces addressed by lanes
// 4 e + i / 4, e < 4 -- a 4 x 16 -> 16 x 4 transpose of 16-bit data.
__device__ __forceinline__ bf16x4_t ds_read_tr16(const uint16_t* p) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(p));
  return __builtin_bit_cast(bf16x4_t, v);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(const u32x4_t& v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

// Gather one 64-token K and V tile into registers: thread handles 16-byte
// chunks tid + 256 u (u < 4) of each 16 KiB tile.
__device__ __forceinline__ void load_tile(const PrefillArgs& a, const uint16_t* kbase,
                                          const uint16_t* vbase, const int32_t* idx, int tile0,
                                          int kv_len, u32x4_t (&kr)[4], u32x4_t (&vr)[4]) {
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int id = threadIdx.x + kThreads * u;
    const int tok = id >> 4;
    const int ch = id & 15;
    const int t = min(tile0 + tok, kv_len - 1);
    const int64_t slot = idx[t];
    kr[u] = ldg128(kbase + slot * a.kv_ss + ch * 8);
    vr[u] = ldg128(vbase + slot * a.kv_ss + ch * 8);
  }
}

__device__ __forceinline__ void store_tile(uint16_t* ks, uint16_t* vs, const u32x4_t (&kr)[4],
                                           const u32x4_t (&vr)[4]) {
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int id = threadIdx.x + kThreads * u;
    const int tok = id >> 4;
    const int ch = id & 15;
    *reinterpret_cast<u32x4_t*>(ks + tok * kPitch + ch * 8) = kr[u];
    *reinterpret_cast<u32x4_t*>(vs + tok * kPitch + ch * 8) = vr[u];
  }
}

__global__ void __launch_bounds__(kThreads, 2) paged_prefill_kernel(PrefillArgs a) {
  const int r = blockIdx.z;
  const int h = blockIdx.y;
  // Heaviest (latest) query tiles first: causal work grows with the tile index.
  const int tile = a.tiles_per_req - 1 - blockIdx.x;
  const int qo_len = a.qo_indptr[r + 1] - a.qo_indptr[r];
  const int qo_beg = a.q_start ? a.q_start[r] : a.qo_indptr[r];
  const int kv_beg = a.kv_indptr[r];
  const int kv_len = a.kv_indptr[r + 1] - kv_beg;
  const int G = a.group;
  const int rows = qo_len * G;
  const int row0 = tile * kBM;
  if (row0 >= rows || kv_len <= 0) return;
  const int off = kv_len - qo_len;  // causal offset (cached prefix length)

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = lane & 31;
  const int hl = lane >> 5;

  // This lane's query row.
  const int prow = row0 + wave * 32 + c;
  const bool row_ok = prow < rows;
  const int qtok = row_ok ? prow / G : 0;
  const int qhead = h * G + (row_ok ? prow - (prow / G) * G : 0);
  const int allow = row_ok ? qtok + off : kv_len - 1;  // last visible kv token

  // Q^T operand: q[qtok][qhead][16 s + 8 hl .. +8], s < 8.
  bf16x8_t qop[8];
  {
    const uint16_t* qp =
        a.q + static_cast<int64_t>(qo_beg + qtok) * a.q_st + static_cast<int64_t>(qhead) * a.q_sh;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      u32x4_t v = row_ok ? ldg128(qp + 16 * s + 8 * hl) : u32x4_t{0, 0, 0, 0};
      qop[s] = as_bf16x8(v);
    }
  }

  // kv range this workgroup needs: up to the last row's visible token.
  const int last_row = min(rows, row0 + kBM) - 1;
  const int kv_end = min(kv_len, last_row / G + off + 1);
  const int ntiles = (kv_end + kBN - 1) / kBN;
  // First token index at which some row of the workgroup may be masked.
  const int first_masked = row0 / G + off + 1;

  __shared__ __attribute__((aligned(16))) uint16_t smem[2][2][kBN * kPitch];

  const uint16_t* kbase = a.kc + static_cast<int64_t>(h) * a.kv_sh;
  const uint16_t* vbase = a.vc + static_cast<int64_t>(h) * a.kv_sh;
  const int32_t* idx = a.indices + kv_beg;

  f32x16_t acc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[db][v] = 0.f;
  float m = -INFINITY;
  float l = 0.f;

  u32x4_t kr[4], vr[4];
  load_tile(a, kbase, vbase, idx, 0, kv_len, kr, vr);
  store_tile(smem[0][0], smem[0][1], kr, vr);
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int tile0 = t * kBN;
    const bool has_next = t + 1 < ntiles;
    if (has_next) load_tile(a, kbase, vbase, idx, tile0 + kBN, kv_len, kr, vr);
    const uint16_t* ks = smem[t & 1][0];
    const uint16_t* vs = smem[t & 1][1];
    // This lane's transpose-read source: group g = lane / 16 takes tokens
    // 4 (g / 2) + (lane % 16) / 4 and columns 16 (g % 2) + 4 (lane % 4).
    const uint16_t* vtr = vs + (4 * (lane >> 5) + ((lane & 15) >> 2)) * kPitch +
                          16 * ((lane >> 4) & 1) + 4 * (lane & 3);

    // S^T for tokens [32 mb, 32 mb + 32) of the tile.
    f32x16_t st[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int v = 0; v < 16; ++v) st[mb][v] = 0.f;
      const uint16_t* krow = ks + (32 * mb + c) * kPitch + 8 * hl;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const u32x4_t kv = *reinterpret_cast<const u32x4_t*>(krow + 16 * s);
        st[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(kv), qop[s], st[mb], 0, 0, 0);
      }
    }
    // Causal / length mask, only on tiles that reach past a row's last
    // visible token (a wave-uniform test, so full tiles skip it entirely).
    if (tile0 + kBN > first_masked || tile0 + kBN > kv_len) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int tok = tile0 + 32 * mb + 8 * (v >> 2) + 4 * hl + (v & 3);
          if (tok > allow || tok >= kv_len) st[mb][v] = -INFINITY;
        }
    }
    float mt = -INFINITY;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int v = 0; v < 16; ++v) mt = fmaxf(mt, st[mb][v]);
    mt = fmaxf(mt, __shfl_xor(mt, 32, kWave)) * a.scale_log2;
    // Lazy rescaling: the reference point m (log2 domain) only moves when a
    // row's max exceeds it by more than kRescaleSlack, so most tiles skip the
    // O rescale. Exact: every p and l use the same m; p <= 2^kRescaleSlack.
    const bool move = mt > m + kRescaleSlack;
    if (__builtin_amdgcn_ballot_w64(move) != 0) {
      const float mn = move ? mt : m;
      const float alpha = __builtin_amdgcn_exp2f(m - mn);  // 0 on the first tile
      l *= alpha;
      m = mn;
#pragma unroll
      for (int db = 0; db < 4; ++db) acc[db] *= alpha;
    }
    const float neg_m = m == -INFINITY ? 0.f : -m;  // a row with nothing visible yet
    float ps = 0.f;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        // v_exp_f32 directly: arguments are <= kRescaleSlack, and results
        // below 2^-126 flush to zero, which a bf16 weight could not hold.
        const float p = __builtin_amdgcn_exp2f(fmaf(st[mb][v], a.scale_log2, neg_m));
        st[mb][v] = p;
        ps += p;
      }
    }
    l += ps;

    // O^T += V^T P^T over 4 k-steps of 16 tokens.
#pragma unroll
    for (int ks4 = 0; ks4 < 4; ++ks4) {
      const int mb = ks4 >> 1;
      const int vb = (ks4 & 1) * 8;
      u32x4_t pw;
#pragma unroll
      for (int k = 0; k < 4; ++k) pw[k] = pack_bf16x2(st[mb][vb + 2 * k], st[mb][vb + 2 * k + 1]);
      const bf16x8_t pop = as_bf16x8(pw);
      // Slots 0-3 <-> tokens 16 ks4 + 4 hl + (0..3), slots 4-7 <-> the same + 8
      // (the S^T accumulator order). V^T rows come straight from the
      // row-major tile with transpose reads: in each 16-lane group, lane j
      // points at V[tok0 + j / 4][d0 + 4 (j % 4) ..] and lane i receives
      // V[tok0 + e][d0 + i] for e < 4.
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const uint16_t* vp = vtr + (16 * ks4) * kPitch + 32 * db;
        const bf16x4_t lo = ds_read_tr16(vp);
        const bf16x4_t hi = ds_read_tr16(vp + 8 * kPitch);
        const bf16x8_t vop = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vop, pop, acc[db], 0, 0, 0);
      }
    }

    if (has_next) store_tile(smem[(t + 1) & 1][0], smem[(t + 1) & 1][1], kr, vr);
    __syncthreads();
  }

  l += __shfl_xor(l, 32, kWave);
  if (!row_ok) return;
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  // acc[db][4 g + i] holds d = 32 db + 8 g + 4 hl + i.
  uint16_t* op =
      a.o + static_cast<int64_t>(qo_beg + qtok) * a.o_st + static_cast<int64_t>(qhead) * a.o_sh;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const u32x2_t w = {pack_bf16x2(acc[db][4 * g] * inv, acc[db][4 * g + 1] * inv),
                         pack_bf16x2(acc[db][4 * g + 2] * inv, acc[db][4 * g + 3] * inv)};
      *reinterpret_cast<u32x2_t*>(op + 32 * db + 8 * g + 4 * hl) = w;
    }
}

}  // namespace
}  // namespace sgl

using namespace sgl;

extern "C" int sgl_paged_prefill(const void* q, int64_t q_stride_token, int64_t q_stride_head,
                                 const void* k_cache, const void* v_cache, int64_t kv_stride_slot,
                                 int64_t kv_stride_head, const int32_t* indices,
                                 const int32_t* qo_indptr, const int32_t* kv_indptr,
                                 const int32_t* q_start, int batch_size, int max_qo_len,
                                 int num_qo_heads,
                                 int num_kv_heads, int head_dim, float sm_scale, void* o,
                                 int64_t o_stride_token, int64_t o_stride_head, void* stream) {
  if (batch_size < 0 || max_qo_len < 0 || num_qo_heads <= 0 || num_kv_heads <= 0)
    return SGL_ERR_INVALID_ARG;
  if (batch_size == 0 || max_qo_len == 0) return SGL_OK;
  if (!q || !k_cache || !v_cache || !indices || !qo_indptr || !kv_indptr || !o)
    return SGL_ERR_INVALID_ARG;
  if (num_qo_heads % num_kv_heads != 0) return SGL_ERR_INVALID_ARG;
  if (head_dim != kD) return SGL_ERR_UNSUPPORTED;
  if (q_stride_head % 8 || q_stride_token % 8 || kv_stride_slot % 8 || kv_stride_head % 8 ||
      o_stride_token % 8 || o_stride_head % 8 || !aligned16(q) || !aligned16(k_cache) ||
      !aligned16(v_cache) || !aligned16(o))
    return SGL_ERR_ALIGNMENT;
  const int group = num_qo_heads / num_kv_heads;
  const int64_t tiles = (static_cast<int64_t>(max_qo_len) * group + kBM - 1) / kBM;
  if (tiles > 0x7fffffff) return SGL_ERR_INVALID_ARG;
  PrefillArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_st = q_stride_token;
  a.q_sh = q_stride_head;
  a.kc = static_cast<const uint16_t*>(k_cache);
  a.vc = static_cast<const uint16_t*>(v_cache);
  a.kv_ss = kv_stride_slot;
  a.kv_sh = kv_stride_head;
  a.indices = indices;
  a.qo_indptr = qo_indptr;
  a.kv_indptr = kv_indptr;
  a.q_start = q_start;
  a.group = group;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.o = static_cast<uint16_t*>(o);
  a.o_st = o_stride_token;
  a.o_sh = o_stride_head;
  a.tiles_per_req = static_cast<int>(tiles);
  hipLaunchKernelGGL(paged_prefill_kernel, dim3(tiles, num_kv_heads, batch_size),
                     dim3(kThreads), 0, static_cast<hipStream_t>(stream), a);
  return launch_status();
}
