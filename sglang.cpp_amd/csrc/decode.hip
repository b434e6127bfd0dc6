// Split-KV paged decode on gfx950.
//
// Reference semantics: FlashInferBackend::forward, decode branch
// (src/attention/flashinfer_backend.cu:553-595): for request r and q head h,
//   o[r, h] = softmax_j(q[r, h] . K[indices[kv_indptr[r] + j], h / G] * sm_scale)
//             . V[indices[kv_indptr[r] + j], h / G]
// with the page table token-granular (page_size 1), no window, no soft-cap.
//
// Schedule: persistent and token balanced. The batch's flattened KV token
// stream (request r owns [kv_indptr[r], kv_indptr[r+1])) is cut into
// num_units units of W tokens, one per resident workgroup, so every
// workgroup streams the same number of tokens to the end instead of a few
// long requests leaving a tail. W is picked on the device from
// kv_indptr[batch], which keeps a plan built for a worst-case batch (graph
// capture) valid and balanced for any shorter batch replayed with it.
//   * One wave per kv head: each K/V byte is read from HBM once and feeds all
//     G query heads of that kv head (GQA sharing).
//   * 16-token steps on the matrix cores: S^T = K . Q^T on
//     v_mfma_f32_16x16x32_bf16 (Q^T from a per-wave LDS copy; K straight
//     from HBM into the operand registers, or, where a CU's own stream rate
//     sets the time, loaded as whole rows and transposed through a per-wave
//     LDS tile), O^T += V^T . P^T on v_mfma_f32_16x16x16bf16_1k fed from the
//     S^T accumulators; the online softmax is lane-local plus two lane
//     exchanges.
//   * K and V of step t+1 are issued before the products of step t.
//   * The decode-only launch keeps each wave's finished pieces (output rows,
//     or split partials) in an LDS ring and writes them when its unit is
//     done (or the ring is full): stores interleaved with the unit's read
//     stream cost far more than their bytes (config 4 shape, same tokens:
//     -1.4% at 256 requests, -7% at 2,048).
// A request that spans units is written as fp32 partials (normalised output
// plus log2-sum-exp) into two slots per unit -- slot 2u for the piece of the
// request running into unit u from before it, slot 2u+1 for the piece of the
// request that starts inside u and runs past it -- and folded by a second,
// short kernel. Merging inside the decode launch would need the pieces
// written coherently across the XCDs' L2s (agent-scope releases, which write
// back the L2, or write-through stores): both measured slower than the
// kernel boundary.
//
// A batch whose tokens exceed the plan's capacity (num_units * W_max) is not
// processed silently wrong: the merge kernel writes NaN to the rows of every
// request reaching past the capacity and sets the workspace's status word to
// SGL_ERR_CAPACITY (cleared by every launch).
#include <math.h>

#include <mutex>
#include <type_traits>

#include "common.h"
#include "prefill_impl.h"

namespace sgl {
namespace {

constexpr int kD = 128;
constexpr int kStep = 16;       // tokens per pipeline step
constexpr int kTile = 32;       // chunk granularity (tokens)
constexpr int kMaxKvHeads = 16; // kv heads per workgroup (one wave each)
constexpr int kMaxGroup = 16;
constexpr int kMinUnit = 64;    // smallest unit: keeps per-unit set-up small next to the stream
constexpr int kMaxChunkTokens = 8192;  // slot indices of a chunk staged in LDS (32 KiB)
constexpr int kQPitch = kD + 8; // LDS row pitch (bf16) of the Q^T copy
constexpr float kRescaleSlack = 8.f;  // log2 units: p <= 256 between rescales

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
  float* part_o;     // [2 num_units, hq, D]
  float* part_lse;   // [2 num_units, hq]
  int32_t* status;   // workspace status word
  int32_t* unit_req; // [num_units]: the request running into unit u from before, or -1
  int chunk;         // W_max: largest unit (LDS staging capacity)
  int chunk_min;     // W_min: smallest unit
  int batch;
  int num_units;     // workgroups of the decode launch
  int out_bytes;     // decode-only launch: bytes of each wave's LDS output ring (0: write directly)
};

// Unit size for this launch: the batch's tokens spread evenly over the
// launched units, in whole 16-token steps, within the plan's [W_min, W_max].
// Read from kv_indptr on the device, so a plan built for a worst-case batch
// (graph capture) stays balanced for the shorter batch actually replayed.
__device__ __forceinline__ int unit_tokens(const DecodeArgs& a, int total) {
  int w = (total + a.num_units - 1) / a.num_units;
  w = (w + 15) / 16 * 16;
  return max(a.chunk_min, min(a.chunk, w));
}

// Per-wave LDS scratch.
struct WaveLds {
  uint16_t q[16 * kQPitch];  // Q rows of the wave's G heads (zero rows past G)
};

// Per-wave LDS of the decode role that loads K as whole rows: Q, and the
// 16-token x 16-chunk K tile of the step being transposed (chunk c of token
// t at 16 t + (c ^ t), which keeps both the row writes and the column reads
// free of bank conflicts).
struct RowKWaveLds : WaveLds {
  u32x4_t kt[256];
};
template <bool kRows>
using UnitWaveLds = std::conditional_t<kRows, RowKWaveLds, WaveLds>;

// Workspace carve-up shared by the plan and the launch: a 256-byte header
// (int32 status word at offset 0), then the partial outputs and their
// log2-sum-exp, two slots per unit, then per unit the request that runs into
// it from an earlier unit (-1 if none).
struct WorkspaceLayout {
  int64_t part_o_off, part_lse_off, unit_req_off, total;
};

inline WorkspaceLayout workspace_layout(int num_units, int hq) {
  WorkspaceLayout w;
  const int64_t npart = 2 * static_cast<int64_t>(num_units) * hq;
  auto align = [](int64_t x) { return (x + 255) / 256 * 256; };
  w.part_o_off = 256;
  w.part_lse_off = w.part_o_off + align(npart * kD * 4);
  w.unit_req_off = w.part_lse_off + align(npart * 4);
  w.total = w.unit_req_off + align(static_cast<int64_t>(num_units) * 4);
  return w;
}

__device__ __forceinline__ bf16x8_t as_bf16x8(const u32x4_t& v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

// Orders LDS traffic between lanes of one wave (the LDS executes a wave's
// operations in order; this only stops the compiler from moving them).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Row addresses are a lane base plus the slot times the slot stride in
// bytes, one 32 x 32 -> 64-bit multiply-add (the stride is < 2^31 bytes and
// slots are non-negative int32).
__device__ __forceinline__ const char* slot_row(const char* lane_base, int slot, uint32_t ss_bytes) {
  return lane_base + static_cast<uint64_t>(static_cast<uint32_t>(slot)) * ss_bytes;
}

// K operand of a 16-token step: lane (n, j) holds K[tok n][32 s + 8 j .. + 8]
// (klane: the head's row 0 plus 8 j elements).
__device__ __forceinline__ void load_k_step(const char* klane, uint32_t ss_bytes, int slot,
                                            u32x4_t (&kr)[4]) {
  const char* row = slot_row(klane, slot, ss_bytes);
#pragma unroll
  for (int s = 0; s < 4; ++s) kr[s] = ldg128(reinterpret_cast<const uint16_t*>(row) + 32 * s);
}

// V rows of a 16-token step: lane (n, j) holds V[tok 4 j + e][8 n .. 8 n + 7]
// for e < 4, so each load instruction reads four whole 256-byte rows
// (vlane: the head's row 0 plus 8 n elements). Tokens at or past `len`
// re-read the last valid row (an L2 hit).
__device__ __forceinline__ void load_v_step(const char* vlane, uint32_t ss_bytes,
                                            const int32_t* sidx, int tb, int len, int j,
                                            u32x4_t (&vr)[4]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int tok = min(tb + 4 * j + e, len - 1);
    // Non-temporal: each V row is read exactly once, whole, by this
    // instruction (measured -9% kernel time at config 4). K rows are not:
    // their 64-byte halves come from two instructions and the second one
    // hits the line the first brought into L2.
    vr[e] = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4_t*>(slot_row(vlane, sidx[tok], ss_bytes)));
  }
}

// A operand of O^T MFMA nb: V^T[d = 8 n + nb][tok 4 j + e] for e < 4, built
// from the four rows by byte permutes (bf16 element nb of each row).
template <int nb>
__device__ __forceinline__ bf16x4_t v_operand(const u32x4_t (&vr)[4]) {
  constexpr int w = nb / 2;
  constexpr uint32_t sel = (nb & 1) ? 0x07060302u : 0x05040100u;
  u32x2_t out;
  out[0] = __builtin_amdgcn_perm(vr[1][w], vr[0][w], sel);
  out[1] = __builtin_amdgcn_perm(vr[3][w], vr[2][w], sel);
  return __builtin_bit_cast(bf16x4_t, out);
}

// Softmax state of one wave's piece (lane (n, j): head n, d = 32 j + 8 i + nb
// in acc[nb][i]), for the small-batch kernel's in-workgroup fold.
struct HeadState {
  float m, l;
  f32x4_t acc[8];
};

// One wave: kv head h over the `len` tokens whose slots are sidx[0, len)
// (one piece of a request). whole: the piece is the whole request (output
// written directly); otherwise it goes to partial slot pslot. kState: leave
// the state in *st instead (no output). kBarrier: a workgroup barrier per
// step, for workgroups whose waves are exactly one unit's kv heads (the
// waves of the small-batch kernel, and units sharing a workgroup, take
// pieces of different lengths).
//
// Per 16-token step (v_mfma, lane l, n = l % 16, j = l / 16):
//   S^T[tok, head] = K . Q^T          4 x 16x16x32: rows tok, columns head
//   O^T[d, head]  += V^T . P^T        8 x 16x16x16: k = the step's 16 tokens
// S^T's accumulator layout (lane holds tokens 4 j .. 4 j + 3 of head n) is
// exactly the B operand P^T the second product needs, and both put the head
// on the lane's column, so max, sum and the rescale of O are lane-local apart
// from one exchange across the four lane groups.
//
// K and V of step t + 1 are in flight during step t; the Q rows are loaded
// first and the first step's K/V rows issued before Q is waited for.
template <bool kState, bool kBarrier = !kState, bool kRows = false>
__device__ __forceinline__ void decode_head(const DecodeArgs& a, WaveLds& L, const int32_t* sidx,
                                            int pslot, bool whole, int h, int len, int qrow,
                                            int lane, HeadState* st = nullptr,
                                            u32x4_t* kt = nullptr, char* oslot = nullptr) {
  const int n = lane & 15;
  const int j = lane >> 4;
  const int G = a.group;
  const bool head_ok = n < G;
  const char* klane = reinterpret_cast<const char*>(a.kc + static_cast<int64_t>(h) * a.kv_sh + 8 * j);
  const char* vlane = reinterpret_cast<const char*>(a.vc + static_cast<int64_t>(h) * a.kv_sh + 8 * n);
  const char* krow = reinterpret_cast<const char*>(a.kc + static_cast<int64_t>(h) * a.kv_sh + 8 * n);
  const uint32_t ss_bytes = static_cast<uint32_t>(a.kv_ss * 2);

  // Q rows of this kv head's G query heads (16 rows x 16 chunks), for LDS.
  u32x4_t qv[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int row = u * 4 + j;
    qv[u] = u32x4_t{0, 0, 0, 0};
    if (row < G)
      qv[u] = ldg128(a.q + static_cast<int64_t>(qrow) * a.q_st +
                     static_cast<int64_t>(h * G + row) * a.q_sh + n * 8);
  }

  // K and V rows of the first step in flight, K issued first as inside the
  // loop (the loop-head wait counts merge both paths).
  u32x4_t kr[4], vr[4];
  // kRows: K is loaded as V is (lane (n, j): token 4 j + e, chunk n, whole
  // rows per instruction) and turned into the operand layout (token n,
  // chunk 4 s + j) through the wave's LDS tile at the top of each step.
  auto transpose_k = [&]() {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int tr = 4 * j + e;
      kt[16 * tr + (n ^ tr)] = kr[e];
    }
    wave_lds_sync();
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) kr[s4] = kt[16 * n + ((4 * s4 + j) ^ n)];
    wave_lds_sync();
  };
  if constexpr (kRows)
    load_v_step(krow, ss_bytes, sidx, 0, len, j, kr);
  else
    load_k_step(klane, ss_bytes, sidx[min(n, len - 1)], kr);
  __builtin_amdgcn_sched_barrier(0);
  load_v_step(vlane, ss_bytes, sidx, 0, len, j, vr);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < 4; ++u) *reinterpret_cast<u32x4_t*>(L.q + (u * 4 + j) * kQPitch + n * 8) = qv[u];
  wave_lds_sync();

  float m = -INFINITY;  // running reference point of head n (replicated over j)
  float l = 0.f;        // partial sum over this lane's tokens of head n
  f32x4_t acc[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) acc[nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // S^T of one step.
  auto qk = [&](const u32x4_t (&k)[4]) {
    f32x4_t sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const bf16x8_t qop = *reinterpret_cast<const bf16x8_t*>(L.q + n * kQPitch + 32 * s + 8 * j);
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(k[s]), qop, sacc, 0, 0, 0);
    }
    return sacc;
  };
  // Online softmax of the step starting at token t, then O^T += V^T P^T.
  auto softmax_pv = [&](const f32x4_t& sacc, const u32x4_t (&vv)[4], int t) {
    // Log2 domain with a lazy reference point: m only moves when a head's
    // step maximum exceeds it by more than kRescaleSlack, so most steps skip
    // the rescale of O. Exact: p and l of a head always use the same m, and
    // p <= 2^kRescaleSlack.
    const int last = len - t - 1;
    float sc[4];
    float mt = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sc[i] = (4 * j + i <= last) ? sacc[i] : -INFINITY;
      mt = fmaxf(mt, sc[i]);
    }
    mt = max_xor32(max_xor16(mt)) * a.scale_log2;
    const bool move = mt > m + kRescaleSlack;
    if (__builtin_amdgcn_ballot_w64(move) != 0) {
      const float mn = move ? mt : m;
      const float alpha = __builtin_amdgcn_exp2f(m - mn);  // 0 on the first step
      l *= alpha;
      m = mn;
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) acc[nb] *= alpha;
    }
    // v_exp_f32 directly: arguments are <= kRescaleSlack, and results below
    // 2^-126 flush to zero, which a bf16 weight could not hold anyway.
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(fmaf(sc[i], a.scale_log2, -m));
    l += (p[0] + p[1]) + (p[2] + p[3]);
    u32x2_t pw = {pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3])};
    const bf16x4_t pop = __builtin_bit_cast(bf16x4_t, pw);
    static_for<0, 8>([&](auto NB) {
      constexpr int nb = decltype(NB)::value;
      acc[nb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(v_operand<nb>(vv), pop, acc[nb], 0, 0, 0);
    });
  };

  for (int t = 0; t < len; t += kStep) {
    // Keep the workgroup's waves (one per kv head) in step: together they
    // read each token's whole [Hkv, D] row, which DRAM serves better as one
    // burst than as per-head pieces spread over time.
    if constexpr (kBarrier) __builtin_amdgcn_s_barrier();
    const int tn = t + kStep;
    f32x4_t sacc;
    if constexpr (kRows) {
      transpose_k();
      sacc = qk(kr);
      __builtin_amdgcn_sched_barrier(0);
      load_v_step(krow, ss_bytes, sidx, tn, len, j, kr);  // K of the next step
    } else {
      const int kslot_next = sidx[min(tn + n, len - 1)];
      sacc = qk(kr);
      __builtin_amdgcn_sched_barrier(0);
      load_k_step(klane, ss_bytes, kslot_next, kr);  // K of the next step
    }
    __builtin_amdgcn_sched_barrier(0);
    softmax_pv(sacc, vr, t);
    __builtin_amdgcn_sched_barrier(0);
    load_v_step(vlane, ss_bytes, sidx, tn, len, j, vr);  // V of the next step
    __builtin_amdgcn_sched_barrier(0);
  }
  l = sum_xor32(sum_xor16(l));
  if constexpr (kState) {
    st->m = m;
    st->l = l;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) st->acc[nb] = acc[nb];
    return;
  }
  if (!head_ok) return;
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  const int head = h * G + n;
  // Lane holds O[head n][d = 32 j + 8 i + nb] in acc[nb][i].
  if (oslot) {
    // Into the wave's LDS output record (head n's row at 16 + 256 n for a
    // whole request's bf16 output, at 16 + 512 n for a partial's fp32, its
    // log2-sum-exp at 16 + 512 G + 4 n); written to memory when the unit is
    // done.
    char* row = oslot + 16 + (whole ? 256 : 512) * n;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (whole) {
        float v[8];
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) v[nb] = acc[nb][i] * inv;
        *reinterpret_cast<u32x4_t*>(row + 2 * (32 * j + 8 * i)) = pack8(v);
      } else {
        f32x4_t v0, v1;
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
          v0[nb] = acc[nb][i] * inv;
          v1[nb] = acc[nb + 4][i] * inv;
        }
        *reinterpret_cast<f32x4_t*>(row + 4 * (32 * j + 8 * i)) = v0;
        *reinterpret_cast<f32x4_t*>(row + 4 * (32 * j + 8 * i + 4)) = v1;
      }
    }
    if (!whole && j == 0)
      *reinterpret_cast<float*>(oslot + 16 + 512 * G + 4 * n) = l > 0.f ? m + log2f(l) : -INFINITY;
    return;
  }
  if (whole) {
    uint16_t* op = a.o + static_cast<int64_t>(qrow) * a.o_st + static_cast<int64_t>(head) * a.o_sh;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v[8];
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) v[nb] = acc[nb][i] * inv;
      stg128(op + 32 * j + 8 * i, pack8(v));
    }
  } else {
    const int64_t pidx = static_cast<int64_t>(pslot) * a.hq + head;
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

// Zero output row of an empty request (kv_len 0), by threads t, t + n, ...
__device__ __forceinline__ void zero_row(const DecodeArgs& a, int qrow, int t, int n) {
  for (int e = t; e < a.hq * (kD / 8); e += n) {
    const int hh = e / (kD / 8);
    stg128(a.o + static_cast<int64_t>(qrow) * a.o_st + static_cast<int64_t>(hh) * a.o_sh +
               (e - hh * (kD / 8)) * 8,
           u32x4_t{0, 0, 0, 0});
  }
}

constexpr size_t kMaxOutRing = 32 * 1024;  // output ring bytes per wave of the decode-only launch

// LDS bytes of one unit: the per-wave Q copies, then the unit's slot
// indices. kRows: the per-wave K tile of whole-row K loads too.
template <bool kRows>
__device__ __host__ inline size_t unit_lds_bytes(int hkv, int chunk) {
  return static_cast<size_t>(hkv) * sizeof(UnitWaveLds<kRows>) +
         static_cast<size_t>(chunk) * sizeof(int32_t);
}

// Offset of the decode-only launch's output rings in a unit's LDS.
__device__ __host__ inline size_t out_ring_offset(int hkv, int chunk) {
  return (unit_lds_bytes<false>(hkv, chunk) + 15) / 16 * 16;
}

// Bytes of one output record: a 16-byte header (whole, row, partial slot,
// record bytes), then the G rows (bf16 for a whole request, fp32 and the
// log2-sum-exp for a partial).
__device__ __host__ inline int out_record_bytes(int group, bool whole) {
  return whole ? 16 + 256 * group : (16 + 512 * group + 4 * group + 15) / 16 * 16;
}

// Writes the records of a wave's output ring ([0, used) bytes) to memory,
// kv head h.
__device__ __forceinline__ void flush_ring(const DecodeArgs& a, const char* ring, int used, int h,
                                           int lane) {
  const int G = a.group;
  wave_lds_sync();
  for (int at = 0; at < used;) {
    const char* sl = ring + at;
    const int* hdr = reinterpret_cast<const int*>(sl);
    const int whole = __builtin_amdgcn_readfirstlane(hdr[0]);
    const int qrow = __builtin_amdgcn_readfirstlane(hdr[1]);
    const int pslot = __builtin_amdgcn_readfirstlane(hdr[2]);
    at += __builtin_amdgcn_readfirstlane(hdr[3]);
    if (whole) {
      for (int e = lane; e < G * 16; e += kWave) {
        const int g = e >> 4, c = e & 15;
        stg128(a.o + static_cast<int64_t>(qrow) * a.o_st + static_cast<int64_t>(h * G + g) * a.o_sh +
                   c * 8,
               *reinterpret_cast<const u32x4_t*>(sl + 16 + 256 * g + 16 * c));
      }
    } else {
      const int64_t p0 = static_cast<int64_t>(pslot) * a.hq + h * G;
      for (int e = lane; e < G * 32; e += kWave) {
        const int g = e >> 5, c = e & 31;
        *reinterpret_cast<f32x4_t*>(a.part_o + (p0 + g) * kD + 4 * c) =
            *reinterpret_cast<const f32x4_t*>(sl + 16 + 512 * g + 16 * c);
      }
      if (lane < G) a.part_lse[p0 + lane] = *reinterpret_cast<const float*>(sl + 16 + 512 * G + 4 * lane);
    }
  }
  wave_lds_sync();
}

// Persistent, token-balanced schedule: unit u takes the tokens
// [u W, (u+1) W) of the flattened stream, which may cover the tail of one
// request, whole requests and the head of another; one wave per kv head.
// The workgroup (index blk) holds UPW units, unit blk UPW + g on waves
// [g hkv, (g + 1) hkv) with LDS region g (unit_lds_bytes each); units past
// num_units idle. kBarrier: the units' waves keep in step (UPW = 1 only).
// kRows: K rows are loaded whole and transposed through LDS (the decode
// role of the fused decode + prefill launch, where the decode has only part
// of the CUs and its per-CU stream rate sets the step: +1.5% on config 5's
// step; with the whole device the HBM bandwidth is the limit and the
// transpose costs 1% on config 4).
template <int UPW, bool kBarrier, bool kRows = false>
__device__ __forceinline__ void decode_units(const DecodeArgs& a, char* smem, int blk) {
  static_assert(UPW == 1 || !kBarrier, "a per-step barrier needs one unit per workgroup");
  const int lane = threadIdx.x & 63;
  const int wave_all = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform per wave
  const int g = UPW == 1 ? 0 : wave_all / a.hkv;
  const int wave = wave_all - g * a.hkv;  // the kv head
  const int gt = static_cast<int>(threadIdx.x) - g * a.hkv * kWave;  // thread index in the unit
  const int gn = a.hkv * kWave;
  const int u = blk * UPW + g;
  const int total = a.kv_indptr[a.batch];
  const int W = unit_tokens(a, total);
  const int tok0 = u * W;
  const int tok1 = min(total, tok0 + W);
  const bool last_unit = tok1 == total;
  // The merge kernel, stream-ordered after this launch, reports capacity
  // overflows; every launch starts from a clear status.
  if (u == 0 && gt == 0) *a.status = SGL_OK;
  const bool active = u < a.num_units && tok0 < tok1;
  char* base = smem + g * unit_lds_bytes<kRows>(a.hkv, a.chunk);
  int32_t* sidx = reinterpret_cast<int32_t*>(base + a.hkv * sizeof(UnitWaveLds<kRows>));
  int r = 0;
  if (active) {
    // First i in [0, batch] with kv_indptr[i] >= tok0 (uniform binary search).
    int lo = 0, hi = a.batch;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (a.kv_indptr[mid] < tok0) lo = mid + 1; else hi = mid;
    }
    // Request lo - 1 runs across tok0 when its end kv_indptr[lo] lies past tok0.
    r = (lo > 0 && a.kv_indptr[lo] > tok0) ? lo - 1 : lo;
    if (gt == 0) a.unit_req[u] = r < a.batch && a.kv_indptr[r] < tok0 ? r : -1;
    // Stage the unit's slot indices (shared by every kv head) in LDS.
    for (int e = gt; e < tok1 - tok0; e += gn) sidx[e] = a.indices[tok0 + e];
  } else if (u < a.num_units && gt == 0) {
    a.unit_req[u] = -1;
  }
  __syncthreads();
  if (!active) {
    // Past the end of the token stream: only an all-empty batch needs work.
    if (total == 0 && u == 0)
      for (int rr = 0; rr < a.batch; ++rr) zero_row(a, a.q_indptr ? a.q_indptr[rr] : rr, gt, gn);
    return;
  }
  UnitWaveLds<kRows>& L = reinterpret_cast<UnitWaveLds<kRows>*>(base)[wave];
  // Decode-only launch: finished pieces go to the wave's LDS output ring and
  // reach memory when the unit is done (or the ring is full): stores
  // interleaved with the unit's read stream cost far more than their bytes.
  const bool defer = UPW == 1 && kBarrier && !kRows && a.out_bytes > 0;
  char* ring = smem + out_ring_offset(a.hkv, a.chunk) + static_cast<size_t>(wave) * a.out_bytes;
  int used = 0;

  for (; r < a.batch; ++r) {
    const int rb = a.kv_indptr[r];
    const int re = a.kv_indptr[r + 1];
    // Requests starting at or past tok1 belong to later units, except empty
    // requests at the very end of the stream, which the last unit owns.
    if (rb >= tok1 && !(last_unit && rb == total)) break;
    const int qrow = a.q_indptr ? a.q_indptr[r] : r;
    if (re == rb) {  // empty request: zero output row
      zero_row(a, qrow, gt, gn);
      continue;
    }
    const int s0 = max(rb, tok0);
    const int s1 = min(re, tok1);
    if (s1 <= s0) continue;
    const bool whole = rb >= tok0 && re <= tok1;
    const int pslot = 2 * u + (rb > tok0 ? 1 : 0);
    u32x4_t* kt = nullptr;
    if constexpr (kRows) kt = L.kt;
    char* oslot = nullptr;
    if (defer) {
      const int rec = out_record_bytes(a.group, whole);
      if (used + rec > a.out_bytes) {
        flush_ring(a, ring, used, wave, lane);
        used = 0;
      }
      oslot = ring + used;
      if (lane == 0) {
        int* hdr = reinterpret_cast<int*>(oslot);
        hdr[0] = whole;
        hdr[1] = qrow;
        hdr[2] = pslot;
        hdr[3] = rec;
      }
      used += rec;
    }
    decode_head<false, kBarrier, kRows>(a, L, sidx + (s0 - tok0), pslot, whole, wave, s1 - s0,
                                        qrow, lane, nullptr, kt, oslot);
  }
  if (defer) flush_ring(a, ring, used, wave, lane);
}

// One unit per workgroup (one wave per kv head), about 8 waves per CU.
// Budget 128 VGPRs (up to 4 waves per SIMD, above the ~2 the schedule keeps
// resident): a tighter budget spills, and scratch traffic in the step loop
// costs ~9%.
__global__ void __launch_bounds__(kMaxKvHeads * kWave)
    __attribute__((amdgpu_waves_per_eu(4))) paged_decode_kernel(DecodeArgs a) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  decode_units<1, true>(a, smem, blockIdx.x);
}


// Decode units and causal-prefill items in one launch: workgroups
// [0, dec_blocks) take UPW decode units each (8 waves = UPW x hkv), the rest
// take the prefill's 8-wave items in heavy-first order. Blocks are
// dispatched in index order, so the decode workgroups occupy dec_blocks CUs
// (one per CU: a workgroup holds every register of its CU) while the
// prefill items fill the others and, as the decode finishes, every CU; the
// HBM-bound decode and the MFMA-bound prefill then run side by side instead
// of one after the other.
template <int UPW>
__global__ void __launch_bounds__(512, 1) mixed_attention_kernel(DecodeArgs d, pf::PrefillArgs p,
                                                                  int dec_blocks) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  if (static_cast<int>(blockIdx.x) < dec_blocks)
    decode_units<UPW, false, true>(d, smem, blockIdx.x);
  else
    pf::prefill_item<8, false, 1>(p, smem, static_cast<int>(blockIdx.x) - dec_blocks,
                                  static_cast<int>(gridDim.x) - dec_blocks);
}

// Small batches (every unit at the 64-token minimum and at most one
// workgroup per CU for each (request, kv head)): one 8-wave workgroup per
// (kv head, request), the request's tokens cut into 8 contiguous pieces, one
// per wave, and the waves' softmax states folded through LDS by wave 0 --
// one launch instead of decode + merge, which is what such a call is bound
// by. The plan's capacity contract is kept: requests reaching past
// num_units * W_max tokens get NaN rows, and workgroup (0, 0) sets the status
// word from kv_indptr[batch] (a request reaches past the capacity exactly
// when the batch's total does), so no other workgroup writes it.
// Each wave streams one kv head's 256-byte row slices, so K is loaded as
// whole rows and transposed through LDS (-13% kernel time at config 1).
constexpr int kSmallWaves = 8;
constexpr int kSmallStage = 8192;  // slot indices staged in LDS (longer requests read them from HBM)

__global__ void __launch_bounds__(kSmallWaves * kWave) paged_decode_small_kernel(DecodeArgs a) {
  __shared__ WaveLds ql[kSmallWaves];
  __shared__ int32_t slots[kSmallStage];
  // The waves' K tiles while they stream, then the exchange of their states.
  __shared__ union {
    u32x4_t kt[kSmallWaves][256];
    float xch[34][kSmallWaves][kWave];
  } xs;
  auto& xch = xs.xch;
  const int h = blockIdx.x;
  const int r = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = a.group;
  const int total = a.kv_indptr[a.batch];
  const int W = unit_tokens(a, total);
  const int64_t cover = static_cast<int64_t>(a.num_units) * W;
  if (h == 0 && r == 0 && threadIdx.x == 0)
    *a.status = static_cast<int64_t>(total) > cover ? SGL_ERR_CAPACITY : SGL_OK;
  const int rb = a.kv_indptr[r];
  const int re = a.kv_indptr[r + 1];
  const int qrow = a.q_indptr ? a.q_indptr[r] : r;
  const int len = re - rb;
  if (static_cast<int64_t>(re) > cover || len <= 0) {
    // Past the capacity: NaN rows; empty request: zero rows (G heads of h).
    const uint32_t fill = len <= 0 ? 0u : 0x7fc07fc0u;
    for (int e = threadIdx.x; e < G * (kD / 8); e += blockDim.x) {
      const int g = e / (kD / 8);
      stg128(a.o + static_cast<int64_t>(qrow) * a.o_st + static_cast<int64_t>(h * G + g) * a.o_sh +
                 (e - g * (kD / 8)) * 8,
             u32x4_t{fill, fill, fill, fill});
    }
    return;
  }
  const int32_t* sp = a.indices + rb;
  if (len <= kSmallStage) {
    for (int e = threadIdx.x; e < len; e += blockDim.x) slots[e] = sp[e];
    __syncthreads();
    sp = slots;
  }
  const int per = ((len + kSmallWaves - 1) / kSmallWaves + kStep - 1) / kStep * kStep;
  const int t0 = min(len, wave * per);
  const int t1 = min(len, t0 + per);
  HeadState st;
  st.m = -INFINITY;
  st.l = 0.f;
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) st.acc[nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  if (t0 < t1)
    decode_head<true, false, true>(a, ql[wave], sp + t0, 0, false, h, t1 - t0, qrow, lane, &st,
                                   xs.kt[wave]);
  __syncthreads();  // every K tile read before the exchange overwrites them
#pragma unroll
  for (int nb = 0; nb < 8; ++nb)
#pragma unroll
    for (int i = 0; i < 4; ++i) xch[4 * nb + i][wave][lane] = st.acc[nb][i];
  xch[32][wave][lane] = st.m;
  xch[33][wave][lane] = st.l;
  __syncthreads();
  if (wave != 0) return;
  // Wave 0 folds the pieces in wave order (the largest log2-sum-exp first,
  // then the weighted sums), as the merge kernel folds units.
  const int n = lane & 15;
  const int j = lane >> 4;
  if (n >= G) return;
  float mx = -INFINITY;
#pragma unroll
  for (int w = 0; w < kSmallWaves; ++w) mx = fmaxf(mx, xch[32][w][lane]);
  float den = 0.f;
  f32x4_t acc[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) acc[nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int w = 0; w < kSmallWaves; ++w) {
    const float mw = xch[32][w][lane];
    const float wgt = mw == -INFINITY ? 0.f : exp2f(mw - mx);
    den += xch[33][w][lane] * wgt;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[nb][i] += xch[4 * nb + i][w][lane] * wgt;
  }
  const float inv = den > 0.f ? 1.0f / den : 0.f;
  uint16_t* op = a.o + static_cast<int64_t>(qrow) * a.o_st + static_cast<int64_t>(h * G + n) * a.o_sh;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float v[8];
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) v[nb] = acc[nb][i] * inv;
    stg128(op + 32 * j + 8 * i, pack8(v));
  }
}

// Folds the partials of every split request: one workgroup per (kv head,
// request), each thread owning 4 consecutive d of one of the G heads. The
// pieces are folded kFoldPieces at a time, every load of a group issued at
// once (a request of up to kFoldPieces pieces is one memory round trip
// after kv_indptr), with a log2-sum-exp reference point that is moved, and
// the folded sum rescaled, only when a group raises it. Requests reaching
// past the plan's token capacity get NaN rows and the CAPACITY status.
constexpr int kFoldPieces = 4;

__device__ __forceinline__ void merge_request(const DecodeArgs& a, int h, int r, int W) {
  const int rb = a.kv_indptr[r];
  const int re = a.kv_indptr[r + 1];
  const int G = a.group;
  const int qrow = a.q_indptr ? a.q_indptr[r] : r;
  if (static_cast<int64_t>(re) > static_cast<int64_t>(a.num_units) * W) {
    for (int e = threadIdx.x; e < G * (kD / 4); e += blockDim.x) {
      const int g = e / (kD / 4);
      const int d4 = (e - g * (kD / 4)) * 4;
      uint16_t* op = a.o + static_cast<int64_t>(qrow) * a.o_st +
                     static_cast<int64_t>(h * G + g) * a.o_sh + d4;
      *reinterpret_cast<u32x2_t*>(op) = u32x2_t{0x7fc07fc0u, 0x7fc07fc0u};  // bf16 NaN
    }
    if (threadIdx.x == 0) *a.status = SGL_ERR_CAPACITY;  // same value from every writer
    return;
  }
  if (re <= rb) return;
  const int u0 = rb / W;
  const int u1 = (re - 1) / W;
  if (u0 == u1) return;  // whole request, written by the decode kernel
  const int s0 = 2 * u0 + (rb > u0 * W ? 1 : 0);  // slot of the first piece
  const int np = u1 - u0 + 1;
  for (int e = threadIdx.x; e < G * (kD / 4); e += blockDim.x) {
    const int g = e / (kD / 4);
    const int d4 = (e - g * (kD / 4)) * 4;
    const int head = h * G + g;
    float m = -INFINITY;
    float den = 0.f;
    f32x4_t accm = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
    for (int c = 0; c < np; c += kFoldPieces) {
      float lse[kFoldPieces];
      f32x4_t v[kFoldPieces];
#pragma unroll
      for (int k = 0; k < kFoldPieces; ++k) {
        const int p = c + k;
        const int slot = p == 0 ? s0 : 2 * (u0 + min(p, np - 1));
        const int64_t pidx = static_cast<int64_t>(slot) * a.hq + head;
        lse[k] = a.part_lse[pidx];
        v[k] = *reinterpret_cast<const f32x4_t*>(a.part_o + pidx * kD + d4);
      }
      float mc = m;
#pragma unroll
      for (int k = 0; k < kFoldPieces; ++k)
        if (c + k < np) mc = fmaxf(mc, lse[k]);
      if (mc > m) {  // rescale what is folded so far to the new reference
        const float sc = m == -INFINITY ? 0.f : exp2f(m - mc);
        den *= sc;
        accm *= sc;
        m = mc;
      }
#pragma unroll
      for (int k = 0; k < kFoldPieces; ++k) {
        if (c + k >= np) break;
        const float wgt = lse[k] == -INFINITY ? 0.f : exp2f(lse[k] - m);
        den += wgt;
        accm += v[k] * wgt;
      }
    }
    const float inv = den > 0.f ? 1.0f / den : 0.f;
    uint16_t* op = a.o + static_cast<int64_t>(qrow) * a.o_st +
                   static_cast<int64_t>(head) * a.o_sh + d4;
    u32x2_t packed = {pack_bf16x2(accm[0] * inv, accm[1] * inv),
                      pack_bf16x2(accm[2] * inv, accm[3] * inv)};
    *reinterpret_cast<u32x2_t*>(op) = packed;
  }
}

// One workgroup per (kv head, request): every request's fold or NaN rows.
__global__ void __launch_bounds__(kMaxGroup * (kD / 4)) decode_merge_kernel(DecodeArgs a) {
  merge_request(a, blockIdx.x, blockIdx.y, unit_tokens(a, a.kv_indptr[a.batch]));
}

// One workgroup per (kv head, unit), for batches of more requests than
// units: the unit where a split request ends folds it (that request is the
// one running into the unit from before, recorded by the decode), and the
// extra row y = num_units writes the NaN rows of requests past the capacity.
__global__ void __launch_bounds__(kMaxGroup * (kD / 4)) decode_merge_units_kernel(DecodeArgs a) {
  const int h = blockIdx.x;
  const int u = blockIdx.y;
  const int total = a.kv_indptr[a.batch];
  const int W = unit_tokens(a, total);
  const int64_t cover = static_cast<int64_t>(a.num_units) * W;
  if (u == a.num_units) {
    if (total <= cover) return;
    int lo = 0, hi = a.batch;  // first request with kv_indptr[r + 1] > cover
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (a.kv_indptr[mid + 1] <= cover) lo = mid + 1; else hi = mid;
    }
    for (int r = lo; r < a.batch; ++r) merge_request(a, h, r, W);
    return;
  }
  const int r = a.unit_req[u];
  if (r < 0) return;
  const int re = a.kv_indptr[r + 1];
  if (static_cast<int64_t>(re) > cover || (re - 1) / W != u) return;
  merge_request(a, h, r, W);
}

}  // namespace
}  // namespace sgl

using namespace sgl;

// Compute units of device 0 (256 on MI355X); 256 when no device is visible,
// so the plan is also computable on a host without a GPU.
static int device_cu_count() {
  static int cached = 0;
  if (cached == 0) {
    int n = 0, dev = 0, cus = 0;
    if (hipGetDeviceCount(&n) == hipSuccess && n > 0 && hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        cus > 0)
      cached = cus;
    else
      cached = 256;
    (void)hipGetLastError();
  }
  return cached;
}

// ------------------------------------------------------------------ no-alloc variant
//
// Callers that cannot allocate (code under graph capture, tight serving
// loops) get the decode with its split workspace in a file-scope device
// array. Each GPU holds its own copy of the array for the life of the
// process; its device address is looked up once per device and used for
// every launch (the array's name is only a host-side stand-in). All calls on
// one GPU share the array: calls that overlap on one GPU (different streams
// without ordering) race on it.

namespace {
constexpr int64_t kScratchBytes = 32ll << 20;
constexpr int kMaxDevices = 64;
}  // namespace

static __device__ __align__(256) char scratch[kScratchBytes];

static void* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

// Device address of `scratch` on the current device, looked up once per
// device with that device current; nullptr with *status set on failure.
// sgl_decode_plan makes the lookup for the current device, so a caller that
// plans before a graph capture never runs it inside the capture.
static void* scratch_on_current_device(int* status) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    *status = static_cast<int>(e);
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    *status = SGL_ERR_UNSUPPORTED;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      *status = e != hipSuccess ? static_cast<int>(e) : SGL_ERR_INVALID_ARG;
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *status = SGL_OK;
  return g_scratch_ptr[dev];
}

// LDS of one fused decode + prefill workgroup (the CU's whole LDS).
constexpr size_t kMixedLds = 160 * 1024;

// Longest unit whose slot indices fit the fused launch's LDS next to the
// other units of its workgroup (8 / hkv units per 8-wave workgroup).
static int mixed_max_unit(int num_kv_heads) {
  const size_t per_unit = kMixedLds / (8 / num_kv_heads);
  const int64_t w = (static_cast<int64_t>(per_unit) -
                     static_cast<int64_t>(unit_lds_bytes<true>(num_kv_heads, 0))) /
                    static_cast<int64_t>(sizeof(int32_t)) / kStep * kStep;
  return static_cast<int>(w < kMaxChunkTokens ? w : kMaxChunkTokens);
}

// A plan whose units number about units_target (0: one unit per resident
// workgroup of the whole device) and hold at most max_unit tokens.
static int decode_plan_for(const int32_t* kv_indptr_host, int batch_size, int num_qo_heads,
                           int num_kv_heads, int head_dim, int64_t units_target, int max_unit,
                           sgl_decode_plan_t* plan) {
  if (!plan || !kv_indptr_host || batch_size < 0 || num_qo_heads <= 0 || num_kv_heads <= 0)
    return SGL_ERR_INVALID_ARG;
  if (num_qo_heads % num_kv_heads != 0) return SGL_ERR_INVALID_ARG;
  const int group = num_qo_heads / num_kv_heads;
  if (head_dim != kD || group > kMaxGroup || num_kv_heads > kMaxKvHeads)
    return SGL_ERR_UNSUPPORTED;
  if (kv_indptr_host[0] != 0) return SGL_ERR_INVALID_ARG;
  int64_t total = 0;
  for (int r = 0; r < batch_size; ++r) {
    const int len = kv_indptr_host[r + 1] - kv_indptr_host[r];
    if (len < 0) return SGL_ERR_INVALID_ARG;
    total += len;
  }
  if (total > 0x7fffffff) return SGL_ERR_UNSUPPORTED;
  // One work unit per resident workgroup (one wave per kv head), about 8
  // waves per CU: measured on MI355X (Qwen3 shapes, 32q/8kv and 32q/4kv,
  // short and 32K contexts), 8 concurrent row streams per CU beat 12 and 16
  // by 3-4% (more streams lose DRAM locality faster than they add latency
  // hiding), and 4 starve long contexts.
  int units_per_cu = 8 / num_kv_heads > 1 ? 8 / num_kv_heads : 1;
  if (units_target <= 0) units_target = static_cast<int64_t>(device_cu_count()) * units_per_cu;
  auto round16 = [](int64_t x) { return (x + kStep - 1) / kStep * kStep; };
  int64_t W = round16((total + units_target - 1) / units_target);
  if (W < kMinUnit) W = kMinUnit;
  if (W > max_unit) W = max_unit;
  const int64_t units = total > 0 ? (total + W - 1) / W : 1;
  if (units > 0x7fffffff / 2) return SGL_ERR_UNSUPPORTED;
  // The device picks w = clamp(round16(ceil(total / units)), W_min, W) <= W.
  int64_t w_dev = round16((total + units - 1) / units);
  if (w_dev < kMinUnit) w_dev = kMinUnit;
  if (w_dev > W) w_dev = W;
  int split = 0;
  for (int r = 0; r < batch_size && !split; ++r) {
    const int rb = kv_indptr_host[r], re = kv_indptr_host[r + 1];
    if (re > rb && (re - 1) / w_dev != rb / w_dev) split = 1;
  }
  plan->kv_chunk_size = static_cast<int32_t>(W);
  plan->min_chunk_size = kMinUnit;
  plan->num_units = static_cast<int32_t>(units);
  plan->split_kv = split;
  plan->batch_size = batch_size;
  plan->num_qo_heads = num_qo_heads;
  plan->num_kv_heads = num_kv_heads;
  plan->head_dim = head_dim;
  plan->max_total_tokens = units * W;
  plan->workspace_bytes = workspace_layout(static_cast<int>(units), num_qo_heads).total;
  return SGL_OK;
}

extern "C" int sgl_decode_plan(const int32_t* kv_indptr_host, int batch_size, int num_qo_heads,
                               int num_kv_heads, int head_dim, sgl_decode_plan_t* plan) {
  const int st = decode_plan_for(kv_indptr_host, batch_size, num_qo_heads, num_kv_heads,
                                 head_dim, 0, kMaxChunkTokens, plan);
  // Resolve the no-alloc scratch address of the current device now (host
  // code, before any capture the caller may begin); without a visible
  // device the lookup is left to the first no-alloc call.
  int n = 0;
  if (st == SGL_OK && hipGetDeviceCount(&n) == hipSuccess && n > 0) {
    int ignored = 0;
    (void)scratch_on_current_device(&ignored);
  }
  (void)hipGetLastError();
  return st;
}

extern "C" int sgl_decode_plan_cus(const int32_t* kv_indptr_host, int batch_size,
                                   int num_qo_heads, int num_kv_heads, int head_dim,
                                   int decode_cus, sgl_decode_plan_t* plan) {
  if (num_kv_heads <= 0 || num_kv_heads > 8 || 8 % num_kv_heads != 0) return SGL_ERR_UNSUPPORTED;
  if (decode_cus <= 0) return SGL_ERR_INVALID_ARG;
  return decode_plan_for(kv_indptr_host, batch_size, num_qo_heads, num_kv_heads, head_dim,
                         static_cast<int64_t>(decode_cus) * (8 / num_kv_heads),
                         mixed_max_unit(num_kv_heads), plan);
}

// Per-CU rates behind the split, measured on MI355X at config 5's shapes
// (32q/4kv, d128): the decode streams about 37.5 GB/s of K/V per CU when it
// has only part of the device (it needs ~170 CUs to reach HBM bandwidth),
// and the causal prefill computes about 3.9 TFLOP/s per CU.
constexpr double kDecodeBytesPerCu = 37.5e9;
constexpr double kPrefillFlopsPerCu = 3.9e12;

extern "C" int sgl_mixed_decode_cus(int64_t decode_kv_tokens, int num_kv_heads, int head_dim,
                                    double prefill_flops) {
  const int cus = device_cu_count();
  if (decode_kv_tokens <= 0 || num_kv_heads <= 0 || head_dim <= 0) return 8;
  if (!(prefill_flops > 0.0)) return cus;
  const double dec = static_cast<double>(decode_kv_tokens) * num_kv_heads * head_dim * 4.0 /
                     kDecodeBytesPerCu;
  const double pre = prefill_flops / kPrefillFlopsPerCu;
  // The decode's share of the CU-time, leaning 5% towards the decode: the
  // prefill absorbs imbalance better (its items fill freed CUs heavy-first).
  int h = static_cast<int>(cus * dec / (dec + pre) * 1.05 / 8.0 + 0.5) * 8;
  if (h < 8) h = 8;
  if (h > cus) h = cus;
  return h;
}

extern "C" int sgl_decode_plan_check(const sgl_decode_plan_t* plan,
                                     const int32_t* kv_indptr_host, int batch_size) {
  if (!plan || !kv_indptr_host || batch_size < 0) return SGL_ERR_INVALID_ARG;
  if (batch_size > plan->batch_size) return SGL_ERR_CAPACITY;
  if (kv_indptr_host[0] != 0) return SGL_ERR_INVALID_ARG;
  for (int r = 0; r < batch_size; ++r)
    if (kv_indptr_host[r + 1] < kv_indptr_host[r]) return SGL_ERR_INVALID_ARG;
  if (static_cast<int64_t>(kv_indptr_host[batch_size]) > plan->max_total_tokens)
    return SGL_ERR_CAPACITY;
  return SGL_OK;
}

extern "C" int sgl_decode_status(const void* workspace, int32_t* status, void* stream) {
  if (!status) return SGL_ERR_INVALID_ARG;
  if (!workspace) {  // the no-alloc entry point's scratch on the current device
    int st = SGL_OK;
    workspace = scratch_on_current_device(&st);
    if (!workspace) return st;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = hipMemcpyAsync(status, workspace, sizeof(int32_t), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  return e == hipSuccess ? SGL_OK : static_cast<int>(e);
}

namespace {

// Checks shared by the decode entry points; fills the kernel arguments
// except the workspace pointers.
int decode_args(const sgl_decode_plan_t* plan, const void* q, int64_t q_stride_token,
                int64_t q_stride_head, const void* k_cache, const void* v_cache,
                int64_t kv_stride_slot, int64_t kv_stride_head, const int32_t* indices,
                const int32_t* kv_indptr, const int32_t* q_indptr, int batch_size,
                int num_qo_heads, int num_kv_heads, int head_dim, float sm_scale, void* o,
                int64_t o_stride_token, int64_t o_stride_head, DecodeArgs& a) {
  if (!plan || batch_size < 0 || num_qo_heads <= 0 || num_kv_heads <= 0)
    return SGL_ERR_INVALID_ARG;
  if (!q || !k_cache || !v_cache || !indices || !kv_indptr || !o) return SGL_ERR_INVALID_ARG;
  if (num_qo_heads % num_kv_heads != 0) return SGL_ERR_INVALID_ARG;
  const int group = num_qo_heads / num_kv_heads;
  if (head_dim != kD || group > kMaxGroup || num_kv_heads > kMaxKvHeads) return SGL_ERR_UNSUPPORTED;
  if (plan->kv_chunk_size <= 0 || plan->kv_chunk_size % kStep != 0 ||
      plan->min_chunk_size <= 0 || plan->min_chunk_size > plan->kv_chunk_size ||
      plan->kv_chunk_size > kMaxChunkTokens || plan->num_units <= 0 ||
      plan->num_units > 0x7fffffff / 2 ||
      plan->max_total_tokens != static_cast<int64_t>(plan->num_units) * plan->kv_chunk_size ||
      plan->workspace_bytes != workspace_layout(plan->num_units, plan->num_qo_heads).total)
    return SGL_ERR_INVALID_ARG;
  if (batch_size > plan->batch_size || num_qo_heads != plan->num_qo_heads ||
      num_kv_heads != plan->num_kv_heads)
    return SGL_ERR_CAPACITY;
  // Row addresses use 32-bit slot byte strides.
  if (kv_stride_slot <= 0 || kv_stride_slot > 0x7fffffff) return SGL_ERR_UNSUPPORTED;
  // Output rows are written with 16-byte stores (whole requests).
  if (q_stride_head % 8 || q_stride_token % 8 || kv_stride_slot % 8 || kv_stride_head % 8 ||
      o_stride_token % 8 || o_stride_head % 8 || !aligned16(q) || !aligned16(k_cache) ||
      !aligned16(v_cache) || !aligned16(o))
    return SGL_ERR_ALIGNMENT;
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
  a.chunk_min = plan->min_chunk_size;
  a.batch = batch_size;
  a.num_units = plan->num_units;
  a.out_bytes = 0;
  return SGL_OK;
}

// Merge workgroup size: one thread per 4 d of each of the G heads, in whole waves.
int merge_threads(int group) { return (group * (kD / 4) + kWave - 1) / kWave * kWave; }

// The merge launch: per request, or per unit when the batch has more
// requests than the plan has units (fewer workgroups that only exit).
void launch_merge(const DecodeArgs& a, hipStream_t s) {
  if (a.batch > a.num_units + 1)
    hipLaunchKernelGGL(decode_merge_units_kernel, dim3(a.hkv, a.num_units + 1),
                       dim3(merge_threads(a.group)), 0, s, a);
  else
    hipLaunchKernelGGL(decode_merge_kernel, dim3(a.hkv, a.batch), dim3(merge_threads(a.group)), 0,
                       s, a);
}

// Points the kernel arguments at a workspace of the plan's layout.
void bind_workspace(DecodeArgs& a, const sgl_decode_plan_t* plan, void* workspace) {
  const WorkspaceLayout w = workspace_layout(plan->num_units, plan->num_qo_heads);
  char* base = static_cast<char*>(workspace);
  a.status = reinterpret_cast<int32_t*>(base);
  a.part_o = reinterpret_cast<float*>(base + w.part_o_off);
  a.part_lse = reinterpret_cast<float*>(base + w.part_lse_off);
  a.unit_req = reinterpret_cast<int32_t*>(base + w.unit_req_off);
}

// Decode launch + merge launch on one stream (or the small-batch kernel alone).
int launch_decode(const DecodeArgs& a, const sgl_decode_plan_t* plan, hipStream_t s) {
  if (plan->kv_chunk_size <= kMinUnit &&
      static_cast<int64_t>(a.batch) * a.hkv <= static_cast<int64_t>(device_cu_count())) {
    hipLaunchKernelGGL(paged_decode_small_kernel, dim3(a.hkv, a.batch), dim3(kSmallWaves * kWave),
                       0, s, a);
    return launch_status();
  }
  const dim3 grid(plan->num_units);
  const dim3 block(a.hkv * kWave);
  // Output rings in what LDS the plan's units per CU leave free (at least
  // one partial record per wave, else the pieces are written directly).
  DecodeArgs da = a;
  const int upc = a.hkv < 8 ? 8 / a.hkv : 1;
  const size_t off = out_ring_offset(a.hkv, plan->kv_chunk_size);
  const size_t budget = 160 * 1024 / upc;
  size_t ring = budget > off ? (budget - off) / a.hkv / 16 * 16 : 0;
  if (ring > kMaxOutRing) ring = kMaxOutRing;
  da.out_bytes = ring >= static_cast<size_t>(out_record_bytes(a.group, false)) ? static_cast<int>(ring) : 0;
  const size_t lds = da.out_bytes > 0 ? off + static_cast<size_t>(a.hkv) * da.out_bytes
                                      : unit_lds_bytes<false>(a.hkv, plan->kv_chunk_size);
  hipLaunchKernelGGL(paged_decode_kernel, grid, block, lds, s, da);
  int st = launch_status();
  if (st != SGL_OK) return st;
  // Always launched: besides folding split requests it is what reports a
  // batch that exceeds the plan.
  launch_merge(a, s);
  return launch_status();
}

}  // namespace

extern "C" int sgl_paged_decode(const sgl_decode_plan_t* plan, const void* q,
                                int64_t q_stride_token, int64_t q_stride_head,
                                const void* k_cache, const void* v_cache, int64_t kv_stride_slot,
                                int64_t kv_stride_head, const int32_t* indices,
                                const int32_t* kv_indptr, const int32_t* q_indptr,
                                int batch_size, int num_qo_heads, int num_kv_heads, int head_dim,
                                float sm_scale, void* o, int64_t o_stride_token,
                                int64_t o_stride_head, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  if (!plan || batch_size < 0) return SGL_ERR_INVALID_ARG;
  if (batch_size == 0) return SGL_OK;
  DecodeArgs a;
  int st = decode_args(plan, q, q_stride_token, q_stride_head, k_cache, v_cache, kv_stride_slot,
                       kv_stride_head, indices, kv_indptr, q_indptr, batch_size, num_qo_heads,
                       num_kv_heads, head_dim, sm_scale, o, o_stride_token, o_stride_head, a);
  if (st != SGL_OK) return st;
  if (workspace == nullptr || workspace_bytes < plan->workspace_bytes) return SGL_ERR_CAPACITY;
  if (!aligned16(workspace)) return SGL_ERR_ALIGNMENT;
  bind_workspace(a, plan, workspace);
  return launch_decode(a, plan, static_cast<hipStream_t>(stream));
}

extern "C" int sgl_paged_mixed(const sgl_decode_plan_t* plan, const void* q,
                               int64_t q_stride_token, int64_t q_stride_head,
                               const void* k_cache, const void* v_cache, int64_t kv_stride_slot,
                               int64_t kv_stride_head, const int32_t* dec_indices,
                               const int32_t* dec_kv_indptr, const int32_t* dec_q_rows,
                               int dec_batch, const int32_t* pre_indices,
                               const int32_t* pre_qo_indptr, const int32_t* pre_kv_indptr,
                               const int32_t* pre_q_start, int pre_batch, int pre_max_qo_len,
                               int num_qo_heads, int num_kv_heads, int head_dim, float sm_scale,
                               void* o, int64_t o_stride_token, int64_t o_stride_head,
                               void* workspace, int64_t workspace_bytes, void* stream) {
  if (!plan || dec_batch < 0 || pre_batch < 0 || pre_max_qo_len < 0) return SGL_ERR_INVALID_ARG;
  if (num_kv_heads <= 0 || num_kv_heads > 8 || 8 % num_kv_heads != 0) return SGL_ERR_UNSUPPORTED;
  const bool has_pre = pre_batch > 0 && pre_max_qo_len > 0;
  // A plan with longer units than the fused launch's LDS holds (one from
  // sgl_decode_plan at 1 or 2 kv heads) runs as the two entry points.
  const bool fits = plan->kv_chunk_size > 0 && plan->kv_chunk_size <= mixed_max_unit(num_kv_heads);
  if (dec_batch == 0 || !has_pre || !fits) {
    int st = SGL_OK;
    if (dec_batch > 0)
      st = sgl_paged_decode(plan, q, q_stride_token, q_stride_head, k_cache, v_cache,
                            kv_stride_slot, kv_stride_head, dec_indices, dec_kv_indptr,
                            dec_q_rows, dec_batch, num_qo_heads, num_kv_heads, head_dim, sm_scale,
                            o, o_stride_token, o_stride_head, workspace, workspace_bytes, stream);
    if (st == SGL_OK && has_pre)
      st = sgl_paged_prefill(q, q_stride_token, q_stride_head, k_cache, v_cache, kv_stride_slot,
                             kv_stride_head, pre_indices, pre_qo_indptr, pre_kv_indptr,
                             pre_q_start, pre_batch, pre_max_qo_len, num_qo_heads, num_kv_heads,
                             head_dim, sm_scale, o, o_stride_token, o_stride_head, stream);
    return st;
  }
  DecodeArgs d;
  int st = decode_args(plan, q, q_stride_token, q_stride_head, k_cache, v_cache, kv_stride_slot,
                       kv_stride_head, dec_indices, dec_kv_indptr, dec_q_rows, dec_batch,
                       num_qo_heads, num_kv_heads, head_dim, sm_scale, o, o_stride_token,
                       o_stride_head, d);
  if (st != SGL_OK) return st;
  if (workspace == nullptr || workspace_bytes < plan->workspace_bytes) return SGL_ERR_CAPACITY;
  if (!aligned16(workspace)) return SGL_ERR_ALIGNMENT;
  bind_workspace(d, plan, workspace);
  pf::PrefillArgs p;
  st = pf::prefill_args(q, q_stride_token, q_stride_head, k_cache, v_cache, kv_stride_slot,
                        kv_stride_head, pre_indices, pre_qo_indptr, pre_kv_indptr, pre_q_start,
                        num_qo_heads, num_kv_heads, head_dim, sm_scale, o, o_stride_token,
                        o_stride_head, p);
  if (st != SGL_OK) return st;
  // The prefill role: 8-wave items of 256 packed rows (unpaired, heavy first).
  const int64_t rows_max = static_cast<int64_t>(pre_max_qo_len) * p.group;
  const int64_t tiles = (rows_max + 255) / 256;
  const int64_t items = tiles * num_kv_heads * pre_batch;
  const int upw = 8 / num_kv_heads;
  // Decode workgroups rounded to a multiple of the 8 XCDs, so the prefill
  // items keep their XCD-aware placement.
  const int64_t dec_blocks = ((plan->num_units + upw - 1) / upw + 7) / 8 * 8;
  if (items + dec_blocks > 0x7fffffff) return SGL_ERR_INVALID_ARG;
  p.tiles_per_req = static_cast<int>(tiles);
  size_t lds = static_cast<size_t>(upw) * unit_lds_bytes<true>(num_kv_heads, plan->kv_chunk_size);
  if (lds < static_cast<size_t>(pf::prefill_lds_bytes<8, 1>()))
    lds = pf::prefill_lds_bytes<8, 1>();
  if (lds > kMixedLds) return SGL_ERR_INVALID_ARG;  // excluded by `fits`
  const dim3 grid(static_cast<uint32_t>(dec_blocks + items));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int db = static_cast<int>(dec_blocks);
  switch (upw) {
    case 1: hipLaunchKernelGGL(mixed_attention_kernel<1>, grid, dim3(512), lds, s, d, p, db); break;
    case 2: hipLaunchKernelGGL(mixed_attention_kernel<2>, grid, dim3(512), lds, s, d, p, db); break;
    case 4: hipLaunchKernelGGL(mixed_attention_kernel<4>, grid, dim3(512), lds, s, d, p, db); break;
    default: hipLaunchKernelGGL(mixed_attention_kernel<8>, grid, dim3(512), lds, s, d, p, db); break;
  }
  st = launch_status();
  if (st != SGL_OK) return st;
  launch_merge(d, s);
  return launch_status();
}

extern "C" int sgl_paged_decode_noalloc(const sgl_decode_plan_t* plan, const void* q,
                                        int64_t q_stride_token, int64_t q_stride_head,
                                        const void* k_cache, const void* v_cache,
                                        int64_t kv_stride_slot, int64_t kv_stride_head,
                                        const int32_t* indices, const int32_t* kv_indptr,
                                        const int32_t* q_indptr, int batch_size,
                                        int num_qo_heads, int num_kv_heads, int head_dim,
                                        float sm_scale, void* o, int64_t o_stride_token,
                                        int64_t o_stride_head, void* stream) {
  if (!plan || batch_size < 0) return SGL_ERR_INVALID_ARG;
  if (batch_size == 0) return SGL_OK;
  DecodeArgs a;
  int st = decode_args(plan, q, q_stride_token, q_stride_head, k_cache, v_cache, kv_stride_slot,
                       kv_stride_head, indices, kv_indptr, q_indptr, batch_size, num_qo_heads,
                       num_kv_heads, head_dim, sm_scale, o, o_stride_token, o_stride_head, a);
  if (st != SGL_OK) return st;
  if (plan->workspace_bytes > kScratchBytes) return SGL_ERR_CAPACITY;
  void* ws = scratch_on_current_device(&st);
  if (!ws) return st;
  bind_workspace(a, plan, ws);
  return launch_decode(a, plan, static_cast<hipStream_t>(stream));
}
