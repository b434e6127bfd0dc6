// Paged causal prefill: the device code shared by the standalone prefill
// launch (prefill.hip) and the fused decode + prefill launch (mixed.hip).
#pragma once

#include <math.h>

#include <type_traits>

#include "common.h"

namespace sgl {
namespace pf {
namespace {

constexpr int kD = 128;
constexpr int kBN = 64;    // kv tokens per LDS tile
constexpr int kXcds = 8;  // MI355X: 8 XCDs, each with its own L2
constexpr float kRescaleSlack = 8.f;  // log2 units: p <= 256 between rescales
constexpr int kKAhead = 4;            // K operand reads in flight ahead of their MFMA (6 measured the same)

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
  int tiles_per_req;  // query tiles per (request, kv head)
  int num_kv_heads;
};

// LDS reads of the tile loop are inline asm with compile-time offsets, and
// their waits are explicit: the compiler's wait insertion cannot tell the
// tile being read from the tile whose gather is in flight and would stall
// every read on that gather, and hand-placed waits let each read run several
// instructions ahead of its use. LDS operations complete in order, so
// lgkmcnt(N) after a read means "this read and all older ones are done" once
// at most N younger LGKM operations are outstanding.

// Byte address of a generic pointer into LDS.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)(p)));
}

template <int OFF>
__device__ __forceinline__ u32x4_t lds_read_b128(uint32_t addr) {
  u32x4_t v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}

template <int OFF>
__device__ __forceinline__ void lds_write_b128(uint32_t addr, const u32x4_t& v) {
  asm volatile("ds_write_b128 %0, %1 offset:%2" : : "v"(addr), "v"(v), "i"(OFF));
}

// ds_read_b64_tr_b16: within each group of 16 lanes, lane i receives element
// i % 4 of the 4-element (8-byte) pieces addressed by lanes 4 e + i / 4,
// e < 4 -- a 4 x 16 -> 16 x 4 transpose of 16-bit data.
template <int OFF>
__device__ __forceinline__ u32x2_t lds_read_tr16(uint32_t addr) {
  u32x2_t v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}

// lgkmcnt(N), tied to the value it guards so no use is scheduled above it.
template <int N, typename T>
__device__ __forceinline__ void lgkm_wait(T& v) {
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(v) : "i"(N));
}

template <int N>
__device__ __forceinline__ void lgkm_wait8(u32x2_t (&v)[8]) {
  asm volatile("s_waitcnt lgkmcnt(%8)"
               : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]),
                 "+v"(v[6]), "+v"(v[7])
               : "i"(N));
}

__device__ __forceinline__ bf16x8_t as_bf16x8(const u32x4_t& v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

// K/V tiles live in LDS as 64 rows of 256 bytes with no padding; row r's
// logical 16-byte chunk c sits at physical chunk c ^ swz(r). swz takes every
// value 0..15 over 16 consecutive rows (conflict-free ds_read_b128 of 16
// rows' same chunk) and gives the 4 rows of an aligned quad distinct upper
// bits (conflict-free transpose reads of 4 rows x 64 bytes).
__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

struct Tile {
  uint16_t k[kBN * kD];
  uint16_t v[kBN * kD];
};

// Slot indices of one 64-token tile for this thread's rows: with W waves
// gathering a tile, a wave instruction covers 4 rows, so thread (wave, lane)
// of the gathering group takes rows 4 W u + 4 wave + lane / 16, u < 16 / W,
// i.e. (tid + 64 W u) / 16 with tid = 64 wave + lane.
template <int W>
__device__ __forceinline__ void load_slots(const int32_t* idx, int tile0, int kv_len, int tid,
                                           int32_t (&sl)[16 / W]) {
#pragma unroll
  for (int u = 0; u < 16 / W; ++u) {
    const int tok = (tid + 64 * W * u) >> 4;
    sl[u] = idx[min(tile0 + tok, kv_len - 1)];
  }
}

// Gathers one K (or V) tile straight into LDS (global_load_lds_dwordx4:
// lane i of a wave writes LDS bytes [16 i, 16 i + 16) after the wave's
// base), so the prefetch holds no registers. Lane i takes physical chunk
// i % 16 of its row and therefore loads logical chunk (i % 16) ^ swz(row);
// row % 16 = 4 W u + 4 wave + i / 16 (mod 16) takes one value for every u
// when 4 | W and two (u even, u odd) when W = 2, so lane_base[0 or 1] (the
// head's row 0 plus that chunk) is fixed per u parity and each address is
// one 32 x 32 -> 64-bit multiply-add of the slot.
template <int W>
__device__ __forceinline__ void issue_half(const char* const (&lane_base)[2], uint32_t ss_bytes,
                                           const int32_t (&sl)[16 / W], uint16_t* dst, int wave) {
#pragma unroll
  for (int u = 0; u < 16 / W; ++u) {
    const int lds_row = 4 * W * u + 4 * wave;  // wave-uniform destination base
    __builtin_amdgcn_global_load_lds(
        lane_base[W == 2 ? (u & 1) : 0] +
            static_cast<uint64_t>(static_cast<uint32_t>(sl[u])) * ss_bytes,
        (__attribute__((address_space(3))) void*)(dst + lds_row * kD), 16, 0, 0);
  }
}

// Waits until this wave's LDS gathers have landed (vmcnt(0); expcnt and
// lgkmcnt left at their maxima).
__device__ __forceinline__ void wait_gathers() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Waits until at most N of this wave's vector memory operations are
// outstanding (they complete in issue order, so every older one is done).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt(((N >> 4) << 14) | 0x0F70 | (N & 15));
}

struct RowState {
  f32x16_t acc[4];  // O^T: acc[db][4 g + i] holds d = 32 db + 8 g + 4 hl + i
  float m, l;
};

// Per-lane LDS byte addresses of the tile loop (tile buffer 0; buffer 1 and
// the unrolled positions are compile-time offsets).
struct LaneAddr {
  uint32_t k[8];  // K row c, logical chunk 2 s + hl, s < 8 (+ 32 rows: +8192)
  uint32_t v[8];  // V transpose-read source for [2 db + hi] at ks4 = 0 (+ 4096 per ks4)
};

constexpr int kTileBytes = 2 * kBN * kD * 2;  // one K + V buffer (32 KiB)
constexpr int kVOffset = kBN * kD * 2;       // V after K in a buffer
static_assert(sizeof(Tile) == kTileBytes, "tile buffers are addressed by fixed offsets");

// S^T = K Q^T for one 64-token tile from LDS buffer BUF: tokens
// [32 mb, 32 mb + 32) in st[mb]. MFMA i uses mb = i % 2, s = i / 2 (the two
// accumulation chains alternate); its K operand is read four MFMAs ahead.
template <int BUF, int I>
__device__ __forceinline__ void k_read(const LaneAddr& la, u32x4_t (&kb)[16]) {
  kb[I] = lds_read_b128<BUF * kTileBytes + (I & 1) * 32 * kD * 2>(la.k[I >> 1]);
}

// The first four K operand reads of S = K Q^T on buffer BUF, issued ahead of
// qk_tile_run (the caller's work in between hides their latency).
template <int BUF>
__device__ __forceinline__ void qk_tile_prefetch(const LaneAddr& la, u32x4_t (&kb)[16]) {
  static_for<0, kKAhead>([&](auto I) { k_read<BUF, decltype(I)::value>(la, kb); });
}

template <int BUF>
__device__ __forceinline__ void qk_tile_run(const LaneAddr& la, const bf16x8_t (&qop)[8],
                                            f32x16_t (&st)[2], u32x4_t (&kb)[16]) {
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int v = 0; v < 16; ++v) st[mb][v] = 0.f;
  auto kread = [&](auto I) { k_read<BUF, decltype(I)::value>(la, kb); };
  static_for<0, 16>([&](auto I) {
    constexpr int i = decltype(I)::value;
    constexpr int younger = (15 - i) < kKAhead - 1 ? (15 - i) : kKAhead - 1;
    lgkm_wait<younger>(kb[i]);
    st[i & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(kb[i]), qop[i >> 1], st[i & 1],
                                                        0, 0, 0);
    if constexpr (i + kKAhead < 16) kread(std::integral_constant<int, i + kKAhead>{});
  });
}

template <int BUF>
__device__ __forceinline__ void qk_tile(const LaneAddr& la, const bf16x8_t (&qop)[8],
                                        f32x16_t (&st)[2]) {
  u32x4_t kb[16];
  qk_tile_prefetch<BUF>(la, kb);
  qk_tile_run<BUF>(la, qop, st, kb);
}

// Mask, running max and (lazy) rescale of the scores of the tile at tile0.
__device__ __forceinline__ void softmax_head(const PrefillArgs& a, f32x16_t (&st)[2],
                                             RowState& rs, int tile0, int first_masked,
                                             int allow, int kv_len, int hl) {
  // Causal / length mask, only on tiles that reach past a row's last visible
  // token (a wave-uniform test, so full tiles skip it entirely).
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
  mt = max_xor32(mt) * a.scale_log2;
  // Lazy rescaling: the reference point m (log2 domain) only moves when a
  // row's max exceeds it by more than kRescaleSlack, so most tiles skip the O
  // rescale. Exact: every p and l use the same m; p <= 2^kRescaleSlack.
  const bool move = mt > rs.m + kRescaleSlack;
  if (__builtin_amdgcn_ballot_w64(move) != 0) {
    const float mn = move ? mt : rs.m;
    const float alpha = __builtin_amdgcn_exp2f(rs.m - mn);  // 0 on the first tile
    rs.l *= alpha;
    rs.m = mn;
#pragma unroll
    for (int db = 0; db < 4; ++db) rs.acc[db] *= alpha;
  }
}

// p = 2^(s scale - m) for the 32 scores of half mb (tokens [32 mb, 32 mb +
// 32)), their sum into rs.l, packed to the bf16 P^T operands of k-steps
// 2 mb and 2 mb + 1. P^T slots 0-3 <-> tokens 16 ks4 + 4 hl + (0..3), slots
// 4-7 <-> the same + 8 (the S^T accumulator order).
template <int MB>
__device__ __forceinline__ void softmax_exp_half(const PrefillArgs& a, f32x16_t (&st)[2],
                                                 RowState& rs, bf16x8_t (&pop)[4]) {
  const float neg_m = rs.m == -INFINITY ? 0.f : -rs.m;  // nothing visible yet
  float ps = 0.f;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    // v_exp_f32 directly: arguments are <= kRescaleSlack, and results below
    // 2^-126 flush to zero, which a bf16 weight could not hold anyway.
    const float p = __builtin_amdgcn_exp2f(fmaf(st[MB][v], a.scale_log2, neg_m));
    st[MB][v] = p;
    ps += p;
  }
  rs.l += ps;
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    u32x4_t pw;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      pw[k] = pack_bf16x2(st[MB][ks * 8 + 2 * k], st[MB][ks * 8 + 2 * k + 1]);
    pop[2 * MB + ks] = as_bf16x8(pw);
  }
}

// O^T += V^T P^T over k-steps [K0, K1) of the tile in LDS buffer BUF. V^T
// comes from the row-major tile by transpose reads, one k-step ahead of its
// MFMAs; the reads of k-step K0 are issued by the caller (pv_reads).
template <int BUF, int KS>
__device__ __forceinline__ void pv_reads(const LaneAddr& la, u32x2_t (&vr)[8]) {
  static_for<0, 8>([&](auto J) {
    constexpr int j = decltype(J)::value;
    vr[j] = lds_read_tr16<BUF * kTileBytes + KS * 16 * kD * 2>(la.v[j]);
  });
}

template <int BUF, int K0, int K1>
__device__ __forceinline__ void pv_steps(const LaneAddr& la, const bf16x8_t (&pop)[4],
                                         u32x2_t (&vr)[4][8], RowState& rs) {
  static_for<K0, K1>([&](auto K) {
    constexpr int ks4 = decltype(K)::value;
    if constexpr (ks4 + 1 < 4) pv_reads<BUF, ks4 + 1>(la, vr[ks4 + 1]);
    lgkm_wait8<(ks4 + 1 < 4 ? 8 : 0)>(vr[ks4]);
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const u32x4_t w = {vr[ks4][2 * db][0], vr[ks4][2 * db][1], vr[ks4][2 * db + 1][0],
                         vr[ks4][2 * db + 1][1]};
      rs.acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(w), pop[ks4], rs.acc[db], 0, 0, 0);
    }
  });
}

// W waves per workgroup, 32 packed query rows each: 4 waves and two
// workgroups per CU, or 8 waves (256 rows sharing each K/V tile, half the
// gather traffic per row) and one workgroup per CU, where waves w and w + 4
// share SIMD w % 4.
//
// Work item w = (request, kv head, query-tile position), head-major. The
// rows of a request form query tiles (G heads of each token packed
// row-wise), and tile i sees about (prefix + i) kv tiles. Workgroups are
// dealt to the 8 XCDs round-robin by linear id, so when the count allows,
// XCD x takes the contiguous share [x S, (x + 1) S), S = N / 8: the tiles of
// one kv head stay on one or two XCDs, whose L2 then holds that head's K/V.
//
// kPair = false: one 32 W-row tile per item. Positions alternate between the
// heavy and the light end (T-1, 0, T-2, 1, ...), so every share carries about
// the same work; inside a share the heavy half is dispatched first, heaviest
// first, then the light half, heaviest first. Suits launches of several
// workgroups per CU, which the dispatcher balances.
//
// kPair = true (W = 8, at most one workgroup per CU): item p takes the
// 16 W-row tiles T - 1 - p (waves 0-3) and p (waves 4-7), so every item
// carries the same work and each SIMD holds one heavy and one light wave.
// Both groups share each gathered K/V tile; a group whose rows can no
// longer see the current tile skips its compute for that step.
//
// KS = 2 (W = 4, for launches that would leave CUs idle): each item is a
// 32 GW-row tile (GW = W / KS = 2 waves) and the workgroup holds KS groups of
// GW waves on the same rows, group g taking the g-th share of the item's kv
// tiles through its own LDS ring; twice the items of a 4-wave launch with
// half the kv tiles each, so small launches reach every CU. The other
// groups' softmax states are folded into group 0's through LDS at the end.
// The work of item `lin` of `n_items` (the kernel's block index and grid
// size, or an offset range of a fused launch), with the workgroup's LDS at
// lds_raw (prefill_lds_bytes<W, KS>() bytes, 16-byte aligned).
// LDS of one group's tiles: two K/V buffers, or with KS = 2 a third K
// buffer after them (the short-share schedule below).
template <int KS>
constexpr int group_lds_bytes() {
  return KS == 2 ? 2 * kTileBytes + kTileBytes / 2 : 2 * kTileBytes;
}

template <int W, int KS>
constexpr int prefill_lds_bytes() {
  constexpr int ring = KS * group_lds_bytes<KS>();
  constexpr int xch = (KS - 1) * 66 * 64 * (W / KS) * 4;
  return ring > xch ? ring : xch;
}

template <int W, bool kPair, int KS>
__device__ __forceinline__ void prefill_item(PrefillArgs a, char* lds_raw, int lin,
                                             int n_items) {
  static_assert(!kPair || (W == 8 && KS == 1),
                "pairing splits 8 waves into two SIMD-sharing groups");
  constexpr int GW = W / KS;  // waves per group (gathering a group's tiles)
  static_assert(GW * KS == W && (GW == 2 || GW == 4 || GW == 8),
                "gather lane bases need row % 16 to take at most two values per lane");
  constexpr int kGM = kPair ? 16 * W : 32 * GW;  // rows per group tile
  int w = lin;
  if (kPair) {
    if (n_items % kXcds == 0) w = (lin % kXcds) * (n_items / kXcds) + lin / kXcds;
  } else if (n_items % (2 * kXcds) == 0) {
    const int share = n_items / kXcds;
    const int j = lin / kXcds;
    w = (lin % kXcds) * share + (j < share / 2 ? 2 * j : 2 * (share - 1 - j) + 1);
  }
  const int per_req = a.tiles_per_req * a.num_kv_heads;
  const int r = w / per_req;
  const int h = (w - r * per_req) / a.tiles_per_req;
  const int pos = w - r * per_req - h * a.tiles_per_req;
  const int qo_len = a.qo_indptr[r + 1] - a.qo_indptr[r];
  const int qo_beg = a.q_start ? a.q_start[r] : a.qo_indptr[r];
  const int kv_beg = a.kv_indptr[r];
  const int kv_len = a.kv_indptr[r + 1] - kv_beg;
  const int G = a.group;
  const int rows = qo_len * G;
  if (kv_len <= 0) {
    // No visible token: zero output rows, as the decode path writes for an
    // empty request. The item at position 0 of each (request, kv head)
    // writes the G heads of that kv head for every query token.
    if (pos == 0)
      for (int e = threadIdx.x; e < rows * (kD / 8); e += blockDim.x) {
        const int prow = e / (kD / 8);
        const int tok = prow / G;
        const int head = h * G + (prow - tok * G);
        stg128(a.o + static_cast<int64_t>(qo_beg + tok) * a.o_st +
                   static_cast<int64_t>(head) * a.o_sh + (e - prow * (kD / 8)) * 8,
               u32x4_t{0, 0, 0, 0});
      }
    return;
  }
  const int lane = threadIdx.x & 63;
  const int wave_all = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int split = KS == 1 ? 0 : wave_all / GW;  // kv share of this wave's group
  const int wave = KS == 1 ? wave_all : wave_all - split * GW;
  const int tid = threadIdx.x - split * 64 * GW;  // thread index inside the group
  const int c = lane & 31;
  const int hl = lane >> 5;
  // Tile of group 0 (the whole workgroup without pairing) and this wave's
  // group, its rows and its position in the group.
  int tile0, row0, gwave;
  bool grp_rows;
  if (kPair) {
    const int T = (rows + kGM - 1) / kGM;
    tile0 = T - 1 - pos;
    if (tile0 < pos) return;  // past this request's pairs
    const int grp = wave / (W / 2);
    grp_rows = grp == 0 || pos < tile0;  // group 1 is empty on the middle tile of an odd T
    row0 = (grp == 0 ? tile0 : pos) * kGM;
    gwave = wave % (W / 2);
  } else {
    tile0 = (pos & 1) ? (pos >> 1) : a.tiles_per_req - 1 - (pos >> 1);
    if (tile0 * kGM >= rows) return;
    grp_rows = true;
    row0 = tile0 * kGM;
    gwave = wave;
  }
  const int off = kv_len - qo_len;  // causal offset (cached prefix length)

  // This lane's query row.
  const int prow = row0 + gwave * 32 + c;
  const bool row_ok = grp_rows && prow < rows;
  const int qtok = row_ok ? prow / G : 0;
  const int qhead = h * G + (row_ok ? prow - (prow / G) * G : 0);
  const int allow = row_ok ? qtok + off : kv_len - 1;  // last visible kv token

  // kv tiles a group needs: up to its last row's visible token. The
  // workgroup gathers group 0's range, which contains group 1's.
  auto tiles_for = [&](int r0) {
    const int last_row = min(rows, r0 + kGM) - 1;
    return (min(kv_len, last_row / G + off + 1) + kBN - 1) / kBN;
  };
  const int ntiles = tiles_for(tile0 * kGM);
  const int my_tiles = !kPair ? ntiles : !grp_rows ? 0 : row0 == tile0 * kGM ? ntiles : tiles_for(row0);
  // First token index at which some row of the group may be masked.
  const int first_masked = row0 / G + off + 1;

  // Two K/V buffers per group; the loop is unrolled by two so each read
  // names its buffer by a compile-time offset. With KS > 1 the same memory
  // then carries the other groups' softmax states to group 0.
  Tile* tiles = reinterpret_cast<Tile*>(lds_raw + split * group_lds_bytes<KS>());
  // This group's kv tiles [tb, te) and the steps every group runs (equal,
  // so the workgroup-wide barriers match).
  const int share = (ntiles + KS - 1) / KS;
  const int tb = min(ntiles, split * share);
  const int te = min(ntiles, tb + share);
  const int nsteps = share;

  const uint16_t* kbase = a.kc + static_cast<int64_t>(h) * a.kv_sh;
  const uint16_t* vbase = a.vc + static_cast<int64_t>(h) * a.kv_sh;
  const int32_t* idx = a.indices + kv_beg;
  const uint32_t ss_bytes = static_cast<uint32_t>(a.kv_ss * 2);
  // Lane bases for rows r and r + 8 (r = 4 wave + lane / 16; the second is
  // used on odd u when GW = 2).
  const int lch0 = (lane & 15) ^ swz(4 * wave + (lane >> 4));
  const int lch1 = (lane & 15) ^ swz((4 * wave + (lane >> 4) + 8) & 15);
  const char* const klane[2] = {reinterpret_cast<const char*>(kbase) + lch0 * 16,
                                reinterpret_cast<const char*>(kbase) + lch1 * 16};
  const char* const vlane[2] = {reinterpret_cast<const char*>(vbase) + lch0 * 16,
                                reinterpret_cast<const char*>(vbase) + lch1 * 16};

  LaneAddr la;
  {
    const uint32_t base = lds_addr(tiles);
    const int sw = swz(c);
#pragma unroll
    for (int s = 0; s < 8; ++s) la.k[s] = base + c * kD * 2 + ((2 * s + hl) ^ sw) * 16;
    // Transpose-read source of lane l: row 4 (l / 32) + (l % 16) / 4 (+ 8 for
    // the upper slots), logical chunk 4 db + 2 ((l / 16) % 2) + (l % 4) / 2,
    // byte 8 (l % 2) within it; the swizzle of row 16 ks4 + vrow + 8 hi does
    // not depend on ks4.
    const int vrow = 4 * (lane >> 5) + ((lane & 15) >> 2);
    const int g = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int hi = 0; hi < 2; ++hi) {
        const int row = vrow + 8 * hi;
        const int phys = (4 * db + g) ^ swz(row);
        la.v[2 * db + hi] = base + kVOffset + row * kD * 2 + phys * 16 + 8 * (lane & 1);
      }
  }

  RowState rs;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int v = 0; v < 16; ++v) rs.acc[db][v] = 0.f;
  rs.m = -INFINITY;
  rs.l = 0.f;

  // Short shares (KS = 2, at most three kv tiles per group; launches that
  // are latency-bound, not bandwidth-bound): every tile's gathers are issued
  // at once -- K(0), V(0), K(1), V(1), K(2) into LDS (the group's 80 KiB) and
  // V(2) into registers, written to V(0)'s buffer once P(0) V(0) is done --
  // so the group waits for one memory round trip instead of one per tile.
  // Every wave issues the same operations whatever its group's tile count
  // (tiles past the share gather the clamped last token), so the vmcnt
  // counts below are exact: 8 gathers per tile half (16 / GW), 8 Q loads.
  auto short_share = [&](auto NSc) {
    constexpr int NS = decltype(NSc)::value;
    static_assert(GW == 2 && NS >= 1 && NS <= 3, "short shares: 2-wave groups, <= 3 tiles");
    constexpr int kOps = 16 / GW;
    int32_t sl[NS][kOps];
    static_for<0, NS>([&](auto I) {
      constexpr int i = decltype(I)::value;
      load_slots<GW>(idx, (tb + i) * kBN, kv_len, tid, sl[i]);
    });
    wait_gathers();
    issue_half<GW>(klane, ss_bytes, sl[0], tiles[0].k, wave);
    issue_half<GW>(vlane, ss_bytes, sl[0], tiles[0].v, wave);
    if constexpr (NS > 1) issue_half<GW>(klane, ss_bytes, sl[1], tiles[1].k, wave);
    // Q^T operand (rows past the item read row 0 and are zeroed: the loads
    // are unconditional so every wave issues the same count).
    bf16x8_t qop[8];
    {
      const uint16_t* qp = a.q + static_cast<int64_t>(qo_beg + qtok) * a.q_st +
                           static_cast<int64_t>(qhead) * a.q_sh;
      u32x4_t qv[8];
#pragma unroll
      for (int s = 0; s < 8; ++s) qv[s] = ldg128(qp + 16 * s + 8 * hl);
#pragma unroll
      for (int s = 0; s < 8; ++s) qop[s] = as_bf16x8(row_ok ? qv[s] : u32x4_t{0, 0, 0, 0});
    }
    if constexpr (NS > 1) issue_half<GW>(vlane, ss_bytes, sl[1], tiles[1].v, wave);
    if constexpr (NS > 2) issue_half<GW>(klane, ss_bytes, sl[2], tiles[2].k, wave);
    // V(2) into registers, lane for lane what issue_half would gather.
    u32x4_t v2[NS > 2 ? kOps : 1];
    if constexpr (NS > 2) {
#pragma unroll
      for (int u = 0; u < kOps; ++u)
        v2[u] = ldg128(vlane[u & 1] + static_cast<uint64_t>(static_cast<uint32_t>(sl[2][u])) *
                                          ss_bytes);
    }
    // K(0), V(0), K(1) and Q landed (younger: V(1), K(2), V(2)).
    wait_vm<(NS > 1 ? kOps : 0) + (NS > 2 ? 2 * kOps : 0)>();
    __builtin_amdgcn_s_barrier();
    LaneAddr la2 = la;
#pragma unroll
    for (int k = 0; k < 8; ++k) la2.k[k] += 2 * kTileBytes;
    f32x16_t s_a[2], s_b[2];
    bf16x8_t pop[4];
    qk_tile<0>(la, qop, s_a);
    // One step: P(t) from s_cur, S(t + 1) into s_next from K buffer KB
    // (none on the last tile), O += P(t) V(t) from V buffer VB.
    auto run = [&](auto Ic, auto KBc, auto VBc, f32x16_t(&s_cur)[2], f32x16_t(&s_next)[2]) {
      constexpr int i = decltype(Ic)::value;
      constexpr int kb = decltype(KBc)::value;
      constexpr int vb = decltype(VBc)::value;
      if (tb + i >= te) return;
      u32x2_t vr[4][8];
      if constexpr (i + 1 < NS) {
        // K buffer 2 lies past the 16-bit LDS offset range from buffer 0's
        // addresses: its reads use addresses rebased to it.
        constexpr int kbo = kb == 2 ? 0 : kb;
        const LaneAddr& lk = kb == 2 ? la2 : la;
        u32x4_t kbuf[16];
        qk_tile_prefetch<kbo>(lk, kbuf);
        softmax_head(a, s_cur, rs, (tb + i) * kBN, first_masked, allow, kv_len, hl);
        lgkm_wait<0>(kbuf[kKAhead - 1]);
        qk_tile_run<kbo>(lk, qop, s_next, kbuf);
      } else {
        softmax_head(a, s_cur, rs, (tb + i) * kBN, first_masked, allow, kv_len, hl);
      }
      softmax_exp_half<0>(a, s_cur, rs, pop);
      pv_reads<vb, 0>(la, vr[0]);
      pv_steps<vb, 0, 2>(la, pop, vr, rs);
      softmax_exp_half<1>(a, s_cur, rs, pop);
      pv_steps<vb, 2, 4>(la, pop, vr, rs);
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    run(I0{}, I1{}, I0{}, s_a, s_b);
    if constexpr (NS > 1) {
      // K(2) and V(1) landed (younger: V(2)); every wave is done with V(0).
      wait_vm<(NS > 2 ? kOps : 0)>();
      __builtin_amdgcn_s_barrier();
      if constexpr (NS > 2) {
        const uint32_t vdst = lds_addr(tiles[0].v) + (4 * wave) * kD * 2 + lane * 16;
        static_for<0, kOps>([&](auto U) {
          constexpr int u = decltype(U)::value;
          lds_write_b128<4 * GW * u * kD * 2>(vdst, v2[u]);
        });
      }
      run(I1{}, I2{}, I1{}, s_b, s_a);
    }
    if constexpr (NS > 2) {
      asm volatile("s_waitcnt lgkmcnt(0)");  // V(2) written by this wave
      __builtin_amdgcn_s_barrier();
      run(I2{}, I0{}, I0{}, s_a, s_b);
    }
  };
  bool short_done = false;
  if constexpr (KS == 2) {
    if (share <= 3) {
      short_done = true;
      if (share == 1) short_share(std::integral_constant<int, 1>{});
      else if (share == 2) short_share(std::integral_constant<int, 2>{});
      else short_share(std::integral_constant<int, 3>{});
    }
  }
  if (!short_done) {
    // Software pipeline over 64-token tiles. Iteration t computes S(t + 1)
    // on the matrix cores while the vector ALUs turn S(t) into P(t), then
    // O += P(t) V(t). K tiles are therefore gathered one tile ahead of V
    // tiles: during iteration t the gathers of K(t + 2) and V(t + 1) are in
    // flight. Tile j's K and V use buffer j % 2. Slot indices of tile t + 2
    // serve K(t + 2) now and V(t + 2) in the next iteration.
    // The slots of tiles 0 and 1 are waited for together before any gather
    // is issued (a gather between them would make the wait for the later
    // slots wait for the gather too: loads complete in order).
    int32_t sl_k[16 / GW], sl_v[16 / GW];
    load_slots<GW>(idx, tb * kBN, kv_len, tid, sl_k);
    load_slots<GW>(idx, (tb + 1) * kBN, kv_len, tid, sl_v);
    wait_gathers();
    if (tb < te) {
      issue_half<GW>(klane, ss_bytes, sl_k, tiles[0].k, wave);
      issue_half<GW>(vlane, ss_bytes, sl_k, tiles[0].v, wave);
    }
    if (tb + 1 < te) issue_half<GW>(klane, ss_bytes, sl_v, tiles[1].k, wave);
    load_slots<GW>(idx, (tb + 2) * kBN, kv_len, tid, sl_k);
    // Q^T operand: q[qtok][qhead][16 s + 8 hl .. +8], s < 8. Loaded after
    // the first gathers are issued: loads complete in order, so Q issued
    // earlier would delay the slot indices the gathers wait for.
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
    wait_gathers();
    __syncthreads();

    // Scores of the current and next tile; the two arrays swap roles every
    // step (the loop is unrolled by two), so no register copies move them.
    f32x16_t s_a[2], s_b[2];
    bf16x8_t pop[4];
    qk_tile<0>(la, qop, s_a);
    __syncthreads();  // every wave has read K(0) before K(2) overwrites it

    auto step = [&](auto B, int t, f32x16_t(&s_cur)[2], f32x16_t(&s_next)[2]) {
      constexpr int buf = decltype(B)::value;  // (t - tb) % 2
      if (t + 2 < te) issue_half<GW>(klane, ss_bytes, sl_k, tiles[buf].k, wave);
      if (t + 1 < te) issue_half<GW>(vlane, ss_bytes, sl_v, tiles[buf ^ 1].v, wave);
  #pragma unroll
      for (int u = 0; u < 16 / GW; ++u) sl_v[u] = sl_k[u];
      load_slots<GW>(idx, (t + 3) * kBN, kv_len, tid, sl_k);
      if (t < te && (!kPair || t < my_tiles)) {
        // S(t + 1)'s first K operand reads go out before the mask / max of
        // S(t), which hides their LDS latency (K(t + 1) landed and became
        // visible at the previous step's barrier). The full wait after the
        // VALU work keeps the counted waits exact whatever the compiler
        // placed in between.
        u32x4_t kb[16];
        qk_tile_prefetch<buf ^ 1>(la, kb);
        softmax_head(a, s_cur, rs, t * kBN, first_masked, allow, kv_len, hl);
        lgkm_wait<0>(kb[kKAhead - 1]);
        // The VALU work of P(t) is split so each half runs beside MFMAs: the
        // first half beside S(t + 1), the second beside the first half of
        // O += P(t) V(t).
        u32x2_t vr[4][8];
        qk_tile_run<buf ^ 1>(la, qop, s_next, kb);  // S(t + 1); unused after the last tile
        softmax_exp_half<0>(a, s_cur, rs, pop);
        pv_reads<buf, 0>(la, vr[0]);
        pv_steps<buf, 0, 2>(la, pop, vr, rs);
        softmax_exp_half<1>(a, s_cur, rs, pop);
        pv_steps<buf, 2, 4>(la, pop, vr, rs);
      }
      wait_gathers();
      __syncthreads();
    };
    for (int i = 0; i < nsteps; i += 2) {
      step(std::integral_constant<int, 0>{}, tb + i, s_a, s_b);
      if (i + 1 >= nsteps) break;
      step(std::integral_constant<int, 1>{}, tb + i + 1, s_b, s_a);
    }

  }

  if constexpr (KS > 1) {
    // Fold groups 1 .. KS-1 into group 0: each writes its (O, m, l) lane-major
    // ([group][value][wave][lane], conflict-free), group 0 reads the entries
    // of its own wave and lane (same rows, same accumulator slots) and
    // rescales every state to the largest reference point. The rings are
    // free once every wave is past its loop.
    float* xch = reinterpret_cast<float*>(lds_raw);
    auto at = [&](int g, int v) -> float& {
      return xch[((g - 1) * 66 + v) * 64 * GW + wave * 64 + lane];
    };
    __syncthreads();
    if (split > 0) {
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) at(split, 16 * db + v) = rs.acc[db][v];
      at(split, 64) = rs.m;
      at(split, 65) = rs.l;
    }
    __syncthreads();
    if (split > 0) return;
#pragma unroll
    for (int g = 1; g < KS; ++g) {
      const float mg = at(g, 64);
      const float mn = fmaxf(rs.m, mg);
      const float w0 = rs.m == -INFINITY ? 0.f : exp2f(rs.m - mn);
      const float wg = mg == -INFINITY ? 0.f : exp2f(mg - mn);
      rs.l = rs.l * w0 + at(g, 65) * wg;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) rs.acc[db][v] = rs.acc[db][v] * w0 + at(g, 16 * db + v) * wg;
      rs.m = mn;
    }
  }

  float l = sum_xor32(rs.l);
  if (!row_ok) return;
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  uint16_t* op =
      a.o + static_cast<int64_t>(qo_beg + qtok) * a.o_st + static_cast<int64_t>(qhead) * a.o_sh;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const u32x2_t w = {pack_bf16x2(rs.acc[db][4 * g] * inv, rs.acc[db][4 * g + 1] * inv),
                         pack_bf16x2(rs.acc[db][4 * g + 2] * inv, rs.acc[db][4 * g + 3] * inv)};
      *reinterpret_cast<u32x2_t*>(op + 32 * db + 8 * g + 4 * hl) = w;
    }
}

// Checks shared by the prefill entry points (pointers, head layout,
// strides, alignment); fills the kernel arguments except the item layout
// (tiles_per_req, num_kv_heads).
inline int prefill_args(const void* q, int64_t q_stride_token, int64_t q_stride_head,
                        const void* k_cache, const void* v_cache, int64_t kv_stride_slot,
                        int64_t kv_stride_head, const int32_t* indices, const int32_t* qo_indptr,
                        const int32_t* kv_indptr, const int32_t* q_start, int num_qo_heads,
                        int num_kv_heads, int head_dim, float sm_scale, void* o,
                        int64_t o_stride_token, int64_t o_stride_head, PrefillArgs& a) {
  if (num_qo_heads <= 0 || num_kv_heads <= 0) return SGL_ERR_INVALID_ARG;
  if (!q || !k_cache || !v_cache || !indices || !qo_indptr || !kv_indptr || !o)
    return SGL_ERR_INVALID_ARG;
  if (num_qo_heads % num_kv_heads != 0) return SGL_ERR_INVALID_ARG;
  if (head_dim != kD) return SGL_ERR_UNSUPPORTED;
  // Gather addresses use 32-bit slot byte strides.
  if (kv_stride_slot <= 0 || kv_stride_slot > 0x7fffffff) return SGL_ERR_UNSUPPORTED;
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
  a.qo_indptr = qo_indptr;
  a.kv_indptr = kv_indptr;
  a.q_start = q_start;
  a.group = num_qo_heads / num_kv_heads;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.o = static_cast<uint16_t*>(o);
  a.o_st = o_stride_token;
  a.o_sh = o_stride_head;
  a.num_kv_heads = num_kv_heads;
  return SGL_OK;
}

}  // namespace
}  // namespace pf
}  // namespace sgl
