// Sampling from probabilities: plain (inverse CDF), top-k, top-p and
// top-k + top-p, the kernels behind the reference's Sampler::sample
// (src/engine/sampling.cu:65-194, called from src/engine/engine.cc:300-345).
//
// The reference calls FlashInfer v0.2.0.post1's sampling kernels; their
// published algorithm, restated here:
//   * inverse-CDF draw with threshold t and uniform u: the first index i
//     (in row order) with p_i > t and sum_{j <= i, p_j > t} p_j > u; when
//     rounding leaves no such index, d - 1.
//   * top-k / top-p / both: rejection rounds with a rising pivot. Round r
//     draws index s with threshold = pivot and u = uniform[r] * q, where q
//     is the mass of the probabilities above the pivot (1 in round 0);
//     then pivot = max(pivot, p_s) and (count, q) = how many probabilities
//     exceed the pivot and their sum. The draw is accepted when count < k
//     (top-k), q < top_p (top-p), or both; otherwise the next round runs.
//     success[row] reports acceptance within the given rounds; the output
//     is the last draw either way.
// The reference's `deterministic` switch selects FlashInfer's ordered
// prefix sum; these kernels sum in a fixed order always, so it is accepted
// and has no effect.
//
// MI355X layout: one 1024-thread workgroup (16 waves) per row. The row is
// cut into blocks of 512 probabilities, eight consecutive ones per lane
// (two 16-byte loads of fp32 probabilities, or one of 16-bit logits); waves
// take blocks round-robin, two blocks in flight. A sweep with a threshold
// leaves in LDS the mass above it of every block (one wave reduction per
// block) and the row's mass and count above it. A draw is wave 0's alone:
// each lane sums a run of block masses, a DPP wave scan finds the lane
// whose run crosses u, that lane walks to the crossing block, and the wave
// scans the block's probabilities in row order to the first crossing
// index. A rejection round is one sweep: the sweep that counts the
// probabilities above the new pivot also gives the next draw its block
// masses. A vocabulary row (Qwen3: 151,936 x 4 B) comes from HBM on the
// first sweep. That sweep also copies into LDS every probability above
// 1/30,464 (at most 30,464 of them in a normalised row), so rounds whose
// pivot clears that threshold sweep the copies instead of the row; when it
// does not, the next sweep of the row copies what exceeds its pivot, space
// allowing. Only the crossing block of a draw is read from the row then.
//
// Draws from 16-bit logits (rows of up to 163,840, 16-byte aligned, length
// a multiple of 8) read the row from HBM once: thread t keeps its 16-byte
// chunks t + 1024 k in registers, which are exactly lane t % 64's share of
// blocks t / 64 + 16 k, computes the row statistics from them, and every
// sweep of the row recomputes the probabilities from the registers.
#include <math.h>

#include "common.h"
#include "sampler_prob.h"

namespace sgl {
namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / kWave;
constexpr int kVec = 4;
constexpr int kSub = 2;                       // 16-byte loads per lane per block
constexpr int kPerLane = kVec * kSub;         // consecutive probabilities per lane
constexpr int kBlock = kWave * kPerLane;      // probabilities per block (512)
constexpr int kMaxBlocks = 4096;              // rows up to 2M probabilities
// Candidate mode (rows of at most kCandBlocks blocks, 1M probabilities): a
// sweep of the row also copies the probabilities above a threshold into
// LDS, grouped by block, and later rounds whose pivot is at or above that
// threshold sweep those copies instead of the row. The copies share one LDS
// pool with the block masses, which then need only kCandBlocks entries.
constexpr int kCandBlocks = 2048;              // one (start, count) word per block
constexpr int kPool = 36864;                   // 144 KiB
constexpr int kCandCap = kPool - kCandBlocks;  // 34,816 copies
// Draws from 16-bit logits hold rows of up to kMaxHeldChunks 16-byte chunks a
// lane (163,840 logits, 80 VGPRs) in registers.
constexpr int kMaxHeldChunks = 20;
// Word 3 of a raw buffer resource on gfx950 (32-bit data format, no
// swizzle, unit stride): byte-addressed loads with a range check.
constexpr int kRawBufferWord3 = 0x00020000;
static_assert(kPool >= kMaxBlocks, "block masses of the longest rows fit the pool");
static_assert(kCandCap < 65536 && kBlock < 65536, "segment words hold two 16-bit fields");

struct SampleArgs {
  const float* probs;
  const float* uniform;    // [rounds, batch] (or [batch] for the plain draw)
  int32_t* out;
  uint8_t* success;        // optional
  const float* top_k_f;    // top-k per row as float (top-k kernel), optional
  const int32_t* top_k_i;  // top-k per row as int32 (top-k + top-p kernel), optional
  const float* top_p_arr;  // optional
  int batch, d, rounds;
  int top_k_val;
  float top_p_val;
  int mode;  // 0 plain, 1 top-k, 2 top-p, 3 top-k + top-p
  bool vec;  // rows 16-byte aligned (d % 4 == 0 and an aligned base)
  // Draws from logits (probs == nullptr): the probabilities are computed on
  // the fly by sampler_prob.h, bit for bit those sgl_softmax_temperature
  // writes.
  const void* logits;
  int64_t x_st;        // logits row stride (elements)
  const float* temps;  // [batch] or null
  float temp;
  bool stats_vec;      // logits rows 16-byte aligned (the softmax kernel's vector path)
  int logit_dtype;
};

// Where a draw reads the probability of element e of its row: the fp32
// probabilities, or the logits through the Sampler's softmax.
struct ProbRow {
  const float* p;
  __device__ f32x4_t load4(int64_t e) const { return *reinterpret_cast<const f32x4_t*>(p + e); }
  __device__ float load1(int64_t e) const { return p[e]; }
};

template <int DT>
struct LogitRow {
  const char* x;
  float sc, nb, inv_s;  // sampler_prob.h's row constants
  // Four consecutive elements from e (e % 4 == 0 on a 16-byte aligned row).
  __device__ f32x4_t load4(int64_t e) const {
    u32x4_t v;
    if constexpr (DT == SGL_DTYPE_F32) {
      v = *reinterpret_cast<const u32x4_t*>(x + e * 4);
    } else {
      const u32x2_t h = *reinterpret_cast<const u32x2_t*>(x + e * 2);
      v = u32x4_t{h[0], h[1], 0u, 0u};
    }
    f32x4_t r;
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = sp::prob(sp::Elem<DT>::at(v, j), sc, nb, inv_s);
    return r;
  }
  __device__ float load1(int64_t e) const {
    return sp::prob(sp::Elem<DT>::load1(x, e), sc, nb, inv_s);
  }
};

struct Shared {
  // pool[b], b < nblk: mass above the current threshold of block b.
  // pool[kCandBlocks + i]: candidate mode's copies, block by block.
  float pool[kPool];
  uint32_t seg[kCandBlocks];  // block b's copies: start | count << 16
  int ncand;                  // copies written (beyond kCandCap: overflow)
  float wave_f[kWaves];
  float wave_n[kWaves];
  int wave_i[kWaves];
  float wave_run[kWaves];  // draw: mass before the crossing block found by a wave
  float total;             // row mass above the threshold
  int count;               // row count above the threshold
  int sampled;
  float sampled_p;
};

__device__ __forceinline__ float wave_sum_f(float x) {
  return sum_xor32(sum_xor16(group_sum<16>(x)));
}

// DPP move with a row mask: rows left out of ROW_MASK, and lanes whose
// source lies outside their row, read 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_rows(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, ROW_MASK, 0xF, false));
}

// Inclusive scan within each row of 16 lanes (DPP row_shr 1, 2, 4, 8).
__device__ __forceinline__ float row_scan(float x) {
  x += dpp_rows<0x111, 0xF>(x);
  x += dpp_rows<0x112, 0xF>(x);
  x += dpp_rows<0x114, 0xF>(x);
  x += dpp_rows<0x118, 0xF>(x);
  return x;
}

// Inclusive scan over the 64 lanes: the row scans, then row_bcast:15 adds
// row r's total to row r + 1 (rows 1 and 3) and row_bcast:31 the first two
// rows' total to rows 2 and 3.
__device__ __forceinline__ float wave_scan(float x) {
  x = row_scan(x);
  x += dpp_rows<0x142, 0xA>(x);
  x += dpp_rows<0x143, 0xC>(x);
  return x;
}

template <typename T>
__device__ __forceinline__ T read_lane(T x, int l) {
  return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
}

// One block of a row: lane l holds probabilities kPerLane l + kVec s + j
// (s < kSub, j < kVec) of the block, in row order; bounds-checked when the
// block is the row's last or the row is not 16-byte aligned.
struct BlockVals {
  f32x4_t v[kSub];
};

template <class Src>
__device__ __forceinline__ void load_block(const Src& row, int b, int d, bool full, BlockVals& bv) {
  const int lane = threadIdx.x & 63;
  const int e0 = b * kBlock + kPerLane * lane;
  if (full) {
#pragma unroll
    for (int s = 0; s < kSub; ++s) bv.v[s] = row.load4(e0 + kVec * s);
  } else {
#pragma unroll
    for (int s = 0; s < kSub; ++s)
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        const int e = e0 + kVec * s + j;
        bv.v[s][j] = e < d ? row.load1(e) : 0.f;
      }
  }
}

// Row totals from the per-wave mass wm and count wn (both wave-uniform):
// wave 0 adds the 16 wave totals in a fixed DPP order.
__device__ __forceinline__ void finish_totals(float wm, int wn, Shared& sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sh.wave_f[wave] = wm;
    sh.wave_n[wave] = static_cast<float>(wn);
  }
  __syncthreads();
  if (wave == 0) {
    const float t = group_sum<16>(lane < kWaves ? sh.wave_f[lane] : 0.f);
    const float c = group_sum<16>(lane < kWaves ? sh.wave_n[lane] : 0.f);
    if (lane == 0) {
      sh.total = t;
      sh.count = static_cast<int>(c);
    }
  }
  __syncthreads();
}

// The lanes below this one whose bit is set in mask.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
}

// Mass and count above thr of one block (mass wave-reduced into pool[b],
// count wave-wide from the comparison masks); kCompact: also the copies
// above cthr, placed element-major (element j of every lane, lanes in
// order, then element j + 1), a fixed order that needs one lane count per
// element that has any copy.
template <bool kCompact>
__device__ __forceinline__ void sweep_block(const BlockVals& bv, int b, float thr, float cthr,
                                            float& wm, int& wn, Shared& sh) {
  const int lane = threadIdx.x & 63;
  float m = 0.f;
#pragma unroll
  for (int s = 0; s < kSub; ++s)
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      const float x = bv.v[s][j];
      const bool above = x > thr;
      m += above ? x : 0.f;
      wn += __builtin_popcountll(__ballot(above));
    }
  m = wave_sum_f(m);
  wm += m;
  if (lane == 0) sh.pool[b] = m;
  if constexpr (kCompact) {
    uint64_t mk[kPerLane];
    int tot = 0;
#pragma unroll
    for (int s = 0; s < kSub; ++s)
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        mk[kVec * s + j] = __ballot(bv.v[s][j] > cthr);
        tot += __builtin_popcountll(mk[kVec * s + j]);
      }
    int base = 0;
    if (tot > 0) {
      if (lane == 0) base = atomicAdd(&sh.ncand, tot);
      base = read_lane(base, 0);
      if (base + tot <= kCandCap) {
        int pos = kCandBlocks + base;
#pragma unroll
        for (int s = 0; s < kSub; ++s)
#pragma unroll
          for (int j = 0; j < kVec; ++j) {
            const uint64_t mj = mk[kVec * s + j];
            if (mj != 0) {
              if (bv.v[s][j] > cthr) sh.pool[pos + lanes_below(mj)] = bv.v[s][j];
              pos += __builtin_popcountll(mj);
            }
          }
      }
    }
    if (lane == 0) sh.seg[b] = static_cast<uint32_t>(base) | static_cast<uint32_t>(tot) << 16;
  }
}

// Block masses, row mass and row count of the probabilities above thr.
// kCompact: also copy the probabilities above cthr (the caller has zeroed
// sh.ncand; an overflow shows as sh.ncand > kCandCap). Waves take blocks
// round-robin, two blocks (8 loads per lane) in flight.
template <bool kCompact, class Src>
__device__ __forceinline__ void sweep(const Src& row, int d, bool vec, float thr, float cthr,
                                      Shared& sh) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nblk = (d + kBlock - 1) / kBlock;
  const int nfull = vec ? d / kBlock : 0;  // blocks loaded without bounds checks
  float wm = 0.f;
  int wn = 0;
  __syncthreads();  // the previous readers of sh are done
  int b = wave;
  for (; b + kWaves < nfull; b += 2 * kWaves) {
    BlockVals x0, x1;
    load_block(row, b, d, true, x0);
    load_block(row, b + kWaves, d, true, x1);
    sweep_block<kCompact>(x0, b, thr, cthr, wm, wn, sh);
    sweep_block<kCompact>(x1, b + kWaves, thr, cthr, wm, wn, sh);
  }
  for (; b < nblk; b += kWaves) {
    BlockVals x0;
    load_block(row, b, d, b < nfull, x0);
    sweep_block<kCompact>(x0, b, thr, cthr, wm, wn, sh);
  }
  finish_totals(wm, wn, sh);
}

// The same sweep over the copies: each group of 16 lanes takes one block
// (wave w, group g: blocks 4 w + g, 4 w + g + 64, ...) and its lanes the
// block's copies.
__device__ __forceinline__ void sweep_cand(int d, float thr, Shared& sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane & 15;
  const int nblk = (d + kBlock - 1) / kBlock;
  float wm = 0.f, wn = 0.f;
  // No leading barrier: only the draw, which ends with one, read the
  // masses since the last sweep.
  for (int b0 = 4 * wave; b0 < nblk; b0 += 4 * kWaves) {
    const int b = b0 + (lane >> 4);
    const uint32_t sg = b < nblk ? sh.seg[b] : 0u;
    const int start = static_cast<int>(sg & 0xFFFF), n = static_cast<int>(sg >> 16);
    float m = 0.f;
    for (int i = sub; i < n; i += 16) {
      const float x = sh.pool[kCandBlocks + start + i];
      m += x > thr ? x : 0.f;
      wn += x > thr ? 1.f : 0.f;
    }
    m = group_sum<16>(m);
    if (b < nblk && sub == 0) sh.pool[b] = m;
    // wave-uniform partial of the four blocks, in group order
    wm += read_lane(m, 0) + read_lane(m, 16) + read_lane(m, 32) + read_lane(m, 48);
  }
  finish_totals(wm, static_cast<int>(wave_sum_f(wn)), sh);
}

// The inverse-CDF draw over the probabilities above thr with target u, from
// the block masses of the last sweep with the same threshold, in two steps.
// find_block (one wave): lane l sums its run of block masses, a wave scan
// finds the first lane whose run crosses u, and that lane walks its run to
// the crossing block; returns it (nblk when no run crosses) and the mass
// before it (wave-uniform).
__device__ __forceinline__ void find_block(int nblk, float u, const Shared& sh, int& bs,
                                           float& base) {
  const int lane = threadIdx.x & 63;
  const int per = (nblk + kWave - 1) / kWave;
  const int b0 = min(nblk, lane * per), b1 = min(nblk, b0 + per);
  float own = 0.f;
  for (int b = b0; b < b1; ++b) own += sh.pool[b];
  const float incl = wave_scan(own);
  const uint64_t cross = __ballot(incl > u);
  bs = nblk;
  base = 0.f;
  if (cross) {
    const int L = __builtin_ctzll(cross);
    float run = incl - own;
    int b = b1 - 1;
    if (lane == L) {
      for (int c = b0; c < b1; ++c) {
        if (run + sh.pool[c] > u) {
          b = c;
          break;
        }
        run += sh.pool[c];
      }
    }
    bs = read_lane(b, L);
    base = read_lane(run, L);
  }
}

// scan_block (one wave): lane l holds the block's probabilities
// [kPerLane l, kPerLane l + kPerLane) in p, element e0 + i of the row, valid
// where below d; the first one above thr whose running mass from base
// exceeds u (lowest lane first: lanes run in row order), else (rounding
// inside the block missed u) the block's last one above thr. Returns false
// when the block has none above thr.
__device__ __forceinline__ bool scan_block(const float (&p)[kPerLane], int e0, int d, float thr,
                                           float base, float u, Shared& sh) {
  const int lane = threadIdx.x & 63;
  int first = d, last_valid = -1;
  float first_p = 0.f, last_p = 0.f;
  float local = 0.f;
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) local += p[i] > thr ? p[i] : 0.f;
  const float cincl = wave_scan(local);
  float cdf = base + (cincl - local);
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) {
    const bool valid = p[i] > thr && e0 + i < d;
    cdf += valid ? p[i] : 0.f;
    if (valid) {
      last_valid = e0 + i;
      last_p = p[i];
    }
    if (valid && cdf > u && first == d) {
      first = e0 + i;
      first_p = p[i];
    }
  }
  const uint64_t has_first = __ballot(first < d);
  const uint64_t has_last = __ballot(last_valid >= 0);
  if (has_first) {
    if (lane == __builtin_ctzll(has_first)) {
      sh.sampled = first;
      sh.sampled_p = first_p;
    }
    return true;
  }
  if (has_last) {
    if (lane == 63 - __builtin_clzll(has_last)) {
      sh.sampled = last_valid;
      sh.sampled_p = last_p;
    }
    return true;
  }
  return false;
}

// The draw by wave 0 alone (one barrier), the crossing block read from the
// row: leaves the index in sh.sampled and its probability in sh.sampled_p
// (d - 1 when no probability above thr is found).
template <class Src>
__device__ __forceinline__ void draw(const Src& row, int d, bool vec, float thr, float u,
                                     Shared& sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nblk = (d + kBlock - 1) / kBlock;
  if (wave == 0) {
    int bs;
    float base;
    find_block(nblk, u, sh, bs, base);
    bool found = false;
    if (bs < nblk) {
      const int e0 = bs * kBlock + kPerLane * lane;
      float p[kPerLane];
      if (vec && e0 + kPerLane <= d) {
#pragma unroll
        for (int s = 0; s < kPerLane / 4; ++s) {
          const f32x4_t v = row.load4(e0 + 4 * s);
#pragma unroll
          for (int j = 0; j < 4; ++j) p[4 * s + j] = v[j];
        }
      } else {
#pragma unroll
        for (int i = 0; i < kPerLane; ++i) p[i] = e0 + i < d ? row.load1(e0 + i) : 0.f;
      }
      found = scan_block(p, e0, d, thr, base, u, sh);
    }
    if (!found && lane == 0) {
      sh.sampled = d - 1;
      sh.sampled_p = row.load1(d - 1);
    }
  }
  __syncthreads();
}

// Sweeps of a row read from memory (fp32 probabilities or logits).
template <class Src>
struct StreamSweep {
  const Src& row;
  int d;
  bool vec;
  template <bool kCompact>
  __device__ __forceinline__ void run(float thr, float cthr, Shared& sh) const {
    sweep<kCompact>(row, d, vec, thr, cthr, sh);
  }
  __device__ __forceinline__ void pick(float thr, float u, Shared& sh) const {
    draw(row, d, vec, thr, u, sh);
  }
};

// Sweeps of a 16-bit logits row held in registers (aligned rows, d % 8 == 0):
// thread t holds chunk c = t + 1024 k (elements [8 c, 8 c + 8)) in held[k],
// which is lane t % 64's share of block t / 64 + 16 k -- the block a wave
// takes in sweep() and in the same per-lane order, so the masses, counts and
// copies are the bits the sweep of the fp32 probabilities gives.
template <int DT, int NC>
struct HeldSweep {
  const u32x4_t (&held)[NC];
  const LogitRow<DT>& row;
  int d;
  float sc, nb, inv_s;
  // The draw reads its crossing block from the row (scanning it from the
  // registers of the wave that holds it, after one more barrier, measured
  // no faster).
  __device__ __forceinline__ void pick(float thr, float u, Shared& sh) const {
    draw(row, d, true, thr, u, sh);
  }
  template <bool kCompact>
  __device__ __forceinline__ void run(float thr, float cthr, Shared& sh) const {
    // Wave-uniform, in a scalar register (block indices and LDS addresses
    // then cost no VGPRs).
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nblk = (d + kBlock - 1) / kBlock;
    const int nchunk = d / kPerLane;
    float wm = 0.f;
    int wn = 0;
    __syncthreads();  // the previous readers of sh are done
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      const int b = wave + kWaves * k;
      if (b < nblk) {
        // An opaque copy: the probabilities are the same every sweep, and
        // hoisted out of the rounds they would take 8 NC VGPRs instead of
        // the packed row's 4 NC.
        u32x4_t h = held[k];
        asm volatile("" : "+v"(h));
        BlockVals bv;
#pragma unroll
        for (int s = 0; s < kSub; ++s)
#pragma unroll
          for (int j = 0; j < kVec; ++j)
            bv.v[s][j] = sp::prob(sp::Elem<DT>::at(h, kVec * s + j), sc, nb, inv_s);
        if (kThreads * (k + 1) > nchunk) {  // the row's last chunks: some lanes hold none
          const bool in = static_cast<int>(threadIdx.x) + kThreads * k < nchunk;
#pragma unroll
          for (int s = 0; s < kSub; ++s)
#pragma unroll
            for (int j = 0; j < kVec; ++j) bv.v[s][j] = in ? bv.v[s][j] : 0.f;
        }
        sweep_block<kCompact>(bv, b, thr, cthr, wm, wn, sh);
      }
      // One block's values live at a time (the row itself takes 4 NC VGPRs).
      __builtin_amdgcn_sched_barrier(0);
    }
    finish_totals(wm, wn, sh);
  }
};

template <class Src, class Sweep>
__device__ __forceinline__ void sample_row(const SampleArgs& a, const Src& row, const Sweep& rs,
                                           Shared& sh) {
  const int row_id = blockIdx.x;
  const bool cand_ok = a.mode != 0 && (a.d + kBlock - 1) / kBlock <= kCandBlocks;
  // The first sweep already copies the probabilities above cand_thr: at
  // most 1 / cand_thr of them in a normalised row, so any pivot at or above
  // cand_thr is served from LDS.
  float cand_thr = 1.f / static_cast<float>(kCandCap - kCandCap / 8);
  bool cand = false;  // the copies hold every probability above cand_thr
  float u = a.uniform[row_id];
  if (cand_ok) {
    if (threadIdx.x == 0) sh.ncand = 0;
    rs.template run<true>(0.f, cand_thr, sh);
    cand = sh.ncand <= kCandCap;
  } else {
    rs.template run<false>(0.f, 0.f, sh);
  }
  if (a.mode == 0) {
    rs.pick(0.f, u, sh);
    if (threadIdx.x == 0) a.out[row_id] = sh.sampled;
    return;
  }
  int k = a.top_k_val;
  if (a.top_k_f) k = static_cast<int>(static_cast<uint32_t>(a.top_k_f[row_id]));
  if (a.top_k_i) k = a.top_k_i[row_id];
  const float top_p = a.top_p_arr ? a.top_p_arr[row_id] : a.top_p_val;
  float pivot = 0.f, q = 1.f;
  int sampled = a.d - 1;
  bool accepted = false;
  for (int r = 0; r < a.rounds; ++r) {
    // The next round's uniform is loaded while this round runs.
    const float u_next =
        r + 1 < a.rounds ? a.uniform[static_cast<int64_t>(r + 1) * a.batch + row_id] : 0.f;
    rs.pick(pivot, u * q, sh);
    sampled = sh.sampled;
    const float ps = sh.sampled_p;
    if (ps > pivot) {
      // Masses above the new pivot: from the copies when they cover it,
      // else from the row, copying what exceeds the pivot when no copies
      // are held (they stay unused if they overflow).
      pivot = ps;
      if (cand && pivot >= cand_thr) {
        sweep_cand(a.d, pivot, sh);
      } else if (!cand && cand_ok) {
        if (threadIdx.x == 0) sh.ncand = 0;
        rs.template run<true>(pivot, pivot, sh);
        cand = sh.ncand <= kCandCap;
        cand_thr = pivot;
      } else {
        rs.template run<false>(pivot, 0.f, sh);
      }
    }
    q = sh.total;
    const int count = sh.count;
    if (a.mode == 1) accepted = static_cast<uint32_t>(count) < static_cast<uint32_t>(k);
    else if (a.mode == 2) accepted = q < top_p;
    else accepted = count < k && q < top_p;
    if (accepted) break;
    u = u_next;
  }
  if (threadIdx.x == 0) {
    a.out[row_id] = sampled;
    if (a.success) a.success[row_id] = accepted ? 1 : 0;
  }
}

// SRC < 0: rows of fp32 probabilities; else logits of element type SRC,
// whose row max and sum are computed first exactly as the softmax kernel
// computes them (one statistics lane per thread).
template <int SRC>
__global__ void __launch_bounds__(kThreads) sampling_kernel(SampleArgs a) {
  __shared__ Shared sh;
  const int row_id = blockIdx.x;
  if constexpr (SRC < 0) {
    const ProbRow row{a.probs + static_cast<int64_t>(row_id) * a.d};
    sample_row(a, row, StreamSweep<ProbRow>{row, a.d, a.vec}, sh);
  } else {
    static_assert(kThreads == sp::kStatLanes, "one statistics lane per thread");
    constexpr int B = 16 / sp::Elem<SRC>::kPer;
    const char* x = static_cast<const char*>(a.logits) + static_cast<int64_t>(row_id) * a.x_st * B;
    const float t = a.temps ? a.temps[row_id] : a.temp;
    const float sc = sp::exp2_scale(t);
    const sp::LaneStats st = sp::lane_stats<SRC>(x, a.d, a.stats_vec, threadIdx.x, sc);
    const float m = sp::block_max<kWaves>(st.mx, sh.wave_f);
    const float inv_s = 1.0f / sp::block_sum<kWaves>(sp::lane_sum_at(st, m, sc), sh.wave_f);
    const LogitRow<SRC> row{x, sc, sp::exp2_offset(m, sc), inv_s};
    sample_row(a, row, StreamSweep<LogitRow<SRC>>{row, a.d, a.vec}, sh);
  }
}

// Draws from 16-bit logits rows of at most NC chunks a lane, aligned and
// d % 8 == 0: the row is read from memory once, into registers, in the
// statistics order of sp::lane_stats (the same bits); every later sweep of
// the row recomputes its probabilities from the registers. Only a draw's
// crossing block is read from memory again.
template <int SRC, int NC>
__global__ void __launch_bounds__(kThreads) sampling_held_kernel(SampleArgs a) {
  __shared__ Shared sh;
  static_assert(kThreads == sp::kStatLanes && sp::Elem<SRC>::kPer == kPerLane,
                "a statistics chunk is a lane's share of a block");
  const int row_id = blockIdx.x;
  const int tid = threadIdx.x;
  const char* x = static_cast<const char*>(a.logits) + static_cast<int64_t>(row_id) * a.x_st * 2;
  const float t = a.temps ? a.temps[row_id] : a.temp;
  const float sc = sp::exp2_scale(t);
  const int nchunk = a.d / kPerLane;
  u32x4_t held[NC];
  const __amdgpu_buffer_rsrc_t rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(x), 0, a.d * 2, kRawBufferWord3);
#pragma unroll
  for (int k = 0; k < NC; ++k)
    held[k] = __builtin_bit_cast(
        u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rsrc, tid * 16, k * kThreads * 16, 0));
  sp::LaneStats st;
#pragma unroll
  for (int k = 0; k < NC; ++k)
    if (tid + k * kThreads < nchunk) {
      float xs[kPerLane];
      sp::unpack<SRC>(held[k], xs);
      sp::online_update(xs, sc, st);
    }
  const float m = sp::block_max<kWaves>(st.mx, sh.wave_f);
  const float inv_s = 1.0f / sp::block_sum<kWaves>(sp::lane_sum_at(st, m, sc), sh.wave_f);
  const float nb = sp::exp2_offset(m, sc);
  // Keeps the packed row, not the statistics pass's fp32 values, live.
#pragma unroll
  for (int k = 0; k < NC; ++k) asm volatile("" : "+v"(held[k]));
  const LogitRow<SRC> row{x, sc, nb, inv_s};
  sample_row(a, row, HeldSweep<SRC, NC>{held, row, a.d, sc, nb, inv_s}, sh);
}

template <int SRC>
void launch_held(const SampleArgs& a, int per_lane, dim3 grid, dim3 block, hipStream_t s) {
  if (per_lane <= 4)
    hipLaunchKernelGGL((sampling_held_kernel<SRC, 4>), grid, block, 0, s, a);
  else if (per_lane <= 8)
    hipLaunchKernelGGL((sampling_held_kernel<SRC, 8>), grid, block, 0, s, a);
  else if (per_lane <= 12)
    hipLaunchKernelGGL((sampling_held_kernel<SRC, 12>), grid, block, 0, s, a);
  else if (per_lane <= 16)
    hipLaunchKernelGGL((sampling_held_kernel<SRC, 16>), grid, block, 0, s, a);
  else if (per_lane <= 19)  // Qwen3's 151,936 logits
    hipLaunchKernelGGL((sampling_held_kernel<SRC, 19>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((sampling_held_kernel<SRC, kMaxHeldChunks>), grid, block, 0, s, a);
}

int launch_sampling(const SampleArgs& a, void* stream) {
  if (a.batch < 0 || a.d <= 0 || (a.mode != 0 && a.rounds <= 0)) return SGL_ERR_INVALID_ARG;
  if ((static_cast<int64_t>(a.d) + kBlock - 1) / kBlock > kMaxBlocks) return SGL_ERR_UNSUPPORTED;
  if (a.batch == 0) return SGL_OK;
  if (!a.uniform || !a.out) return SGL_ERR_INVALID_ARG;
  const dim3 grid(a.batch), block(kThreads);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a.probs) {
    hipLaunchKernelGGL(sampling_kernel<-1>, grid, block, 0, s, a);
  } else if (a.logits) {
    const int per_lane = (a.d / kPerLane + kThreads - 1) / kThreads;
    const bool held = a.logit_dtype != SGL_DTYPE_F32 && a.vec && a.d % kPerLane == 0 &&
                      per_lane <= kMaxHeldChunks;
    if (held && a.logit_dtype == SGL_DTYPE_BF16)
      launch_held<SGL_DTYPE_BF16>(a, per_lane, grid, block, s);
    else if (held)
      launch_held<SGL_DTYPE_F16>(a, per_lane, grid, block, s);
    else if (a.logit_dtype == SGL_DTYPE_BF16)
      hipLaunchKernelGGL(sampling_kernel<SGL_DTYPE_BF16>, grid, block, 0, s, a);
    else if (a.logit_dtype == SGL_DTYPE_F16)
      hipLaunchKernelGGL(sampling_kernel<SGL_DTYPE_F16>, grid, block, 0, s, a);
    else
      hipLaunchKernelGGL(sampling_kernel<SGL_DTYPE_F32>, grid, block, 0, s, a);
  } else {
    return SGL_ERR_INVALID_ARG;
  }
  return launch_status();
}

SampleArgs base_args(const float* probs, const float* uniform, int32_t* out, uint8_t* success,
                     int batch, int d, int rounds, int mode) {
  SampleArgs a{};
  a.probs = probs;
  a.uniform = uniform;
  a.out = out;
  a.success = success;
  a.batch = batch;
  a.d = d;
  a.rounds = rounds;
  a.mode = mode;
  a.vec = d % 4 == 0 && aligned16(probs);
  return a;
}

}  // namespace
}  // namespace sgl

using namespace sgl;

extern "C" int sgl_sampling_from_probs(const float* probs, const float* uniform, int32_t* out,
                                       int batch_size, int d, int deterministic, void* stream) {
  (void)deterministic;
  return launch_sampling(base_args(probs, uniform, out, nullptr, batch_size, d, 1, 0), stream);
}

extern "C" int sgl_top_k_sampling_from_probs(const float* probs, const float* uniform,
                                             int32_t* out, uint8_t* success, const float* top_k_arr,
                                             int batch_size, int top_k_val, int d, int max_rounds,
                                             int deterministic, void* stream) {
  (void)deterministic;
  SampleArgs a = base_args(probs, uniform, out, success, batch_size, d, max_rounds, 1);
  a.top_k_f = top_k_arr;
  a.top_k_val = top_k_val;
  return launch_sampling(a, stream);
}

extern "C" int sgl_top_p_sampling_from_probs(const float* probs, const float* uniform,
                                             int32_t* out, uint8_t* success, const float* top_p_arr,
                                             int batch_size, float top_p_val, int d, int max_rounds,
                                             int deterministic, void* stream) {
  (void)deterministic;
  SampleArgs a = base_args(probs, uniform, out, success, batch_size, d, max_rounds, 2);
  a.top_p_arr = top_p_arr;
  a.top_p_val = top_p_val;
  return launch_sampling(a, stream);
}

extern "C" int sgl_top_k_top_p_sampling_from_probs(const float* probs, const float* uniform,
                                                   const int32_t* top_k_arr, const float* top_p_arr,
                                                   int32_t* out, uint8_t* success, int batch_size,
                                                   int top_k_val, float top_p_val, int d,
                                                   int max_rounds, int deterministic,
                                                   void* stream) {
  (void)deterministic;
  SampleArgs a = base_args(probs, uniform, out, success, batch_size, d, max_rounds, 3);
  a.top_k_i = top_k_arr;
  a.top_k_val = top_k_val;
  a.top_p_arr = top_p_arr;
  a.top_p_val = top_p_val;
  return launch_sampling(a, stream);
}

extern "C" int sgl_sampling_from_logits(const void* logits, int64_t logits_stride_row,
                                        int logits_dtype, const float* temperatures,
                                        float temperature, const float* uniform, int mode,
                                        const float* top_k_f, const int32_t* top_k_i,
                                        int top_k_val, const float* top_p_arr, float top_p_val,
                                        int32_t* out, uint8_t* success, int batch_size, int d,
                                        int max_rounds, void* stream) {
  if (mode < 0 || mode > 3 || d <= 0 || logits_stride_row < d) return SGL_ERR_INVALID_ARG;
  if (batch_size == 0) return SGL_OK;
  if (!logits || (!temperatures && !(temperature > 0.f))) return SGL_ERR_INVALID_ARG;
  int esize;
  if (logits_dtype == SGL_DTYPE_BF16 || logits_dtype == SGL_DTYPE_F16) esize = 2;
  else if (logits_dtype == SGL_DTYPE_F32) esize = 4;
  else return SGL_ERR_UNSUPPORTED;
  SampleArgs a = base_args(nullptr, uniform, out, mode == 0 ? nullptr : success, batch_size, d,
                           mode == 0 ? 1 : max_rounds, mode);
  a.logits = logits;
  a.x_st = logits_stride_row;
  a.logit_dtype = logits_dtype;
  a.temps = temperatures;
  a.temp = temperature;
  a.stats_vec = aligned16(logits) && (logits_stride_row * esize) % 16 == 0;
  a.vec = d % 4 == 0 && a.stats_vec;
  if (mode == 1) a.top_k_f = top_k_f;
  if (mode == 3) a.top_k_i = top_k_i;
  a.top_k_val = top_k_val;
  if (mode >= 2) {
    a.top_p_arr = top_p_arr;
    a.top_p_val = top_p_val;
  }
  return launch_sampling(a, stream);
}
