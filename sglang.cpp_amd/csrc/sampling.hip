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
// cut into blocks of 256 probabilities, one coalesced 16-byte load per lane
// of a wave; waves take blocks round-robin. A sweep with a threshold
// leaves in LDS the mass above it of every block (one wave reduction per
// block) and the row's count above it. A draw scans the block masses
// across the workgroup (each thread a run of consecutive blocks, then a
// wave scan and the wave totals through LDS) to the block holding the
// crossing, and one wave scans that block's 256 probabilities to the first
// crossing index. A rejection round is one sweep: the sweep that counts the
// probabilities above the new pivot also gives the next draw its block
// masses. A vocabulary row (Qwen3: 151,936 x 4 B) comes from HBM on the
// first sweep and from L2 afterwards.
#include <math.h>

#include "common.h"

namespace sgl {
namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / kWave;
constexpr int kVec = 4;
constexpr int kBlock = kWave * kVec;  // probabilities per block
constexpr int kMaxBlocks = 8192;      // rows up to 2M probabilities (32 KiB of block masses)

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
};

struct Shared {
  float blk[kMaxBlocks];  // mass above the current threshold, per block
  float wave_f[kWaves];
  int wave_i[kWaves];
  float wave_run[kWaves];  // draw: mass before the crossing block found by a wave
  float total;            // row mass above the threshold
  int count;              // row count above the threshold
  int blk_star;
  int sampled;
};

__device__ __forceinline__ void load4(const float* row, int e0, int d, bool vec, float (&p)[kVec]) {
  if (vec && e0 + kVec <= d) {
    const f32x4_t v = *reinterpret_cast<const f32x4_t*>(row + e0);
#pragma unroll
    for (int j = 0; j < kVec; ++j) p[j] = v[j];
  } else {
#pragma unroll
    for (int j = 0; j < kVec; ++j) p[j] = e0 + j < d ? row[e0 + j] : 0.f;
  }
}

__device__ __forceinline__ float wave_sum_f(float x) {
  return sum_xor32(sum_xor16(group_sum<16>(x)));
}
__device__ __forceinline__ int wave_sum_i(int x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, kWave);
  return x;
}

// Inclusive scan over the 64 lanes of a wave.
__device__ __forceinline__ float wave_inclusive_scan(float x, int lane) {
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const float y = __shfl_up(x, off, kWave);
    if (lane >= off) x += y;
  }
  return x;
}

// Block masses, row mass and row count of the probabilities above thr.
__device__ void sweep(const float* row, int d, bool vec, float thr, Shared& sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nblk = (d + kBlock - 1) / kBlock;
  float wm = 0.f;
  int wn = 0;
  __syncthreads();  // the previous readers of sh are done
  // Four blocks per iteration: their loads are in flight together.
  constexpr int kUnroll = 4;
  for (int b = wave; b < nblk; b += kWaves * kUnroll) {
    float p[kUnroll][kVec];
#pragma unroll
    for (int x = 0; x < kUnroll; ++x) {
      const int bx = b + x * kWaves;
      if (bx < nblk) load4(row, bx * kBlock + lane * kVec, d, vec, p[x]);
    }
#pragma unroll
    for (int x = 0; x < kUnroll; ++x) {
      const int bx = b + x * kWaves;
      if (bx >= nblk) break;
      float m = 0.f;
      int n = 0;
#pragma unroll
      for (int j = 0; j < kVec; ++j)
        if (p[x][j] > thr) {
          m += p[x][j];
          ++n;
        }
      m = wave_sum_f(m);
      wn += n;
      wm += m;
      if (lane == 0) sh.blk[bx] = m;
    }
  }
  wn = wave_sum_i(wn);
  if (lane == 0) {
    sh.wave_f[wave] = wm;
    sh.wave_i[wave] = wn;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
    int c = 0;
    for (int w = 0; w < kWaves; ++w) {
      t += sh.wave_f[w];
      c += sh.wave_i[w];
    }
    sh.total = t;
    sh.count = c;
  }
  __syncthreads();
}

// The inverse-CDF draw over the probabilities above thr with target u,
// from the block masses of the last sweep with the same threshold.
__device__ int draw(const float* row, int d, bool vec, float thr, float u, Shared& sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nblk = (d + kBlock - 1) / kBlock;
  // Thread t owns blocks [t G, (t + 1) G).
  const int G = (nblk + kThreads - 1) / kThreads;
  const int b0 = min(nblk, static_cast<int>(threadIdx.x) * G), b1 = min(nblk, b0 + G);
  float own = 0.f;
  for (int b = b0; b < b1; ++b) own += sh.blk[b];
  const float incl = wave_inclusive_scan(own, lane);
  if (threadIdx.x == 0) {
    sh.blk_star = nblk;
    sh.sampled = d - 1;
  }
  if (lane == 63) sh.wave_f[wave] = incl;
  __syncthreads();
  float before = 0.f;
  for (int w = 0; w < wave; ++w) before += sh.wave_f[w];
  // The first thread whose run crosses u walks its run to the crossing block.
  float run = before + (incl - own);
  bool cross = run + own > u;
  const uint64_t ballot = __ballot(cross);
  const bool first_in_wave = cross && lane == __builtin_ctzll(ballot);
  if (first_in_wave) {
    int bs = b1 - 1;
    for (int b = b0; b < b1; ++b) {
      if (run + sh.blk[b] > u) {
        bs = b;
        break;
      }
      run += sh.blk[b];
    }
    sh.wave_i[wave] = bs;
    sh.wave_run[wave] = run;  // mass before block bs
  } else if (lane == 0 && ballot == 0) {
    sh.wave_i[wave] = nblk;
  }
  __syncthreads();
  int bs = nblk;
  float base = 0.f;
  for (int w = 0; w < kWaves; ++w)
    if (sh.wave_i[w] < nblk) {
      bs = sh.wave_i[w];
      base = sh.wave_run[w];
      break;
    }
  // One wave scans the crossing block.
  if (bs < nblk && wave == 0) {
    const int e0 = bs * kBlock + lane * kVec;
    float p[kVec], m[kVec];
    load4(row, e0, d, vec, p);
    float local = 0.f;
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      m[j] = p[j] > thr ? p[j] : 0.f;
      local += m[j];
    }
    const float cincl = wave_inclusive_scan(local, lane);
    float cdf = base + (cincl - local);
    int first = d, last_valid = -1;
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      cdf += m[j];
      const bool valid = p[j] > thr && e0 + j < d;
      if (valid) last_valid = e0 + j;
      if (valid && cdf > u && first == d) first = e0 + j;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      first = min(first, __shfl_xor(first, off, kWave));
      last_valid = max(last_valid, __shfl_xor(last_valid, off, kWave));
    }
    // Rounding inside the block may miss u: then its last candidate.
    if (lane == 0) sh.sampled = first < d ? first : (last_valid >= 0 ? last_valid : d - 1);
  }
  __syncthreads();
  return sh.sampled;
}

__global__ void __launch_bounds__(kThreads) sampling_kernel(SampleArgs a) {
  __shared__ Shared sh;
  const int row_id = blockIdx.x;
  const float* row = a.probs + static_cast<int64_t>(row_id) * a.d;
  sweep(row, a.d, a.vec, 0.f, sh);
  if (a.mode == 0) {
    const int s = draw(row, a.d, a.vec, 0.f, a.uniform[row_id], sh);
    if (threadIdx.x == 0) a.out[row_id] = s;
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
    const float u = a.uniform[static_cast<int64_t>(r) * a.batch + row_id] * q;
    sampled = draw(row, a.d, a.vec, pivot, u, sh);
    const float ps = row[sampled];
    if (ps > pivot) {
      pivot = ps;
      sweep(row, a.d, a.vec, pivot, sh);  // masses above the new pivot
    }
    q = sh.total;
    const int count = sh.count;
    if (a.mode == 1) accepted = static_cast<uint32_t>(count) < static_cast<uint32_t>(k);
    else if (a.mode == 2) accepted = q < top_p;
    else accepted = count < k && q < top_p;
    if (accepted) break;
  }
  if (threadIdx.x == 0) {
    a.out[row_id] = sampled;
    if (a.success) a.success[row_id] = accepted ? 1 : 0;
  }
}

int launch_sampling(const SampleArgs& a, void* stream) {
  if (a.batch < 0 || a.d <= 0 || (a.mode != 0 && a.rounds <= 0)) return SGL_ERR_INVALID_ARG;
  if ((static_cast<int64_t>(a.d) + kBlock - 1) / kBlock > kMaxBlocks) return SGL_ERR_UNSUPPORTED;
  if (a.batch == 0) return SGL_OK;
  if (!a.probs || !a.uniform || !a.out) return SGL_ERR_INVALID_ARG;
  hipLaunchKernelGGL(sampling_kernel, dim3(a.batch), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), a);
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
