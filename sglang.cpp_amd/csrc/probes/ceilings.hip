// Hardware-ceiling probes for the benchmark harness (libsgl_probes.so).
//
// Not part of the attention path and not behind the drop-in boundary: these
// kernels measure what this MI355X sustains, so the attention kernels'
// fractions of the published peaks can be read against practical ceilings
// measured on the same box, in the same process:
//   * a plain streaming read of device memory (16-byte loads, grid-stride,
//     4, 8 or 16 loads in flight per lane, cached or non-temporal): the HBM
//     ceiling decode and the stores are held against;
//   * a paged read: random 32 KiB pages (one 16-token page of an 8-kv-head
//     bf16 pool), each read whole: the same ceiling for a paged KV stream;
//   * back-to-back v_mfma_f32_32x32x16_bf16 with register operands (four
//     independent accumulator chains per wave, eight waves per CU), once on
//     constant operands and once on random bf16 operands, with the shader
//     clock each ran at (cycle counter over the 100 MHz real-time counter):
//     the matrix-core ceiling prefill is held against, and how far the clock
//     falls under high-toggle matrix work;
//   * a streaming copy (read and write in equal parts), an in-place
//     read-modify-write and a fill, cached or non-temporal: the ceiling of
//     kernels that write as much as they read (the fused store, the
//     residual norm, the Sampler's probabilities);
//   * an empty kernel: the per-launch floor of short calls.
// Apart from the copy probe's destination, the only global writes are a
// guard store that never fires for the read probe (it keeps the loads live)
// and one value plus four clock stamps per workgroup for the MFMA probe.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../common.h"

namespace {

using sgl::bf16x8_t;
using sgl::f32x16_t;
using sgl::u32x4_t;

constexpr int kThreads = 256;

// Grid-stride order (kBlocked false: each load instruction of the grid
// covers one contiguous span) or block-contiguous order (kBlocked true: each
// workgroup walks its own contiguous 1/grid of the buffer).
template <int kDepth, bool kNonTemporal, bool kBlocked>
__global__ void __launch_bounds__(kThreads) stream_read_kernel(const u32x4_t* __restrict__ src,
                                                               int64_t n16,
                                                               uint32_t* __restrict__ sink) {
  int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if constexpr (kBlocked) {
    const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const int64_t b0 = static_cast<int64_t>(blockIdx.x) * per;
    i = b0 + threadIdx.x;
    n16 = min(n16, b0 + per);
    stride = kThreads;
  }
  u32x4_t acc = {0u, 0u, 0u, 0u};
  for (; i + (kDepth - 1) * stride < n16; i += kDepth * stride) {
    u32x4_t v[kDepth];
#pragma unroll
    for (int k = 0; k < kDepth; ++k)
      v[k] = kNonTemporal ? __builtin_nontemporal_load(src + i + k * stride) : src[i + k * stride];
#pragma unroll
    for (int k = 0; k < kDepth; ++k) acc ^= v[k];
  }
  for (; i < n16; i += stride) acc ^= src[i];
  const uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (x == 0x9e3779b9u && (acc[0] + acc[1]) == 0x7f4a7c15u) sink[0] = x;  // never taken in practice
}

// Streaming copy (or, with dst == src, an in-place read-modify-write; with
// kWriteOnly, a fill): block-contiguous, each workgroup walks its own
// contiguous 1/grid of the buffer, kDepth 16-byte loads in flight per lane,
// then the kDepth stores. Loads and stores each cached or non-temporal.
template <int kDepth, bool kNtLoad, bool kNtStore, bool kWriteOnly>
__global__ void __launch_bounds__(kThreads) stream_copy_kernel(const u32x4_t* __restrict__ src,
                                                               u32x4_t* dst, int64_t n16) {
  const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const int64_t b0 = static_cast<int64_t>(blockIdx.x) * per;
  const int64_t end = min(n16, b0 + per);
  int64_t i = b0 + threadIdx.x;
  for (; i + (kDepth - 1) * kThreads < end; i += kDepth * kThreads) {
    u32x4_t v[kDepth];
#pragma unroll
    for (int k = 0; k < kDepth; ++k) {
      if constexpr (kWriteOnly) {
        const uint32_t x = static_cast<uint32_t>(i + k * kThreads);
        v[k] = u32x4_t{x, x ^ 1u, x ^ 2u, x ^ 3u};
      } else {
        v[k] = kNtLoad ? __builtin_nontemporal_load(src + i + k * kThreads) : src[i + k * kThreads];
      }
    }
#pragma unroll
    for (int k = 0; k < kDepth; ++k) {
      v[k] ^= u32x4_t{1u, 0u, 0u, 0u};
      if (kNtStore)
        __builtin_nontemporal_store(v[k], dst + i + k * kThreads);
      else
        dst[i + k * kThreads] = v[k];
    }
  }
  for (; i < end; i += kThreads) {
    u32x4_t v = kWriteOnly ? u32x4_t{0u, 0u, 0u, 0u} : src[i];
    dst[i] = v ^ u32x4_t{1u, 0u, 0u, 0u};
  }
}

// Paged read: workgroup b reads pages order[b * per .. (b + 1) * per) of
// page_bytes each (a multiple of 4 KiB), each page as contiguous 16-byte
// loads, kPages pages in flight (the access pattern of a paged KV stream).
template <int kPages>
__global__ void __launch_bounds__(kThreads) page_read_kernel(const u32x4_t* __restrict__ src,
                                                             const int32_t* __restrict__ order,
                                                             int npages, int page16,
                                                             uint32_t* __restrict__ sink) {
  const int per = (npages + gridDim.x - 1) / gridDim.x;
  const int p0 = blockIdx.x * per;
  const int p1 = min(npages, p0 + per);
  u32x4_t acc = {0u, 0u, 0u, 0u};
  for (int p = p0; p < p1; p += kPages) {
    int pg[kPages];
#pragma unroll
    for (int k = 0; k < kPages; ++k) pg[k] = order[min(p + k, p1 - 1)];
    for (int off = threadIdx.x; off < page16; off += 8 * kThreads) {
      u32x4_t v[kPages][8];
#pragma unroll
      for (int k = 0; k < kPages; ++k)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int o = min(off + j * kThreads, page16 - 1);
          v[k][j] = __builtin_nontemporal_load(src + static_cast<int64_t>(pg[k]) * page16 + o);
        }
#pragma unroll
      for (int k = 0; k < kPages; ++k)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc ^= v[k][j];
    }
  }
  const uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (x == 0x9e3779b9u && (acc[0] + acc[1]) == 0x7f4a7c15u) sink[0] = x;  // never taken in practice
}

// The paged decode's load pattern without its arithmetic: workgroups of 8
// waves (one per kv head of an [slots, 8, 128] bf16 pool) walk a contiguous
// share of a token order (its slots staged in LDS) 16 tokens per step, the
// next step's loads issued
// before the current step's are consumed, a workgroup barrier per step.
// V rows: lane (n, j) reads V[tok 4 j + e][head][8 n .. 8 n + 8] for e < 4
// (whole 256-byte head rows), non-temporal. K by kmode: 0 = the MFMA operand
// mapping (lane (n, j) reads K[tok n][head][32 s + 8 j .. + 8] for s < 4:
// 64-byte pieces, two instructions per 128-byte line), cached; 1 = the same,
// non-temporal; 2 = whole rows like V, non-temporal; 3 = whole rows, cached.
constexpr int kDecodeProbeMaxShare = 8192;

template <int kMode, bool kBarrier, int kDepth>
__global__ void __launch_bounds__(512) decode_read_kernel(const uint16_t* __restrict__ kp,
                                                          const uint16_t* __restrict__ vp,
                                                          const int32_t* order,
                                                          int ntok, uint32_t* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  const int h = threadIdx.x >> 6;
  const int n = lane & 15, j = lane >> 4;
  const int per = ((ntok + gridDim.x - 1) / gridDim.x + 15) / 16 * 16;
  const int t0 = blockIdx.x * per;
  const int t1 = min(ntok, t0 + per);
  constexpr int64_t kRow = 8 * 128;  // elements per slot
  // The share's slots staged in LDS first, as the decode stages a unit's.
  __shared__ int32_t sl[kDecodeProbeMaxShare];
  for (int i = threadIdx.x; i < t1 - t0; i += 512) sl[i] = order[t0 + i];
  __syncthreads();
  order = sl - t0;
  u32x4_t acc = {0u, 0u, 0u, 0u};
  u32x4_t kr[kDepth][4], vr[kDepth][4];
  auto issue = [&](u32x4_t(&kb)[4], u32x4_t(&vb)[4], int tb) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int tv = min(tb + 4 * j + e, t1 - 1);
      const u32x4_t* va =
          reinterpret_cast<const u32x4_t*>(vp + order[tv] * kRow + h * 128 + 8 * n);
      vb[e] = __builtin_nontemporal_load(va);
      if constexpr (kMode >= 2) {
        const u32x4_t* ka =
            reinterpret_cast<const u32x4_t*>(kp + order[tv] * kRow + h * 128 + 8 * n);
        kb[e] = kMode == 2 ? __builtin_nontemporal_load(ka) : *ka;
      } else {
        const int tk = min(tb + n, t1 - 1);
        const u32x4_t* ka =
            reinterpret_cast<const u32x4_t*>(kp + order[tk] * kRow + h * 128 + 32 * e + 8 * j);
        kb[e] = kMode == 1 ? __builtin_nontemporal_load(ka) : *ka;
      }
    }
  };
  // kDepth steps in flight: a ring of register buffers, rotated by unrolling.
  static_assert(kDepth == 2 || kDepth == 3, "depth");
  int tb = t0;
  sgl::static_for<0, kDepth - 1>([&](auto i) {
    if (t0 + 16 * i.value < t1) issue(kr[i.value], vr[i.value], t0 + 16 * i.value);
  });
  while (tb < t1) {
    bool done = false;
    sgl::static_for<0, kDepth>([&](auto i) {
      if (done) return;
      constexpr int cur = i.value;
      constexpr int nxt = (i.value + kDepth - 1) % kDepth;
      if (tb + 16 * (kDepth - 1) < t1) issue(kr[nxt], vr[nxt], tb + 16 * (kDepth - 1));
#pragma unroll
      for (int e = 0; e < 4; ++e) acc ^= kr[cur][e] ^ vr[cur][e];
      if constexpr (kBarrier) __syncthreads();
      tb += 16;
      if (tb >= t1) done = true;
    });
  }
  const uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (x == 0x9e3779b9u && (acc[0] + acc[1]) == 0x7f4a7c15u) sink[0] = x;  // never taken in practice
}

__device__ __forceinline__ uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

// Eight bf16 operands of a lane: uniform in [-2, 2) from a hash of
// (seed, lane, register), or 1.0 everywhere.
__device__ __forceinline__ bf16x8_t operand(bool random, uint32_t seed, uint32_t tag) {
  bf16x8_t v;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float f = 1.0f;
    if (random) {
      const uint32_t h = mix32(seed ^ mix32(tag * 8u + static_cast<uint32_t>(e)));
      f = static_cast<float>(h >> 8) * (4.0f / 16777216.0f) - 2.0f;
    }
    v[e] = static_cast<__bf16>(f);
  }
  return v;
}

// Each wave runs `iters` rounds of 4 MFMAs (4 accumulator chains, the A/B
// pairs rotating so consecutive MFMAs take different operands). Two
// workgroups of four waves per CU: two waves per SIMD.
__global__ void __launch_bounds__(kThreads, 2) mfma_bf16_kernel(int iters, int random,
                                                                 uint32_t seed,
                                                                 float* __restrict__ sink,
                                                                 int64_t* __restrict__ clocks) {
  const uint32_t tid = blockIdx.x * kThreads + threadIdx.x;
  const bool rnd = random != 0;
  const bf16x8_t a0 = operand(rnd, seed, tid * 8u + 0u), a1 = operand(rnd, seed, tid * 8u + 1u);
  const bf16x8_t a2 = operand(rnd, seed, tid * 8u + 2u), a3 = operand(rnd, seed, tid * 8u + 3u);
  const bf16x8_t b0 = operand(rnd, seed, tid * 8u + 4u), b1 = operand(rnd, seed, tid * 8u + 5u);
  const bf16x8_t b2 = operand(rnd, seed, tid * 8u + 6u), b3 = operand(rnd, seed, tid * 8u + 7u);
  f32x16_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
  __syncthreads();
  const int64_t t0 = clock64();
  const int64_t r0 = wall_clock64();
  for (int it = 0; it < iters; it += 2) {
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a2, b2, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a3, b3, c3, 0, 0, 0);
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b2, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a2, b3, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a3, b0, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b1, c3, 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 16; ++e) s += c0[e] + c1[e] + c2[e] + c3[e];
  __syncthreads();
  const int64_t t1 = clock64();
  const int64_t r1 = wall_clock64();
  if (threadIdx.x == 0) {
    clocks[blockIdx.x * 4 + 0] = t0;
    clocks[blockIdx.x * 4 + 1] = t1;
    clocks[blockIdx.x * 4 + 2] = r0;
    clocks[blockIdx.x * 4 + 3] = r1;
  }
  if (threadIdx.x == 0) sink[blockIdx.x] = s;
}

__global__ void empty_kernel() {}

int status_of_launch() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : static_cast<int>(e);
}

}  // namespace

// Streams `bytes` (a multiple of 16, 16-byte aligned) from src with `grid`
// workgroups of 256 threads; variant: bit 0 = non-temporal loads, bits 1-2 =
// loads in flight per lane (0: 4, 1: 8, 2: 16), bit 3 = block-contiguous
// order. sink: one writable uint32
// (written only if the data hash hits a fixed 64-bit pattern).
extern "C" int sgl_probe_stream_read(const void* src, int64_t bytes, int grid, int variant,
                                     void* sink, void* stream) {
  if (!src || !sink || bytes <= 0 || bytes % 16 || grid <= 0 || variant < 0 || variant > 13 || (variant & 6) == 6 ||
      reinterpret_cast<uintptr_t>(src) % 16)
    return SGL_ERR_INVALID_ARG;
  const auto* p = static_cast<const u32x4_t*>(src);
  auto* k = static_cast<uint32_t*>(sink);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t n = bytes / 16;
#define SGL_PROBE_READ(D_, NT_, B_)                                                          \
  hipLaunchKernelGGL((stream_read_kernel<D_, NT_, B_>), dim3(grid), dim3(kThreads), 0, s, p, n, k)
  const bool nt = variant & 1, blocked = variant & 8;
  const int depth = 4 << ((variant >> 1) & 3);
  if (blocked) {
    if (depth == 4) { if (nt) SGL_PROBE_READ(4, true, true); else SGL_PROBE_READ(4, false, true); }
    else if (depth == 8) { if (nt) SGL_PROBE_READ(8, true, true); else SGL_PROBE_READ(8, false, true); }
    else { if (nt) SGL_PROBE_READ(16, true, true); else SGL_PROBE_READ(16, false, true); }
  } else {
    if (depth == 4) { if (nt) SGL_PROBE_READ(4, true, false); else SGL_PROBE_READ(4, false, false); }
    else if (depth == 8) { if (nt) SGL_PROBE_READ(8, true, false); else SGL_PROBE_READ(8, false, false); }
    else { if (nt) SGL_PROBE_READ(16, true, false); else SGL_PROBE_READ(16, false, false); }
  }
#undef SGL_PROBE_READ
  return status_of_launch();
}

// Streams `bytes` (a multiple of 16, 16-byte aligned) from src to dst with
// `grid` workgroups of 256 threads; dst == src is an in-place
// read-modify-write. variant: bit 0 = non-temporal loads, bit 1 =
// non-temporal stores, bit 2 = 16 rather than 8 accesses in flight per lane,
// bit 3 = write only (a fill of dst; src unused and may be null).
extern "C" int sgl_probe_stream_copy(const void* src, void* dst, int64_t bytes, int grid,
                                     int variant, void* stream) {
  const bool write_only = variant & 8;
  if ((!src && !write_only) || !dst || bytes <= 0 || bytes % 16 || grid <= 0 || variant < 0 ||
      variant > 15 || reinterpret_cast<uintptr_t>(dst) % 16 ||
      reinterpret_cast<uintptr_t>(src) % 16)
    return SGL_ERR_INVALID_ARG;
  const auto* p = static_cast<const u32x4_t*>(src);
  auto* q = static_cast<u32x4_t*>(dst);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t n = bytes / 16;
#define SGL_PROBE_COPY(D_, L_, S_, W_) \
  hipLaunchKernelGGL((stream_copy_kernel<D_, L_, S_, W_>), dim3(grid), dim3(kThreads), 0, s, p, q, n)
#define SGL_PROBE_COPY_D(L_, S_, W_) \
  if (variant & 4) SGL_PROBE_COPY(16, L_, S_, W_); else SGL_PROBE_COPY(8, L_, S_, W_);
  if (write_only) {
    if (variant & 2) { SGL_PROBE_COPY_D(false, true, true) } else { SGL_PROBE_COPY_D(false, false, true) }
  } else {
    switch (variant & 3) {
      case 0: SGL_PROBE_COPY_D(false, false, false) break;
      case 1: SGL_PROBE_COPY_D(true, false, false) break;
      case 2: SGL_PROBE_COPY_D(false, true, false) break;
      default: SGL_PROBE_COPY_D(true, true, false) break;
    }
  }
#undef SGL_PROBE_COPY_D
#undef SGL_PROBE_COPY
  return status_of_launch();
}

// Reads npages pages of page_bytes (a multiple of 4096) from src in the
// order given by `order` (device int32 [npages]), `grid` workgroups each
// walking a contiguous share of that order, pages_in_flight (1 or 2) pages at
// a time per workgroup.
extern "C" int sgl_probe_page_read(const void* src, const int32_t* order, int npages,
                                   int64_t page_bytes, int grid, int pages_in_flight, void* sink,
                                   void* stream) {
  if (!src || !order || !sink || npages <= 0 || grid <= 0 || page_bytes <= 0 ||
      page_bytes % 4096 || page_bytes / 16 > 0x7fffffff || (pages_in_flight != 1 && pages_in_flight != 2) ||
      reinterpret_cast<uintptr_t>(src) % 16)
    return SGL_ERR_INVALID_ARG;
  const auto* p = static_cast<const u32x4_t*>(src);
  auto* k = static_cast<uint32_t*>(sink);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int page16 = static_cast<int>(page_bytes / 16);
  if (pages_in_flight == 1)
    hipLaunchKernelGGL((page_read_kernel<1>), dim3(grid), dim3(kThreads), 0, s, p, order, npages, page16, k);
  else
    hipLaunchKernelGGL((page_read_kernel<2>), dim3(grid), dim3(kThreads), 0, s, p, order, npages, page16, k);
  return status_of_launch();
}

// The decode's load pattern over K and V pools of `slots` slots each
// ([slots, 8, 128] bf16), tokens in the order `order` (device int32
// [ntok], slot of each token), `grid` workgroups of 8 waves; kmode as
// decode_read_kernel; barrier: a workgroup barrier per step; depth: steps
// of loads in flight (2 or 3).
extern "C" int sgl_probe_decode_read(const void* k_pool, const void* v_pool, const int32_t* order,
                                     int ntok, int grid, int kmode, int barrier, int depth,
                                     void* sink, void* stream) {
  if (!k_pool || !v_pool || !order || !sink || ntok <= 0 || grid <= 0 || kmode < 0 ||
      kmode > 3 || (depth != 2 && depth != 3))
    return SGL_ERR_INVALID_ARG;
  const int64_t per = ((static_cast<int64_t>(ntok) + grid - 1) / grid + 15) / 16 * 16;
  if (per > kDecodeProbeMaxShare) return SGL_ERR_CAPACITY;
  const auto* kp = static_cast<const uint16_t*>(k_pool);
  const auto* vp = static_cast<const uint16_t*>(v_pool);
  auto* k = static_cast<uint32_t*>(sink);
  hipStream_t s = static_cast<hipStream_t>(stream);
#define SGL_PROBE_DEC(M_, B_, D_) \
  hipLaunchKernelGGL((decode_read_kernel<M_, B_, D_>), dim3(grid), dim3(512), 0, s, kp, vp, order, ntok, k)
#define SGL_PROBE_DEC_BD(M_)                                   \
  if (barrier && depth == 2) SGL_PROBE_DEC(M_, true, 2);       \
  else if (barrier) SGL_PROBE_DEC(M_, true, 3);                \
  else if (depth == 2) SGL_PROBE_DEC(M_, false, 2);            \
  else SGL_PROBE_DEC(M_, false, 3);
  switch (kmode) {
    case 0: SGL_PROBE_DEC_BD(0) break;
    case 1: SGL_PROBE_DEC_BD(1) break;
    case 2: SGL_PROBE_DEC_BD(2) break;
    default: SGL_PROBE_DEC_BD(3) break;
  }
#undef SGL_PROBE_DEC_BD
#undef SGL_PROBE_DEC
  return status_of_launch();
}

// grid workgroups of 4 waves, each wave `iters` (even) MFMAs per chain, 4
// chains: grid * 4 * iters * 4 * 32768 flops. sink: grid floats;
// clocks: grid * 4 int64 (cycle counter start/end, 100 MHz real time
// start/end, per workgroup).
extern "C" int sgl_probe_mfma_bf16(int grid, int iters, int random_operands, uint32_t seed,
                                   float* sink, int64_t* clocks, void* stream) {
  if (grid <= 0 || iters <= 0 || iters % 2 || !sink || !clocks) return SGL_ERR_INVALID_ARG;
  hipLaunchKernelGGL(mfma_bf16_kernel, dim3(grid), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), iters, random_operands, seed, sink, clocks);
  return status_of_launch();
}

extern "C" int sgl_probe_empty(int grid, int block, void* stream) {
  if (grid <= 0 || block <= 0 || block > 1024) return SGL_ERR_INVALID_ARG;
  hipLaunchKernelGGL(empty_kernel, dim3(grid), dim3(block), 0, static_cast<hipStream_t>(stream));
  return status_of_launch();
}
