// Page-table and token-pool plumbing (integer gathers and scatters).
//
// Reference: build_decode_indices_kernel (src/attention/flashinfer_backend.cu:43-70),
// write_token_pool_kernel / gather_int32_2d_kernel (src/kernels/token_pool.cu:10-49).
// The page table is token-granular: row r, column p holds the pool slot of
// request r's p-th token.
#include <algorithm>

#include "common.h"

namespace sgl {
namespace {

// kBlocksPerRequest workgroups per request stride over its run; a thread
// moves 4 consecutive slots (one 16-byte load from the table row, whose
// start is 16-byte aligned when the row stride is a multiple of 4), so a
// 32K-token request is spread over several CUs instead of one.
constexpr int kBlocksPerRequest = 8;

__global__ void __launch_bounds__(256) build_indices_kernel(
    const int32_t* __restrict__ page_table, int64_t rows, int64_t stride, int64_t cols,
    const int32_t* __restrict__ table_indices, const int32_t* __restrict__ kv_indptr,
    int32_t* __restrict__ indices, int batch_size, bool vec) {
  const int r = blockIdx.y;
  if (r >= batch_size) return;
  const int32_t row = table_indices[r];
  const int32_t start = kv_indptr[r];
  const int32_t len = kv_indptr[r + 1] - start;
  if (row < 0 || row >= rows || len <= 0) return;
  const int32_t* src = page_table + static_cast<int64_t>(row) * stride;
  int32_t* dst = indices + start;
  for (int32_t p = (blockIdx.x * blockDim.x + threadIdx.x) * 4; p < len;
       p += kBlocksPerRequest * blockDim.x * 4) {
    if (vec && p + 4 <= cols) {
      const u32x4_t v = ldg128(src + p);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (p + i < len) dst[p + i] = static_cast<int32_t>(v[i]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (p + i < len) dst[p + i] = p + i < cols ? src[p + i] : 0;
    }
  }
}

__global__ void __launch_bounds__(256) write_token_pool_kernel(
    int32_t* __restrict__ pool, int64_t rows, int64_t stride, int64_t cols,
    const int32_t* __restrict__ req_indices, const int32_t* __restrict__ positions,
    const int32_t* __restrict__ tokens, int64_t count) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= count) return;
  const int64_t r = req_indices[i];
  const int64_t p = positions[i];
  if (r < 0 || r >= rows || p < 0 || p >= cols) return;
  pool[r * stride + p] = tokens[i];
}

__global__ void __launch_bounds__(256) gather_int32_2d_kernel(
    const int32_t* __restrict__ table, int64_t rows, int64_t stride, int64_t cols,
    const int32_t* __restrict__ req_indices, const int32_t* __restrict__ positions,
    int32_t* __restrict__ out, int64_t count) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= count) return;
  const int64_t r = req_indices[i];
  const int64_t p = positions[i];
  out[i] = (r >= 0 && r < rows && p >= 0 && p < cols) ? table[r * stride + p] : 0;
}

// Several int32 copies in one launch (the capture buffers of a replayed
// step); every workgroup strides over each entry in turn, 16 bytes per lane
// where source and destination allow it.
struct CopyArgs {
  sgl_i32_copy_t c[SGL_MAX_I32_COPIES];
  int n;
};

__global__ void __launch_bounds__(256) copy_i32_kernel(CopyArgs a) {
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int j = 0; j < a.n; ++j) {
    const int32_t* src = a.c[j].src;
    int32_t* dst = a.c[j].dst;
    const int64_t n = a.c[j].count;
    const bool vec = ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0;
    int64_t head = 0;
    if (vec) {
      head = n / 4 * 4;
      for (int64_t i = tid * 4; i < head; i += stride * 4) stg128(dst + i, ldg128(src + i));
    }
    for (int64_t i = head + tid; i < n; i += stride) dst[i] = src[i];
  }
}

// Page allocation -> token-granular page table. Allocation a = (row,
// first_page, last_page) takes page starts [pre[a], pre[a+1]) of the batch's
// allocated pages, pre the exclusive prefix sum of last - first. Each block
// rebuilds pre in LDS (a few hundred allocations at most per scheduler
// step), then each thread takes one token of the flattened page list: page
// k = t / P of allocation a (binary search on pre) writes slot
// page_starts[k] + t % P at column (first_page + k - pre[a]) * P + t % P of
// its row -- P consecutive columns per page, so a wave writes whole pages.
constexpr int kMaxAllocs = 8192;

__global__ void __launch_bounds__(256) write_page_table_kernel(
    int32_t* __restrict__ table, int64_t rows, int64_t stride, int64_t cols,
    const int32_t* __restrict__ page_starts, int64_t num_pages,
    const int32_t* __restrict__ alloc, int n_alloc, int page_size) {
  __shared__ int32_t pre[kMaxAllocs + 1];
  __shared__ int32_t part[256];
  const int t = threadIdx.x;
  // Per-thread runs of allocations, then a serial scan of the 256 run sums.
  const int per = (n_alloc + 255) / 256;
  const int a0 = min(n_alloc, t * per), a1 = min(n_alloc, a0 + per);
  int32_t run = 0;
  for (int a = a0; a < a1; ++a) run += max(0, alloc[3 * a + 2] - alloc[3 * a + 1]);
  part[t] = run;
  __syncthreads();
  if (t == 0) {
    int32_t acc = 0;
    for (int i = 0; i < 256; ++i) {
      const int32_t v = part[i];
      part[i] = acc;
      acc += v;
    }
    pre[n_alloc] = acc;
  }
  __syncthreads();
  run = part[t];
  for (int a = a0; a < a1; ++a) {
    pre[a] = run;
    run += max(0, alloc[3 * a + 2] - alloc[3 * a + 1]);
  }
  __syncthreads();
  const int64_t count = num_pages * page_size;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + t; i < count;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t k = i / page_size;
    const int off = static_cast<int>(i - k * page_size);
    if (k >= pre[n_alloc]) continue;  // more page starts than the allocations take
    int lo = 0, hi = n_alloc - 1;     // last a with pre[a] <= k
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (pre[mid] <= k) lo = mid; else hi = mid - 1;
    }
    const int64_t r = alloc[3 * lo];
    const int64_t col = (static_cast<int64_t>(alloc[3 * lo + 1]) + (k - pre[lo])) * page_size + off;
    if (r < 0 || r >= rows || col < 0 || col >= cols) continue;
    table[r * stride + col] = page_starts[k] + off;
  }
}

int launch_build_indices(const int32_t* page_table, int64_t rows, int64_t stride, int64_t cols,
                         const int32_t* table_indices, const int32_t* kv_indptr,
                         int32_t* indices, int batch_size, void* stream) {
  if (batch_size < 0 || rows < 0 || cols < 0 || stride < cols) return SGL_ERR_INVALID_ARG;
  if (batch_size == 0) return SGL_OK;
  if (!page_table || !table_indices || !kv_indptr || !indices) return SGL_ERR_INVALID_ARG;
  hipLaunchKernelGGL(build_indices_kernel, dim3(kBlocksPerRequest, batch_size), dim3(256), 0,
                     static_cast<hipStream_t>(stream), page_table, rows, stride, cols,
                     table_indices, kv_indptr, indices, batch_size,
                     (stride & 3) == 0 && aligned16(page_table));
  return launch_status();
}

}  // namespace
}  // namespace sgl

extern "C" int sgl_build_decode_indices(const int32_t* page_table, int64_t rows, int64_t stride,
                                        int64_t cols, const int32_t* table_indices,
                                        const int32_t* kv_indptr, int32_t* indices,
                                        int batch_size, void* stream) {
  return sgl::launch_build_indices(page_table, rows, stride, cols, table_indices, kv_indptr,
                                   indices, batch_size, stream);
}

extern "C" int sgl_build_prefill_indices(const int32_t* page_table, int64_t rows, int64_t stride,
                                         int64_t cols, const int32_t* table_indices,
                                         const int32_t* kv_indptr, int32_t* indices,
                                         int batch_size, void* stream) {
  return sgl::launch_build_indices(page_table, rows, stride, cols, table_indices, kv_indptr,
                                   indices, batch_size, stream);
}

extern "C" int sgl_write_token_pool(int32_t* pool, int64_t rows, int64_t stride, int64_t cols,
                                    const int32_t* req_indices, const int32_t* positions,
                                    const int32_t* tokens, int64_t count, void* stream) {
  if (count < 0 || rows < 0 || cols < 0 || stride < cols) return SGL_ERR_INVALID_ARG;
  if (count == 0) return SGL_OK;
  if (!pool || !req_indices || !positions || !tokens) return SGL_ERR_INVALID_ARG;
  const int64_t blocks = (count + 255) / 256;
  hipLaunchKernelGGL(sgl::write_token_pool_kernel, dim3(blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), pool, rows, stride, cols, req_indices,
                     positions, tokens, count);
  return sgl::launch_status();
}

extern "C" int sgl_gather_int32_2d(const int32_t* table, int64_t rows, int64_t stride,
                                   int64_t cols, const int32_t* req_indices,
                                   const int32_t* positions, int32_t* out, int64_t count,
                                   void* stream) {
  if (count < 0 || rows < 0 || cols < 0 || stride < cols) return SGL_ERR_INVALID_ARG;
  if (count == 0) return SGL_OK;
  if (!table || !req_indices || !positions || !out) return SGL_ERR_INVALID_ARG;
  const int64_t blocks = (count + 255) / 256;
  hipLaunchKernelGGL(sgl::gather_int32_2d_kernel, dim3(blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), table, rows, stride, cols, req_indices,
                     positions, out, count);
  return sgl::launch_status();
}

extern "C" int sgl_write_page_table(int32_t* page_table, int64_t rows, int64_t stride,
                                    int64_t cols, const int32_t* page_starts, int64_t num_pages,
                                    const int32_t* alloc_info, int num_allocs, int page_size,
                                    void* stream) {
  if (num_pages < 0 || num_allocs < 0 || page_size <= 0 || rows < 0 || cols < 0 ||
      stride < cols)
    return SGL_ERR_INVALID_ARG;
  if (num_pages == 0 || num_allocs == 0) return SGL_OK;
  if (!page_table || !page_starts || !alloc_info) return SGL_ERR_INVALID_ARG;
  if (num_allocs > sgl::kMaxAllocs) return SGL_ERR_UNSUPPORTED;
  const int64_t count = num_pages * page_size;
  if (count > (int64_t{1} << 40)) return SGL_ERR_INVALID_ARG;
  const int64_t blocks = std::min<int64_t>((count + 255) / 256, 4096);
  hipLaunchKernelGGL(sgl::write_page_table_kernel, dim3(static_cast<uint32_t>(blocks)),
                     dim3(256), 0, static_cast<hipStream_t>(stream), page_table, rows, stride,
                     cols, page_starts, num_pages, alloc_info, num_allocs, page_size);
  return sgl::launch_status();
}

extern "C" int sgl_copy_i32(const sgl_i32_copy_t* copies, int num_copies, void* stream) {
  if (num_copies < 0 || num_copies > SGL_MAX_I32_COPIES || (num_copies > 0 && !copies))
    return SGL_ERR_INVALID_ARG;
  sgl::CopyArgs a{};
  int64_t most = 0;
  for (int j = 0; j < num_copies; ++j) {
    const sgl_i32_copy_t& c = copies[j];
    if (c.count < 0 || (c.count > 0 && (!c.src || !c.dst))) return SGL_ERR_INVALID_ARG;
    if (c.count == 0) continue;
    a.c[a.n++] = c;
    most = std::max(most, c.count);
  }
  if (a.n == 0) return SGL_OK;
  const int64_t blocks = std::min<int64_t>(1024, (most + 1023) / 1024);
  hipLaunchKernelGGL(sgl::copy_i32_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return sgl::launch_status();
}

extern "C" const char* sgl_status_string(int status) {
  switch (status) {
    case SGL_OK: return "ok";
    case SGL_ERR_INVALID_ARG: return "invalid argument";
    case SGL_ERR_UNSUPPORTED: return "unsupported configuration";
    case SGL_ERR_CAPACITY: return "workspace or plan capacity exceeded";
    case SGL_ERR_ALIGNMENT: return "pointer or stride misaligned";
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown status";
}

extern "C" int sgl_abi_version(void) { return SGL_ABI_VERSION; }
