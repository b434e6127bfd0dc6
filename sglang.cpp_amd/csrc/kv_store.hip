// KV-cache scatter store: k_cache[out_loc[t]] = k[t], v_cache[out_loc[t]] = v[t].
//
// Reference semantics: store_kv_cache_kernel (src/kvcache/mha_kvcache.cu:13-41)
// copies one token row per 32-lane warp with 2-byte scalar copies. Here each
// lane moves one 16-byte chunk of K and one of V, so a wave64 covers 1 KiB of
// a row per instruction and every HBM transaction is a full 128-bit access.
// The copy is bitwise, so bf16 and fp16 share the kernel.
#include "common.h"

namespace sgl {
namespace {

template <typename index_t>
__global__ void __launch_bounds__(256) store_kv_vec_kernel(
    uint8_t* __restrict__ k_cache, uint8_t* __restrict__ v_cache,
    const uint8_t* __restrict__ k, const uint8_t* __restrict__ v,
    const index_t* __restrict__ out_loc, int64_t num_tokens,
    int64_t chunks_per_token, int64_t row_bytes, int64_t k_stride_bytes,
    int64_t v_stride_bytes) {
  const int64_t total = num_tokens * chunks_per_token;
  const int64_t step = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += step) {
    const int64_t t = i / chunks_per_token;
    const int64_t c = i - t * chunks_per_token;
    const int64_t slot = static_cast<int64_t>(out_loc[t]);
    const u32x4_t kv = ldg128(k + t * k_stride_bytes + c * 16);
    const u32x4_t vv = ldg128(v + t * v_stride_bytes + c * 16);
    stg128(k_cache + slot * row_bytes + c * 16, kv);
    stg128(v_cache + slot * row_bytes + c * 16, vv);
  }
}

// Fallback for rows or strides that are not 16-byte multiples.
template <typename index_t>
__global__ void __launch_bounds__(256) store_kv_scalar_kernel(
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const index_t* __restrict__ out_loc, int64_t num_tokens, int64_t elems,
    int64_t k_stride, int64_t v_stride) {
  const int64_t total = num_tokens * elems;
  const int64_t step = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += step) {
    const int64_t t = i / elems;
    const int64_t e = i - t * elems;
    const int64_t slot = static_cast<int64_t>(out_loc[t]);
    k_cache[slot * elems + e] = k[t * k_stride + e];
    v_cache[slot * elems + e] = v[t * v_stride + e];
  }
}

template <typename index_t>
int launch_store(void* k_cache, void* v_cache, const void* k, const void* v,
                 const void* out_loc, int64_t num_tokens, int64_t elems,
                 int64_t k_stride, int64_t v_stride, hipStream_t stream) {
  const bool vec = (elems % 8 == 0) && (k_stride % 8 == 0) && (v_stride % 8 == 0) &&
                   aligned16(k_cache) && aligned16(v_cache) && aligned16(k) && aligned16(v);
  constexpr int threads = 256;
  const int64_t max_blocks = 256 * 32;  // 32 waves-worth of blocks per CU, then grid-stride
  if (vec) {
    const int64_t cpt = elems / 8;
    int64_t blocks = (num_tokens * cpt + threads - 1) / threads;
    if (blocks > max_blocks) blocks = max_blocks;
    hipLaunchKernelGGL(store_kv_vec_kernel<index_t>, dim3(blocks), dim3(threads), 0, stream,
                       static_cast<uint8_t*>(k_cache), static_cast<uint8_t*>(v_cache),
                       static_cast<const uint8_t*>(k), static_cast<const uint8_t*>(v),
                       static_cast<const index_t*>(out_loc), num_tokens, cpt, elems * 2,
                       k_stride * 2, v_stride * 2);
  } else {
    int64_t blocks = (num_tokens * elems + threads - 1) / threads;
    if (blocks > max_blocks) blocks = max_blocks;
    hipLaunchKernelGGL(store_kv_scalar_kernel<index_t>, dim3(blocks), dim3(threads), 0, stream,
                       static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache),
                       static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
                       static_cast<const index_t*>(out_loc), num_tokens, elems, k_stride,
                       v_stride);
  }
  return launch_status();
}

}  // namespace
}  // namespace sgl

extern "C" int sgl_store_kv(void* k_cache, void* v_cache, const void* k, const void* v,
                            const void* out_loc, int index_dtype, int64_t num_tokens,
                            int64_t elems_per_token, int64_t k_stride_token,
                            int64_t v_stride_token, void* stream) {
  if (num_tokens < 0 || elems_per_token <= 0) return SGL_ERR_INVALID_ARG;
  if (num_tokens == 0) return SGL_OK;
  if (!k_cache || !v_cache || !k || !v || !out_loc) return SGL_ERR_INVALID_ARG;
  if (k_stride_token < elems_per_token || v_stride_token < elems_per_token)
    return SGL_ERR_INVALID_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (index_dtype == SGL_INDEX_I32)
    return sgl::launch_store<int32_t>(k_cache, v_cache, k, v, out_loc, num_tokens,
                                      elems_per_token, k_stride_token, v_stride_token, s);
  if (index_dtype == SGL_INDEX_I64)
    return sgl::launch_store<int64_t>(k_cache, v_cache, k, v, out_loc, num_tokens,
                                      elems_per_token, k_stride_token, v_stride_token, s);
  return SGL_ERR_UNSUPPORTED;
}
