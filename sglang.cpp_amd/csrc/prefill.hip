// Paged causal prefill (ragged, prefix-cache aware) on gfx950 matrix cores.
//
// Reference semantics: FlashInferBackend::forward, prefill branch
// (src/attention/flashinfer_backend.cu:596-679) with MaskMode::kCausal:
// query i of request r (qo_len q_r, kv_len k_r) attends kv token j iff
// j <= i + (k_r - q_r) (bottom-right alignment, so cached prefix tokens are
// visible to every new token), kv slots taken from the token-granular
// indices[kv_indptr[r] + j].
//
// Work decomposition: one workgroup (4 or 8 waves, 32 query rows each) per
// (request, kv head, query tile), or per pair of tiles from both ends of the
// causal range (see paged_prefill_kernel). The G query heads that share a kv
// head are packed row-wise (packed row p -> token p / G, head h G + p % G),
// so each K/V tile staged in LDS feeds G heads. K/V tiles of 64 tokens are
// gathered from the pool (one 16-byte chunk per lane, slots from the index
// list) into a double-buffered LDS ring; the gathers of the next tiles are
// in flight while the current one is on the matrix cores.
//
// Matrix formulation (v_mfma_f32_32x32x16_bf16, lane l, c = l % 32, hl = l / 32):
//   S^T[tok, row] = K[tok, :] . Q[row, :]      (A = K from LDS, B = Q^T in VGPRs)
//   O^T[d, row]  += V^T[d, tok] . P^T[tok, row] (A = V^T by LDS transpose reads)
// The query row sits on the lane's column c in both products, so the online
// softmax (max, sum, rescale of O) is lane-local apart from one exchange with
// lane l ^ 32. V^T comes straight from the row-major V tile through
// ds_read_b64_tr_b16.
#include "prefill_impl.h"

namespace sgl {
namespace pf {
namespace {

// Two workgroups per CU at 4 waves, one at 8; the split-kv variant (KS = 2)
// holds the whole LDS, so one.
template <int W, bool kPair, int KS>
__global__ void __launch_bounds__(64 * W, KS == 2 ? 1 : 8 / W) paged_prefill_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) char lds_raw[prefill_lds_bytes<W, KS>()];
  prefill_item<W, kPair, KS>(a, lds_raw, blockIdx.x, gridDim.x);
}

}  // namespace
}  // namespace pf
}  // namespace sgl

using namespace sgl;
using namespace sgl::pf;

// Compute units of the current device (256 on MI355X; 256 when none is visible).
static int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) == hipSuccess &&
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
      cus > 0)
    return cus;
  return 256;
}

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
  PrefillArgs a;
  const int st = prefill_args(q, q_stride_token, q_stride_head, k_cache, v_cache, kv_stride_slot,
                              kv_stride_head, indices, qo_indptr, kv_indptr, q_start,
                              num_qo_heads, num_kv_heads, head_dim, sm_scale, o,
                              o_stride_token, o_stride_head, a);
  if (st != SGL_OK) return st;
  const int group = a.group;
  // 8-wave workgroups pay off on long chunks that still fill every CU once
  // (measured: 2048-token chunks at G = 8, 4096 at G = 4); short or few
  // chunks keep 4-wave workgroups, two per CU.
  const int64_t rows_max = static_cast<int64_t>(max_qo_len) * group;
  const int64_t tiles8 = (rows_max + 255) / 256;
  const bool wide = rows_max >= 8192 &&
                    tiles8 * num_kv_heads * batch_size >= static_cast<int64_t>(device_cus());
  // Pairing (one tile from each end of the causal range per workgroup) when
  // the launch is at most one workgroup per CU: the dispatcher cannot then
  // even out unequal tiles, and measured it is 3-6% faster; with several
  // workgroups per CU, heavy-first dispatch balances better.
  const int64_t pairs = ((rows_max + 127) / 128 + 1) / 2;
  const bool pair = wide && pairs * num_kv_heads * batch_size <= static_cast<int64_t>(device_cus());
  // Launches that would leave CUs idle even with 64-row items split each
  // item's kv tiles between two 2-wave groups (KS = 2): 64-row items reach
  // twice the CUs, each group streaming half the kv tiles.
  const bool split_kv = !wide && ((rows_max + 63) / 64) * num_kv_heads * batch_size <=
                                     static_cast<int64_t>(device_cus());
  const int bm = wide ? 256 : split_kv ? 64 : 128;
  const int64_t tiles = pair ? pairs : (rows_max + bm - 1) / bm;
  const int64_t items = tiles * num_kv_heads * batch_size;
  if (items > 0x7fffffff) return SGL_ERR_INVALID_ARG;
  a.tiles_per_req = static_cast<int>(tiles);
  a.num_kv_heads = num_kv_heads;
  const dim3 grid(static_cast<uint32_t>(items));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (pair)
    hipLaunchKernelGGL((paged_prefill_kernel<8, true, 1>), grid, dim3(512), 0, s, a);
  else if (wide)
    hipLaunchKernelGGL((paged_prefill_kernel<8, false, 1>), grid, dim3(512), 0, s, a);
  else if (split_kv)
    hipLaunchKernelGGL((paged_prefill_kernel<4, false, 2>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((paged_prefill_kernel<4, false, 1>), grid, dim3(256), 0, s, a);
  return launch_status();
}
