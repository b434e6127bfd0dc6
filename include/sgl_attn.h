/*
 * sgl_attn.h — C ABI of the MI355X (gfx950) attention hot path.
 *
 * Every entry point takes plain device pointers, element counts and
 * strides (in elements), a hipStream_t passed as `void*`, and returns an
 * int status: 0 on success, a negative SGL_ERR_* code for an argument the
 * call rejects before launching anything, or a positive hipError_t when the
 * HIP runtime refuses the launch. No entry point allocates device memory;
 * workspaces are passed in by the caller. The pool layout is the
 * reference's MHAKVCache: one layer's K (or V) cache is [slots, Hkv, D]
 * bf16, token-granular (a "page" of page_size P is P consecutive slots).
 *
 * Each declaration names the reference interface (allen-shaw/sglang.cpp,
 * file:line) it replaces.
 */
#ifndef SGL_ATTN_H_
#define SGL_ATTN_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SGL_OK 0
#define SGL_ERR_INVALID_ARG (-1)  /* null pointer, bad size, bad stride */
#define SGL_ERR_UNSUPPORTED (-2)  /* head_dim / group size / dtype not built */
#define SGL_ERR_CAPACITY (-3)     /* workspace or plan capacity exceeded */
#define SGL_ERR_ALIGNMENT (-4)    /* pointer / stride misaligned for vector path */

#define SGL_INDEX_I32 0
#define SGL_INDEX_I64 1

#define SGL_DTYPE_BF16 0  /* 16-bit element types (norm, RoPE and residual-path kernels) */
#define SGL_DTYPE_F16 1
#define SGL_DTYPE_F32 2   /* fp32 (accepted where a declaration says so) */

/* Human-readable text for a status code (static storage). */
const char* sgl_status_string(int status);

/* Library version, to check that the loaded .so matches this header. */
int sgl_abi_version(void);
#define SGL_ABI_VERSION 15

/* ------------------------------------------------------------------ */
/* KV-cache store                                                      */
/* ------------------------------------------------------------------ */

/*
 * k_cache[out_loc[t], :] = k[t, :] and v_cache[out_loc[t], :] = v[t, :]
 * for t < num_tokens, copying elems_per_token 2-byte elements (bf16 or
 * fp16: the copy is bitwise). k/v rows are strided by k_stride_token /
 * v_stride_token elements (the narrow views of a qkv row); cache rows are
 * contiguous, elems_per_token apart. out_loc is int32 (index_dtype
 * SGL_INDEX_I32) or int64 (SGL_INDEX_I64).
 * Replaces: MHAKVCache::store_kv + store_kv_cache_kernel
 *           (src/kvcache/mha_kvcache.cu:111-155, :13-41).
 */
int sgl_store_kv(void* k_cache, void* v_cache, const void* k, const void* v,
                 const void* out_loc, int index_dtype, int64_t num_tokens,
                 int64_t elems_per_token, int64_t k_stride_token,
                 int64_t v_stride_token, void* stream);

/* ------------------------------------------------------------------ */
/* Page-table / token-pool plumbing                                    */
/* ------------------------------------------------------------------ */

/*
 * indices[kv_indptr[r] + p] = page_table[table_indices[r] * stride + p]
 * for p < kv_indptr[r+1]-kv_indptr[r] (0 where p >= cols); rows whose
 * table index is outside [0, rows) are left untouched.
 * Replaces: build_decode_indices_kernel (src/attention/flashinfer_backend.cu:43-70).
 */
int sgl_build_decode_indices(const int32_t* page_table, int64_t rows,
                             int64_t stride, int64_t cols,
                             const int32_t* table_indices,
                             const int32_t* kv_indptr, int32_t* indices,
                             int batch_size, void* stream);

/*
 * Prefill metadata gather: indices = cat_r(page_table[table_indices[r], :kv_len_r]),
 * with kv_indptr the prefix sum of kv_len. Device-side replacement of the
 * torch::cat over page-table slices.
 * Replaces: prefill branch of FlashInferBackend::prepare_metadata
 *           (src/attention/flashinfer_backend.cu:466-484).
 */
int sgl_build_prefill_indices(const int32_t* page_table, int64_t rows,
                              int64_t stride, int64_t cols,
                              const int32_t* table_indices,
                              const int32_t* kv_indptr, int32_t* indices,
                              int batch_size, void* stream);

/*
 * pool[req_indices[i] * stride + positions[i]] = tokens[i]; entries with an
 * out-of-range row or column are skipped.
 * Replaces: write_token_pool (src/kernels/token_pool.cu:53-93, kernel :10-29).
 */
int sgl_write_token_pool(int32_t* pool, int64_t rows, int64_t stride,
                         int64_t cols, const int32_t* req_indices,
                         const int32_t* positions, const int32_t* tokens,
                         int64_t count, void* stream);

/*
 * Page allocation -> token-granular page table, on the device. The
 * allocations alloc_info[a] = (table_idx, first_page, last_page), int32
 * [num_allocs, 3], take consecutive entries of page_starts (the slot of each
 * allocated page's first token, num_pages of them, in allocation order);
 * page p of allocation a writes
 *   page_table[table_idx * stride + p * page_size + i] = page_start + i,
 * i < page_size, skipping out-of-range rows and columns as
 * sgl_write_token_pool does. Pages beyond what the allocations take are
 * ignored; the caller keeps sum(last_page - first_page) == num_pages, as the
 * reference checks on the host. At most 8192 allocations per call.
 * Replaces: CacheManager::write_page_table + pages_to_tokens
 *           (src/scheduler/prefill.cc:144-187, :103-119): the host expansion
 *           loop and its three token-sized H2D copies.
 */
int sgl_write_page_table(int32_t* page_table, int64_t rows, int64_t stride,
                         int64_t cols, const int32_t* page_starts, int64_t num_pages,
                         const int32_t* alloc_info, int num_allocs, int page_size,
                         void* stream);

/*
 * out[i] = table[req_indices[i] * stride + positions[i]] (0 when out of range).
 * Replaces: gather_int32_2d (src/kernels/token_pool.cu:95-133, kernel :31-49).
 */
int sgl_gather_int32_2d(const int32_t* table, int64_t rows, int64_t stride,
                        int64_t cols, const int32_t* req_indices,
                        const int32_t* positions, int32_t* out, int64_t count,
                        void* stream);

/*
 * Up to SGL_MAX_I32_COPIES device-to-device int32 copies in one launch:
 * dst[i] = src[i] for i < count of each entry (entries must not overlap).
 * The graph-replay path refreshes every capture buffer of a step (indptrs,
 * row maps, indices) with this one call instead of one copy per buffer.
 * Replaces: the per-buffer copies of FlashInferBackend::prepare_for_replay
 *           (src/attention/flashinfer_backend.cu:267-352).
 */
typedef struct {
  const int32_t* src;
  int32_t* dst;
  int64_t count;
} sgl_i32_copy_t;
#define SGL_MAX_I32_COPIES 8
int sgl_copy_i32(const sgl_i32_copy_t* copies, int num_copies, void* stream);

/* ------------------------------------------------------------------ */
/* RoPE and q/k RMSNorm                                                */
/* ------------------------------------------------------------------ */

/*
 * cos[p, i] = cos(p * inv_freq[i]), sin likewise, for p < max_pos,
 * i < rotary_dim/2, inv_freq[i] = 1 / base^(2i / rotary_dim), fp32.
 * Replaces: RotaryEmbedding ctor cache build (src/layers/rotary_embedding.cu:75-94).
 */
int sgl_rope_cos_sin_cache(float* cos_cache, float* sin_cache, int64_t max_pos,
                           int rotary_dim, float base, void* stream);

/*
 * In-place per-(token, head) RMSNorm of q [tokens, q_heads, d] and
 * k [tokens, k_heads, d] (strided views, last dim contiguous):
 * x <- T(x * rsqrt(mean(x^2) + eps) * w), fp32 accumulation, T = bf16 or
 * fp16 (dtype SGL_DTYPE_*; q, k and the weights share it, as the reference
 * dispatches both at :346-372).
 * Pass k = NULL / k_heads = 0 to normalise q only.
 * Replaces: fused_qk_rmsnorm_inplace_3d_strided (src/layers/normalization.cu:318-384)
 *           and RMSNorm::forward_inplace_3d_strided (:271-316).
 */
int sgl_qk_rmsnorm(void* q, void* k, const void* q_weight,
                   const void* k_weight, int64_t tokens, int64_t q_heads,
                   int64_t k_heads, int64_t d, int64_t q_stride_token,
                   int64_t q_stride_head, int64_t k_stride_token,
                   int64_t k_stride_head, float eps, int dtype, void* stream);

/*
 * In-place NeoX (rotate-half) RoPE of q [nnz, q_heads, head_dim] and
 * k [nnz, kv_heads, head_dim] at positions[t] (int32), using fp32 cos/sin
 * caches of width cos_width (rotary_dim/2 or rotary_dim). Elements at
 * index >= rotary_dim pass through. q and k are bf16 or fp16 (dtype
 * SGL_DTYPE_*, the reference dispatches both at :124-168); fp32 math, one
 * rounding per element.
 * Replaces: RotaryEmbedding::forward_inplace (src/layers/rotary_embedding.cu:96-178;
 *           formula :50-66).
 */
int sgl_rope(void* q, void* k, const float* cos_cache, const float* sin_cache,
             const int32_t* positions, int64_t nnz, int64_t q_heads,
             int64_t kv_heads, int64_t rotary_dim, int64_t head_dim,
             int64_t cos_width, int64_t q_stride_token, int64_t q_stride_head,
             int64_t k_stride_token, int64_t k_stride_head, int dtype, void* stream);

/*
 * One pass over the qkv activation [T, (Hq + 2 Hkv) * D] (row stride
 * qkv_stride_token): per token, q/k heads are RMS-normalised (weights
 * q_weight / k_weight, skipped when NULL), rounded to bf16, rotated by
 * RoPE at positions[t] (full rotary, half-width fp32 cos/sin cache
 * [max_pos, D/2]), rounded to bf16 and written back in place; the rotated
 * k row and the raw v row are also written to k_cache / v_cache at slot
 * out_loc[t] (int32). Bitwise the same as running sgl_qk_rmsnorm, then
 * sgl_rope, then sgl_store_kv. flags: 0, or SGL_FUSED_NO_K_WRITEBACK to
 * leave the k part of qkv untouched (the rotated k goes to k_cache only;
 * the reference writes it back, but nothing reads it after the store).
 * Replaces the sequence AttentionLayer::forward -> qk-norm -> RoPE ->
 * store_kv (src/layers/attention_layer.cc:27-47, flashinfer_backend.cu:530-532).
 */
int sgl_fused_qknorm_rope_store(void* qkv, int64_t qkv_stride_token,
                                void* k_cache, void* v_cache,
                                const void* q_weight, const void* k_weight,
                                const float* cos_cache, const float* sin_cache,
                                const int32_t* positions, const int32_t* out_loc,
                                int64_t num_tokens, int num_qo_heads,
                                int num_kv_heads, int head_dim, float eps,
                                int flags, void* stream);
#define SGL_FUSED_NO_K_WRITEBACK 1

/* ------------------------------------------------------------------ */
/* Paged attention                                                     */
/* ------------------------------------------------------------------ */

/* Split-KV decode plan (host). */
typedef struct {
  int32_t kv_chunk_size;  /* W_max: largest unit in tokens (multiple of 16, <= 8192) */
  int32_t min_chunk_size; /* W_min: smallest unit (64) */
  int32_t num_units;      /* work units = workgroups launched */
  int32_t split_kv;       /* 1 when a request of the planned batch spans units */
  int32_t batch_size;     /* largest batch the plan serves */
  int32_t num_qo_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int64_t max_total_tokens; /* capacity: num_units * kv_chunk_size tokens per call */
  int64_t workspace_bytes;  /* 256-byte header (status word) + fp32 partials, two per unit,
                               + one int32 per unit */
} sgl_decode_plan_t;

/*
 * Token-balanced schedule from the host copy of kv_indptr (kv_indptr[0] must
 * be 0): the batch's flattened token stream is cut into num_units equal
 * units, one per resident workgroup (the count comes from the device's CU
 * count, 256 when no device is visible). The launch picks the unit size on
 * the device, clamp(ceil(total / num_units), min_chunk_size, kv_chunk_size)
 * rounded to 16 tokens, from kv_indptr[batch], so a plan built from a
 * kv_indptr with every request at its maximum length stays valid and
 * balanced for any batch of at most batch_size requests and at most
 * max_total_tokens tokens, whatever the per-request lengths (graph capture /
 * replay without re-planning).
 * Replaces: FlashInfer DecodePlan as called from
 *           FlashInferBackend::initialize_decode_metadata_once
 *           (src/attention/flashinfer_backend.cu:354-397).
 */
int sgl_decode_plan(const int32_t* kv_indptr_host, int batch_size,
                    int num_qo_heads, int num_kv_heads, int head_dim,
                    sgl_decode_plan_t* plan);

/*
 * Host-side check that a batch (host kv_indptr, batch_size requests) fits a
 * plan: SGL_OK, or SGL_ERR_CAPACITY when it has more requests than
 * plan->batch_size or more tokens than plan->max_total_tokens.
 * Replaces: the batch-size / length checks of
 *           FlashInferBackend::prepare_for_replay (src/attention/flashinfer_backend.cu:267-352).
 */
int sgl_decode_plan_check(const sgl_decode_plan_t* plan, const int32_t* kv_indptr_host,
                          int batch_size);

/*
 * Paged decode: for request r (rows q[q_row(r)], q_row(r) = r, or
 * q_indptr[r] when q_indptr is non-NULL) and q head h,
 * o[q_row, h] = softmax_j(q.K[indices[kv_indptr[r] + j], h / G] * sm_scale)
 *               . V[indices[...], h / G]
 * over j < kv_indptr[r+1] - kv_indptr[r]; an empty request gets a zero row.
 * G = Hq / Hkv. q is strided (q_stride_token, q_stride_head), o likewise
 * (strides multiples of 8 elements); k_cache/v_cache are one layer's
 * [slots, Hkv, D] (slot stride kv_stride_slot, head stride kv_stride_head).
 * workspace (plan->workspace_bytes, 16-byte aligned) holds the split
 * partials and, at offset 0, an int32 status word: each call clears it, and
 * when the device kv_indptr[batch] exceeds plan->max_total_tokens the rows
 * of every request reaching past the capacity are written as NaN and the
 * word is set to SGL_ERR_CAPACITY (read it with sgl_decode_status). Two
 * kernels run on the stream (decode, then merge: one workgroup per (kv
 * head, request), or per (kv head, unit) when the batch has more requests
 * than the plan has units), or one for small batches
 * (plans at the 64-token minimum unit with batch_size x Hkv workgroups at
 * most the CU count). Calls that share one workspace must be stream-ordered.
 * Replaces: BatchDecodeWithPagedKVCacheDispatched call in
 *           FlashInferBackend::forward (src/attention/flashinfer_backend.cu:553-595).
 */
int sgl_paged_decode(const sgl_decode_plan_t* plan, const void* q,
                     int64_t q_stride_token, int64_t q_stride_head,
                     const void* k_cache, const void* v_cache,
                     int64_t kv_stride_slot, int64_t kv_stride_head,
                     const int32_t* indices, const int32_t* kv_indptr,
                     const int32_t* q_indptr, int batch_size,
                     int num_qo_heads, int num_kv_heads, int head_dim,
                     float sm_scale, void* o, int64_t o_stride_token,
                     int64_t o_stride_head, void* workspace,
                     int64_t workspace_bytes, void* stream);

/*
 * sgl_paged_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). The split partials live in a file-scope
 * device array of SGL_DECODE_SCRATCH_BYTES (32 MiB) that each GPU holds
 * until the process ends; plans with workspace_bytes above it get
 * SGL_ERR_CAPACITY. Nothing is allocated. Calls on one GPU share the array
 * and must be stream-ordered: calls that overlap on one GPU race. A batch
 * past the plan's capacity gets NaN rows and the CAPACITY status word as in
 * sgl_paged_decode; sgl_decode_status(NULL, ...) reads that word from the
 * current device's scratch. sgl_decode_plan looks the scratch address up
 * for the current device, so a call captured into a graph after a plan was
 * made runs no lookup inside the capture.
 * Replaces: no counterpart in the reference; it exists for callers that
 *           cannot allocate.
 */
int sgl_paged_decode_noalloc(const sgl_decode_plan_t* plan, const void* q,
                             int64_t q_stride_token, int64_t q_stride_head,
                             const void* k_cache, const void* v_cache,
                             int64_t kv_stride_slot, int64_t kv_stride_head,
                             const int32_t* indices, const int32_t* kv_indptr,
                             const int32_t* q_indptr, int batch_size,
                             int num_qo_heads, int num_kv_heads, int head_dim,
                             float sm_scale, void* o, int64_t o_stride_token,
                             int64_t o_stride_head, void* stream);
#define SGL_DECODE_SCRATCH_BYTES (32ll << 20)

/*
 * Reads the status word a decode call left in its workspace (waits for the
 * stream): SGL_OK, or SGL_ERR_CAPACITY when the batch exceeded its plan.
 * workspace NULL reads the word of sgl_paged_decode_noalloc's scratch on the
 * current device.
 * Replaces: no device-side counterpart in the reference (FlashInfer's plan
 *           is host-side); pairs with sgl_paged_decode.
 */
int sgl_decode_status(const void* workspace, int32_t* status, void* stream);

/*
 * Paged causal prefill over ragged requests: query i (0-based inside
 * request r, qo_len = qo_indptr[r+1]-qo_indptr[r]) attends kv j with
 * j <= i + kv_len - qo_len (bottom-right alignment), kv_len =
 * kv_indptr[r+1]-kv_indptr[r], slots from indices[kv_indptr[r] + j].
 * Request r's query (and output) rows start at q_start[r], or at
 * qo_indptr[r] when q_start is NULL (a subset of a batch's requests can so
 * be run in place). max_qo_len bounds qo_len over the batch (sizes the grid).
 * Replaces: BatchPrefillWithPagedKVCacheDispatched<..., kCausal, ...> in
 *           FlashInferBackend::forward (src/attention/flashinfer_backend.cu:596-679).
 */
int sgl_paged_prefill(const void* q, int64_t q_stride_token,
                      int64_t q_stride_head, const void* k_cache,
                      const void* v_cache, int64_t kv_stride_slot,
                      int64_t kv_stride_head, const int32_t* indices,
                      const int32_t* qo_indptr, const int32_t* kv_indptr,
                      const int32_t* q_start, int batch_size, int max_qo_len,
                      int num_qo_heads,
                      int num_kv_heads, int head_dim, float sm_scale, void* o,
                      int64_t o_stride_token, int64_t o_stride_head,
                      void* stream);

/*
 * A mixed batch (decode rows beside prefill rows, the chunked-prefill step
 * of FlashInferBackend::forward's prefill phase with one-token requests) in
 * one launch plus the split merge: the first workgroups run the decode rows
 * on decode_cus CUs while the causal-prefill items run on the others, then
 * on every CU as the decode finishes (the HBM-bound decode and the
 * MFMA-bound prefill side by side). num_kv_heads must divide 8.
 *   sgl_mixed_decode_cus: the CU share for the decode rows (a multiple of
 *     8), from their K/V token count and the prefill's flops
 *     (4 D Hq sum_r sum_i (kv_r - qo_r + i + 1)).
 *   sgl_decode_plan_cus: a decode plan (as sgl_decode_plan) whose units fill
 *     decode_cus CUs, each unit short enough for the fused launch's LDS
 *     (at 1 or 2 kv heads long batches then get more units than that); like
 *     any plan it serves smaller batches on replay.
 *   sgl_paged_mixed: decode rows as sgl_paged_decode (dec_q_rows: query row
 *     of each decode request, or NULL for rows 0..dec_batch-1) and prefill
 *     rows as sgl_paged_prefill, sharing q, the caches and o. With no rows
 *     of one kind it runs the other entry point alone; with a plan whose
 *     units are too long for the fused launch (sgl_decode_plan at 1 or 2
 *     kv heads) it runs the two entry points one after the other.
 * Replaces: the decode and prefill calls of one mixed step
 *           (src/attention/flashinfer_backend.cu:553-679); the reference
 *           runs them as separate kernels.
 */
int sgl_mixed_decode_cus(int64_t decode_kv_tokens, int num_kv_heads, int head_dim,
                         double prefill_flops);
int sgl_decode_plan_cus(const int32_t* kv_indptr_host, int batch_size,
                        int num_qo_heads, int num_kv_heads, int head_dim,
                        int decode_cus, sgl_decode_plan_t* plan);
int sgl_paged_mixed(const sgl_decode_plan_t* plan, const void* q,
                    int64_t q_stride_token, int64_t q_stride_head,
                    const void* k_cache, const void* v_cache,
                    int64_t kv_stride_slot, int64_t kv_stride_head,
                    const int32_t* dec_indices, const int32_t* dec_kv_indptr,
                    const int32_t* dec_q_rows, int dec_batch,
                    const int32_t* pre_indices, const int32_t* pre_qo_indptr,
                    const int32_t* pre_kv_indptr, const int32_t* pre_q_start,
                    int pre_batch, int pre_max_qo_len, int num_qo_heads,
                    int num_kv_heads, int head_dim, float sm_scale, void* o,
                    int64_t o_stride_token, int64_t o_stride_head,
                    void* workspace, int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------ */
/* Residual path: RMSNorm, fused add + RMSNorm, gated activations      */
/* ------------------------------------------------------------------ */

/*
 * out[r, :] = T(x[r, :] * rsqrt(mean(x[r, :]^2) + eps) * weight) for
 * r < rows, fp32 arithmetic, T = bf16 or fp16 (dtype SGL_DTYPE_*; weight
 * has the same type). Rows of d elements, x_stride_row / out_stride_row
 * elements apart; out may equal x (in place).
 * Replaces: RMSNorm::forward / forward_inplace
 *           (src/layers/normalization.cu:236-269).
 */
int sgl_rmsnorm(void* out, const void* x, const void* weight, int64_t rows,
                int64_t d, int64_t x_stride_row, int64_t out_stride_row,
                int dtype, float eps, void* stream);

/*
 * In place, per row: s = x + residual (fp32); residual = T(s);
 * x = T(s * rsqrt(mean(s^2) + eps) * weight). Rows longer than 8192
 * elements normalise T(s) instead of s (a second pass re-reads it).
 * Replaces: RMSNorm::fused_add_forward_inplace
 *           (src/layers/normalization.cu:386-416).
 */
int sgl_fused_add_rmsnorm(void* x, void* residual, const void* weight,
                          int64_t rows, int64_t d, int64_t x_stride_row,
                          int64_t residual_stride_row, int dtype, float eps,
                          void* stream);

/*
 * out[t, i] = T(silu(in[t, i]) * in[t, d + i]), silu(x) = x / (1 + e^-x),
 * for t < tokens, i < d; input rows hold 2 d elements (gate, then up).
 * Replaces: silu_and_mul (src/layers/activation.cu:8-10, 15-45).
 */
int sgl_silu_and_mul(void* out, const void* input, int64_t tokens, int64_t d,
                     int64_t in_stride_row, int64_t out_stride_row, int dtype,
                     void* stream);

/*
 * As sgl_silu_and_mul with the tanh GELU
 * gelu(x) = 0.5 x (1 + tanh(0.7978845608 (x + 0.044715 x^3))).
 * Replaces: gelu_and_mul (src/layers/activation.cu:12-14, 47-77).
 */
int sgl_gelu_and_mul(void* out, const void* input, int64_t tokens, int64_t d,
                     int64_t in_stride_row, int64_t out_stride_row, int dtype,
                     void* stream);

/* ------------------------------------------------------------------ */
/* Probabilities from logits, then sampling from probabilities         */
/* ------------------------------------------------------------------ */

/*
 * probs[r, i] = softmax_i(float(logits[r, i]) / t_r) over i < vocab, fp32,
 * for r < batch; t_r = temperatures[r] (fp32 [batch]) or, when temperatures
 * is NULL, the scalar temperature (> 0). logits_dtype: SGL_DTYPE_BF16,
 * SGL_DTYPE_F16 or SGL_DTYPE_F32; row strides in elements (>= vocab). One
 * workgroup per row; aligned 16-bit rows of up to 163,840 elements are
 * held in registers and read from HBM once. Exponentials as
 * 2^(fma(x, a, -max a)) with a = log2e / t (relative error of a probability
 * below ~1e-5 against the exact softmax of float(x) / t). A row whose
 * temperature is not positive gets NaN probabilities.
 * Replaces: the probabilities of Sampler::sample, logits.to(kFloat32) /
 *           temperatures then torch::softmax (src/engine/engine.cc:306-308).
 */
int sgl_softmax_temperature(float* probs, int64_t probs_stride_row, const void* logits,
                            int64_t logits_stride_row, int logits_dtype,
                            const float* temperatures, float temperature, int64_t batch,
                            int64_t vocab, void* stream);

/*
 * probs: fp32 [batch_size, d], rows contiguous (the softmax of the
 * temperature-scaled logits). out: int32 [batch_size]. The draw with
 * uniform u is the first index i with probs[i] > 0 whose running sum of
 * such probabilities exceeds u (d - 1 if rounding leaves none). uniform is
 * fp32 [batch_size]. deterministic is accepted for the reference's
 * signature; sums here always run in a fixed order. Rows of up to 2^21
 * probabilities (SGL_ERR_UNSUPPORTED beyond). One 1024-thread workgroup
 * per row, about 153 KiB of LDS; nothing is allocated.
 * Replaces: flashinfer_sample_from_probs (src/engine/sampling.cu:65-84).
 */
int sgl_sampling_from_probs(const float* probs, const float* uniform, int32_t* out,
                            int batch_size, int d, int deterministic, void* stream);

/*
 * Top-k draw by rejection rounds: round r draws from the probabilities
 * above a pivot with u = uniform[r, row] * (their mass), the pivot rises to
 * the drawn probability, and the draw is accepted once fewer than k
 * probabilities exceed it. uniform: fp32 [max_rounds, batch_size]; k is
 * top_k_arr[row] (fp32, as the reference passes it) or top_k_val when
 * top_k_arr is NULL. success (bool bytes, optional) = accepted within
 * max_rounds; out holds the last draw either way.
 * Replaces: flashinfer_top_k_sample_from_probs (src/engine/sampling.cu:86-116).
 */
int sgl_top_k_sampling_from_probs(const float* probs, const float* uniform, int32_t* out,
                                  uint8_t* success, const float* top_k_arr,
                                  int batch_size, int top_k_val, int d, int max_rounds,
                                  int deterministic, void* stream);

/*
 * As above, accepting once the mass above the pivot is below top_p
 * (top_p_arr[row], or top_p_val when top_p_arr is NULL).
 * Replaces: flashinfer_top_p_sample_from_probs (src/engine/sampling.cu:118-148).
 */
int sgl_top_p_sampling_from_probs(const float* probs, const float* uniform, int32_t* out,
                                  uint8_t* success, const float* top_p_arr,
                                  int batch_size, float top_p_val, int d, int max_rounds,
                                  int deterministic, void* stream);

/*
 * Both filters: accepted once fewer than k probabilities exceed the pivot
 * and their mass is below top_p. top_k_arr is int32 here, as the
 * reference passes it.
 * Replaces: flashinfer_top_k_top_p_sample_from_probs
 *           (src/engine/sampling.cu:150-192).
 */
int sgl_top_k_top_p_sampling_from_probs(const float* probs, const float* uniform,
                                        const int32_t* top_k_arr, const float* top_p_arr,
                                        int32_t* out, uint8_t* success, int batch_size,
                                        int top_k_val, float top_p_val, int d,
                                        int max_rounds, int deterministic, void* stream);

/*
 * The draws above from logits instead of probabilities: row r's
 * probabilities are those sgl_softmax_temperature would write for the same
 * logits and temperature (computed on the fly, the same bits when its probs
 * buffer is 16-byte aligned), so the samples and success flags equal those
 * of sgl_softmax_temperature followed by the mode's draw; the probabilities
 * are never stored. mode: 0 plain (uniform fp32 [batch_size]), 1 top-k
 * (top_k_f fp32 [batch] or top_k_val), 2 top-p (top_p_arr or top_p_val),
 * 3 top-k + top-p (top_k_i int32 [batch] or top_k_val, and top p); modes
 * 1-3 take uniform fp32 [max_rounds, batch_size] and write success when
 * given. logits_dtype and temperatures as for sgl_softmax_temperature.
 * Replaces: Sampler::sample's probabilities and draw together
 *           (src/engine/engine.cc:306-333: torch::softmax of the scaled
 *           logits, then flashinfer_*_sample_from_probs).
 */
int sgl_sampling_from_logits(const void* logits, int64_t logits_stride_row, int logits_dtype,
                             const float* temperatures, float temperature, const float* uniform,
                             int mode, const float* top_k_f, const int32_t* top_k_i,
                             int top_k_val, const float* top_p_arr, float top_p_val,
                             int32_t* out, uint8_t* success, int batch_size, int d,
                             int max_rounds, void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* SGL_ATTN_H_ */
