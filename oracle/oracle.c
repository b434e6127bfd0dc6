/*
 * oracle.c — CPU restatement of the reference attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the parity tests and
 * the bench's cpu_baseline leg compare the HIP library against. Nothing in
 * the product (sglang.cpp_amd/) links, loads or calls it.
 *
 * Each function names the reference file:line it restates
 * (allen-shaw/sglang.cpp). Attention outputs are fp32 (an fp32-softmax
 * reference); the elementwise kernels reproduce the reference's bf16
 * rounding points exactly. How each function is pinned (closed forms,
 * library routines, invariants) is in tests/test_oracle_pins.py; none is left
 * unpinned.
 *
 * Build: oracle/Makefile (gcc, OpenMP). Floating-point contraction is off so
 * products and sums round exactly as written.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------- bf16 ---------- */

static inline float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* Round to nearest even, NaN kept quiet (what a bf16 cast does). */
static inline uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

int oracle_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void oracle_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

void oracle_f32_to_bf16(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f32_to_bf16(in[i]);
}

/* ---------- KV store: src/kvcache/mha_kvcache.cu:13-41 ---------- */

void oracle_store_kv(uint16_t* k_cache, uint16_t* v_cache, const uint16_t* k,
                     const uint16_t* v, const int64_t* out_loc, int64_t num_tokens,
                     int64_t elems, int64_t k_stride, int64_t v_stride) {
  for (int64_t t = 0; t < num_tokens; ++t) {
    const int64_t slot = out_loc[t];
    memcpy(k_cache + slot * elems, k + t * k_stride, (size_t)elems * 2);
    memcpy(v_cache + slot * elems, v + t * v_stride, (size_t)elems * 2);
  }
}

/* ---------- decode indices: src/attention/flashinfer_backend.cu:43-70 ---------- */

void oracle_build_indices(const int32_t* page_table, int64_t rows, int64_t stride,
                          int64_t cols, const int32_t* table_indices,
                          const int32_t* kv_indptr, int32_t* indices, int batch) {
  for (int r = 0; r < batch; ++r) {
    const int32_t row = table_indices[r];
    const int32_t start = kv_indptr[r];
    const int32_t len = kv_indptr[r + 1] - start;
    if (row < 0 || row >= rows || len <= 0) continue;
    for (int32_t p = 0; p < len; ++p)
      indices[start + p] = p < cols ? page_table[(int64_t)row * stride + p] : 0;
  }
}

/* ---------- token pool: src/kernels/token_pool.cu:10-49 ---------- */

void oracle_write_token_pool(int32_t* pool, int64_t rows, int64_t stride, int64_t cols,
                             const int32_t* req, const int32_t* pos, const int32_t* tok,
                             int64_t count) {
  for (int64_t i = 0; i < count; ++i) {
    const int64_t r = req[i], p = pos[i];
    if (r < 0 || r >= rows || p < 0 || p >= cols) continue;
    pool[r * stride + p] = tok[i];
  }
}

void oracle_gather_int32_2d(const int32_t* table, int64_t rows, int64_t stride, int64_t cols,
                            const int32_t* req, const int32_t* pos, int32_t* out,
                            int64_t count) {
  for (int64_t i = 0; i < count; ++i) {
    const int64_t r = req[i], p = pos[i];
    out[i] = (r >= 0 && r < rows && p >= 0 && p < cols) ? table[r * stride + p] : 0;
  }
}

/* ---------- page allocation -> page table: src/scheduler/prefill.cc:103-187 ----------
 * Expands page starts (slot of a page's first token) into token slots and
 * writes row table_idx, positions [first_page*P, last_page*P).           */
void oracle_pages_to_tokens(const int32_t* page_starts, int64_t npages, int page_size,
                            int32_t* tokens) {
  for (int64_t p = 0; p < npages; ++p)
    for (int i = 0; i < page_size; ++i) tokens[p * page_size + i] = page_starts[p] + i;
}

/* CacheManager::write_page_table (src/scheduler/prefill.cc:144-187): the
 * allocations, in order, take consecutive entries of page_starts; page p of
 * allocation (table_idx, first_page, last_page) writes positions
 * p*P .. p*P+P-1 of row table_idx with page_start + 0 .. P-1, through the
 * token-pool write (out-of-range rows / columns skipped, token_pool.cu:10-29).
 * Returns the number of page starts consumed (the reference checks that it
 * equals npages).                                                         */
int64_t oracle_write_page_table(int32_t* table, int64_t rows, int64_t stride, int64_t cols,
                                const int32_t* page_starts, int64_t npages,
                                const int32_t* alloc, int64_t nalloc, int page_size) {
  int64_t used = 0;
  for (int64_t a = 0; a < nalloc; ++a) {
    const int32_t row = alloc[3 * a], first = alloc[3 * a + 1], last = alloc[3 * a + 2];
    for (int32_t page = first; page < last; ++page) {
      if (used >= npages) return -1;
      const int32_t start = page_starts[used++];
      for (int i = 0; i < page_size; ++i) {
        const int32_t tok = start + i;
        const int32_t pos = page * page_size + i;
        oracle_write_token_pool(table, rows, stride, cols, &row, &pos, &tok, 1);
      }
    }
  }
  return used;
}

/* ---------- RoPE cache: src/layers/rotary_embedding.cu:75-94 ---------- */

void oracle_cos_sin_cache(float* cos_cache, float* sin_cache, int64_t max_pos, int rotary_dim,
                          float base) {
  const int half = rotary_dim / 2;
  for (int k = 0; k < half; ++k) {
    const float expo = (float)(2 * k) / (float)rotary_dim;
    const float inv_freq = 1.0f / powf(base, expo);
    for (int64_t p = 0; p < max_pos; ++p) {
      const float f = (float)p * inv_freq;
      cos_cache[p * half + k] = cosf(f);
      sin_cache[p * half + k] = sinf(f);
    }
  }
}

/* ---------- fp16 bit patterns (IEEE binary16) ---------- */

static float round_t(float x, int dtype);

static inline float f16_to_f32(uint16_t h) {
  const int sign = (h >> 15) & 1, e = (h >> 10) & 0x1f, m = h & 0x3ff;
  float v;
  if (e == 0) v = ldexpf((float)m, -24);                 /* zero / subnormal */
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = ldexpf((float)(m | 0x400), e - 25);
  return sign ? -v : v;
}

/* Round to nearest even (round_t), then encode. */
static inline uint16_t f32_to_f16(float x) {
  const float r = round_t(x, 1);
  const uint16_t sign = signbit(r) ? 0x8000 : 0;
  if (isnan(r)) return 0x7e00;
  const float a = fabsf(r);
  if (isinf(a)) return sign | 0x7c00;
  if (a < 6.103515625e-05f) return sign | (uint16_t)(a * 16777216.0f); /* subnormal: a / 2^-24 */
  int e;
  const float m = frexpf(a, &e);               /* a = m 2^e, m in [0.5, 1) */
  const int field = e - 1 + 15;
  const uint16_t man = (uint16_t)((m * 2.0f - 1.0f) * 1024.0f);
  return sign | (uint16_t)(field << 10) | man;
}

/* 16-bit element load / store: dtype 0 = bf16, 1 = fp16. */
static inline float ld16(uint16_t b, int dtype) { return dtype ? f16_to_f32(b) : bf16_to_f32(b); }
static inline uint16_t st16(float x, int dtype) { return dtype ? f32_to_f16(x) : f32_to_bf16(x); }

void oracle_f16_bits(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f32_to_f16(in[i]);
}
void oracle_f16_values(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f16_to_f32(in[i]);
}

/* ---------- q/k RMSNorm: src/layers/normalization.cu:99-170 ---------- */

static void rmsnorm_row(uint16_t* row, const uint16_t* w, int64_t d, float eps, int dtype) {
  float ss = 0.f;
  for (int64_t i = 0; i < d; ++i) {
    const float x = ld16(row[i], dtype);
    ss += x * x;
  }
  const float scale = 1.0f / sqrtf(ss / (float)d + eps);
  for (int64_t i = 0; i < d; ++i)
    row[i] = st16((ld16(row[i], dtype) * scale) * ld16(w[i], dtype), dtype);
}

void oracle_qk_rmsnorm(uint16_t* q, uint16_t* k, const uint16_t* qw, const uint16_t* kw,
                       int64_t tokens, int64_t qh, int64_t kh, int64_t d, int64_t q_st,
                       int64_t q_sh, int64_t k_st, int64_t k_sh, float eps, int dtype) {
  for (int64_t t = 0; t < tokens; ++t) {
    for (int64_t h = 0; h < qh; ++h) rmsnorm_row(q + t * q_st + h * q_sh, qw, d, eps, dtype);
    if (k)
      for (int64_t h = 0; h < kh; ++h) rmsnorm_row(k + t * k_st + h * k_sh, kw, d, eps, dtype);
  }
}

/* ---------- RoPE: src/layers/rotary_embedding.cu:50-66 (NeoX rotate-half) ---------- */

static void rope_row(uint16_t* row, const float* cos_row, const float* sin_row,
                     int64_t rotary_dim, int64_t cos_width, int dtype) {
  const int64_t half = rotary_dim / 2;
  float buf[4096];
  for (int64_t i = 0; i < rotary_dim; ++i) {
    const int first = i < half;
    const int64_t pair = first ? i : i - half;
    const int64_t other = first ? i + half : i - half;
    const int64_t ci = cos_width == rotary_dim ? i : pair;
    const float v = ld16(row[i], dtype);
    const float o = ld16(row[other], dtype);
    const float c = cos_row[ci], s = sin_row[ci];
    buf[i] = first ? (v * c - o * s) : (v * c + o * s);
  }
  for (int64_t i = 0; i < rotary_dim; ++i) row[i] = st16(buf[i], dtype);
}

int oracle_rope(uint16_t* q, uint16_t* k, const float* cos_cache, const float* sin_cache,
                const int32_t* positions, int64_t nnz, int64_t qh, int64_t kh,
                int64_t rotary_dim, int64_t cos_width, int64_t q_st, int64_t q_sh,
                int64_t k_st, int64_t k_sh, int dtype) {
  if (rotary_dim > 4096) return -1;
  for (int64_t t = 0; t < nnz; ++t) {
    const int64_t p = positions[t];
    const float* cr = cos_cache + p * cos_width;
    const float* sr = sin_cache + p * cos_width;
    for (int64_t h = 0; h < qh; ++h)
      rope_row(q + t * q_st + h * q_sh, cr, sr, rotary_dim, cos_width, dtype);
    for (int64_t h = 0; h < kh; ++h)
      rope_row(k + t * k_st + h * k_sh, cr, sr, rotary_dim, cos_width, dtype);
  }
  return 0;
}

/* ---------- attention core (fp32 softmax) ----------
 * o[h, :] = sum_j softmax_j(q[h].K[j] * sm_scale) V[j], over the visible j.
 * The max-subtracted softmax of src/attention/flashinfer_backend.cu:553-679
 * (FlashInfer's online softmax computes the same quantity).             */

static void attend_row(const uint16_t* qrow, const uint16_t* k_cache, const uint16_t* v_cache,
                       int64_t kv_ss, const int32_t* slots, int64_t nvis, int64_t D,
                       float sm_scale, float* out, float* scores, float* qf) {
  for (int64_t d = 0; d < D; ++d) qf[d] = bf16_to_f32(qrow[d]);
  float mx = -INFINITY;
  for (int64_t j = 0; j < nvis; ++j) {
    const uint16_t* kr = k_cache + (int64_t)slots[j] * kv_ss;
    float s = 0.f;
    for (int64_t d = 0; d < D; ++d) s += qf[d] * bf16_to_f32(kr[d]);
    s *= sm_scale;
    scores[j] = s;
    if (s > mx) mx = s;
  }
  float den = 0.f;
  for (int64_t j = 0; j < nvis; ++j) {
    scores[j] = expf(scores[j] - mx);
    den += scores[j];
  }
  for (int64_t d = 0; d < D; ++d) out[d] = 0.f;
  for (int64_t j = 0; j < nvis; ++j) {
    const uint16_t* vr = v_cache + (int64_t)slots[j] * kv_ss;
    const float p = scores[j] / den;
    for (int64_t d = 0; d < D; ++d) out[d] += p * bf16_to_f32(vr[d]);
  }
}

/* Decode: src/attention/flashinfer_backend.cu:553-595. out is fp32
 * [rows, hq, D] contiguous; q row of request r is q_indptr ? q_indptr[r] : r.
 * kv_ss / kv_sh: slot and head strides of one layer's cache (elements).  */
void oracle_decode(const uint16_t* q, int64_t q_st, int64_t q_sh, const uint16_t* k_cache,
                   const uint16_t* v_cache, int64_t kv_ss, int64_t kv_sh,
                   const int32_t* indices, const int32_t* kv_indptr, const int32_t* q_indptr,
                   int batch, int hq, int hkv, int D, float sm_scale, float* out) {
  const int G = hq / hkv;
#pragma omp parallel
  {
    int64_t maxlen = 0;
    for (int r = 0; r < batch; ++r) {
      const int64_t len = kv_indptr[r + 1] - kv_indptr[r];
      if (len > maxlen) maxlen = len;
    }
    float* scores = (float*)malloc(sizeof(float) * (size_t)(maxlen + 1));
    float* qf = (float*)malloc(sizeof(float) * (size_t)D);
#pragma omp for schedule(dynamic)
    for (int64_t rh = 0; rh < (int64_t)batch * hq; ++rh) {
      const int r = (int)(rh / hq), h = (int)(rh % hq);
      const int64_t row = q_indptr ? q_indptr[r] : r;
      const int64_t beg = kv_indptr[r], len = kv_indptr[r + 1] - beg;
      float* o = out + (row * hq + h) * D;
      if (len <= 0) {
        for (int d = 0; d < D; ++d) o[d] = 0.f;
        continue;
      }
      const int64_t kvh = h / G;
      attend_row(q + row * q_st + h * q_sh, k_cache + kvh * kv_sh, v_cache + kvh * kv_sh, kv_ss,
                 indices + beg, len, D, sm_scale, o, scores, qf);
    }
    free(scores);
    free(qf);
  }
}

/* Causal prefill: src/attention/flashinfer_backend.cu:596-679 (kCausal):
 * query i of request r sees kv j <= i + kv_len - qo_len. out fp32 [sum qo, hq, D]. */
void oracle_prefill(const uint16_t* q, int64_t q_st, int64_t q_sh, const uint16_t* k_cache,
                    const uint16_t* v_cache, int64_t kv_ss, int64_t kv_sh,
                    const int32_t* indices, const int32_t* qo_indptr, const int32_t* kv_indptr,
                    int batch, int hq, int hkv, int D, float sm_scale, float* out) {
  const int G = hq / hkv;
  int64_t total_rows = qo_indptr[batch];
#pragma omp parallel
  {
    int64_t maxlen = 0;
    for (int r = 0; r < batch; ++r) {
      const int64_t len = kv_indptr[r + 1] - kv_indptr[r];
      if (len > maxlen) maxlen = len;
    }
    float* scores = (float*)malloc(sizeof(float) * (size_t)(maxlen + 1));
    float* qf = (float*)malloc(sizeof(float) * (size_t)D);
#pragma omp for schedule(dynamic, 4)
    for (int64_t th = 0; th < total_rows * hq; ++th) {
      const int64_t row = th / hq;
      const int h = (int)(th % hq);
      int r = 0;
      while (qo_indptr[r + 1] <= row) ++r;
      const int64_t i = row - qo_indptr[r];
      const int64_t qo_len = qo_indptr[r + 1] - qo_indptr[r];
      const int64_t beg = kv_indptr[r], kv_len = kv_indptr[r + 1] - beg;
      int64_t nvis = i + kv_len - qo_len + 1;
      if (nvis > kv_len) nvis = kv_len;
      float* o = out + (row * hq + h) * D;
      if (nvis <= 0) {
        for (int d = 0; d < D; ++d) o[d] = 0.f;
        continue;
      }
      const int64_t kvh = h / G;
      attend_row(q + row * q_st + h * q_sh, k_cache + kvh * kv_sh, v_cache + kvh * kv_sh, kv_ss,
                 indices + beg, nvis, D, sm_scale, o, scores, qf);
    }
    free(scores);
    free(qf);
  }
}

/* ---------- residual path ----------
 * RMSNorm::forward (src/layers/normalization.cu:236-269), fused add + RMSNorm
 * (:386-416) and silu_and_mul / gelu_and_mul (src/layers/activation.cu:8-77),
 * whose values FlashInfer v0.2.0.post1's norm / activation kernels compute in
 * fp32 and round once to the tensor type T (bf16 or fp16). Here values are
 * carried as fp32 arrays holding T-representable numbers; dtype 0 = bf16,
 * 1 = fp16. The sum of squares is accumulated in double (any fp32 order is
 * within the tests' one-ulp tolerance of it); the scale and products follow
 * the fp32 steps. */

/* Round to the nearest T value, ties to even. fp16: scale to the 11-bit
 * quantum of the value's binade (subnormal quantum 2^-24) and round there;
 * results above the largest finite fp16 (65504) become infinity. */
static float round_t(float x, int dtype) {
  if (dtype == 0) return bf16_to_f32(f32_to_bf16(x));
  if (isnan(x) || isinf(x) || x == 0.f) return x;
  const double a = fabs((double)x);
  int e;
  frexp(a, &e); /* a = m 2^e, m in [0.5, 1): leading bit 2^(e-1) */
  int lead = e - 1;
  if (lead < -14) lead = -14;
  const double quantum = ldexp(1.0, lead - 10);
  double r = nearbyint(a / quantum) * quantum;
  if (r > 65504.0) r = INFINITY;
  return (float)copysign(r, (double)x);
}

static void norm_row(const float* s, const float* w, float* out, int64_t d, float eps,
                     int dtype) {
  double acc = 0.0;
  for (int64_t i = 0; i < d; ++i) acc += (double)s[i] * (double)s[i];
  const float ss = (float)acc;
  const float scale = 1.0f / sqrtf(ss / (float)d + eps);
  for (int64_t i = 0; i < d; ++i) out[i] = round_t((s[i] * scale) * w[i], dtype);
}

/* out[r] = T(x[r] * rsqrt(mean(x[r]^2) + eps) * w); rows contiguous. */
void oracle_rmsnorm(const float* x, const float* w, float* out, int64_t rows, int64_t d,
                    float eps, int dtype) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) norm_row(x + r * d, w, out + r * d, d, eps, dtype);
}

/* s = x + residual (fp32); residual_out = T(s); x_out = T(norm(s) * w). */
void oracle_fused_add_rmsnorm(const float* x, const float* residual, const float* w,
                              float* x_out, float* residual_out, int64_t rows, int64_t d,
                              float eps, int dtype) {
#pragma omp parallel
  {
    float* s = (float*)malloc(sizeof(float) * (size_t)d);
#pragma omp for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
      for (int64_t i = 0; i < d; ++i) {
        s[i] = x[r * d + i] + residual[r * d + i];
        residual_out[r * d + i] = round_t(s[i], dtype);
      }
      norm_row(s, w, x_out + r * d, d, eps, dtype);
    }
    free(s);
  }
}

/* out[t, i] = T(act(in[t, i]) * in[t, d + i]); act 0 = silu x / (1 + e^-x),
 * act 1 = tanh GELU 0.5 x (1 + tanh(0.7978845608 (x + 0.044715 x^3))),
 * evaluated in double. in rows hold 2 d values, out rows d. */
void oracle_act_and_mul(const float* in, float* out, int64_t tokens, int64_t d, int act,
                        int dtype) {
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < tokens; ++t) {
    for (int64_t i = 0; i < d; ++i) {
      const double x = in[t * 2 * d + i], y = in[t * 2 * d + d + i];
      const double a = act == 0 ? x / (1.0 + exp(-x))
                                : 0.5 * x * (1.0 + tanh(0.7978845608 * (x + 0.044715 * x * x * x)));
      out[t * d + i] = round_t((float)(a * y), dtype);
    }
  }
}

void oracle_round_t(const float* in, float* out, int64_t n, int dtype) {
  for (int64_t i = 0; i < n; ++i) out[i] = round_t(in[i], dtype);
}

/* ---------- sampling from probabilities ----------
 * src/engine/sampling.cu:65-194 (FlashInfer v0.2.0.post1's SamplingFromProb,
 * TopK/TopP/TopKTopPSamplingFromProb, published algorithm): an inverse-CDF
 * draw over the probabilities above a threshold, and rejection rounds with
 * a rising pivot for the filtered draws. Running sums are kept in double:
 * exact for inputs whose partial sums are exact in fp32 (the dyadic
 * fixtures), and the true CDF otherwise; the fp32 kernels' sums differ
 * from it by their summation error only. The target u * q is rounded to
 * fp32, as the kernels compute it. */

static int64_t draw_row(const float* p, int64_t d, float thr, float u) {
  double agg = 0.0;
  for (int64_t i = 0; i < d; ++i) {
    if (p[i] > thr) {
      agg += p[i];
      if (agg > (double)u) return i;
    }
  }
  return d - 1;
}

/* mode 0 plain (uniform [batch]), 1 top-k (k from top_k_f or top_k_val),
 * 2 top-p, 3 top-k + top-p (k from top_k_i); uniform [rounds, batch]. */
void oracle_sample(const float* probs, const float* uniform, int32_t* out, uint8_t* success,
                   int64_t batch, int64_t d, int rounds, int mode, const float* top_k_f,
                   const int32_t* top_k_i, int top_k_val, const float* top_p_arr,
                   float top_p_val) {
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t b = 0; b < batch; ++b) {
    const float* p = probs + b * d;
    if (mode == 0) {
      out[b] = (int32_t)draw_row(p, d, 0.f, uniform[b]);
      continue;
    }
    int64_t k = top_k_val;
    if (top_k_f) k = (int64_t)(uint32_t)top_k_f[b];
    if (top_k_i) k = top_k_i[b];
    const float top_p = top_p_arr ? top_p_arr[b] : top_p_val;
    float pivot = 0.f, q = 1.f;
    int64_t sampled = d - 1, count = 0;
    int accepted = 0;
    for (int r = 0; r < rounds; ++r) {
      const float u = uniform[(int64_t)r * batch + b] * q;
      sampled = draw_row(p, d, pivot, u);
      if (p[sampled] > pivot) pivot = p[sampled];
      double qd = 0.0;
      count = 0;
      for (int64_t i = 0; i < d; ++i)
        if (p[i] > pivot) {
          qd += p[i];
          ++count;
        }
      q = (float)qd;
      if (mode == 1) accepted = count < k;
      else if (mode == 2) accepted = q < top_p;
      else accepted = count < k && q < top_p;
      if (accepted) break;
    }
    out[b] = (int32_t)sampled;
    if (success) success[b] = (uint8_t)accepted;
  }
}
