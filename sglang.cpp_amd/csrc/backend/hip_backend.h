// MI355X attention backend: the reference's BaseAttnBackend contract over the
// gfx950 HIP kernels of libsgl_attn.so. LibTorch tensors are containers only;
// all compute goes through the C ABI in include/sgl_attn.h.
//
// Replaces: FlashInferBackend (include/sglang/attention/flashinfer_backend.h:16-100,
//           src/attention/flashinfer_backend.cu), MHAKVCache
//           (include/sglang/kvcache/mha_kvcache.h:16-41), RMSNorm qk paths and
//           RotaryEmbedding (include/sglang/layers/{normalization,rotary_embedding}.h),
//           AttentionLayer::forward (src/layers/attention_layer.cc:17-51).
#pragma once

#include <c10/core/Stream.h>
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime.h>
#include <torch/torch.h>

#include <map>
#include <tuple>
#include <memory>
#include <vector>

#include "../../../include/sgl_attn.h"
#include "attn_types.h"

namespace sglang {

// Throws c10::Error (as TORCH_CHECK does) with the library's status text.
void check_sgl(int status, const char* what);

// KV pool [2, L, slots, Hkv, D]; k_cache(l) / v_cache(l) are [slots, Hkv, D].
// Slots = num_pages * page_size (token-granular, as the reference pool).
class MHAKVCache : public BaseKVCachePool {
 public:
  MHAKVCache(int num_kv_heads, int num_layers, int head_dim, int num_pages, int page_size,
             torch::Dtype dtype, torch::Device device);
  torch::Tensor k_cache(int layer_id) const override;
  torch::Tensor v_cache(int layer_id) const override;
  // k[t] -> k_cache[out_loc[t]], v likewise (src/kvcache/mha_kvcache.cu:111-155).
  void store_kv(const torch::Tensor& key, const torch::Tensor& val, const torch::Tensor& out_loc,
                int layer_id) override;
  torch::Device device() const override { return device_; }
  torch::Dtype dtype() const override { return kv_buffer_.scalar_type(); }
  int num_layers() const override { return num_layers_; }
  const torch::Tensor& buffer() const { return kv_buffer_; }

 private:
  torch::Tensor kv_buffer_;
  torch::Device device_;
  int num_layers_, kv_heads_, head_dim_;
};

// Per-batch metadata (the reference's FlashInferAttnMetadata,
// include/sglang/attention/flashinfer_backend.h:16-37).
struct HipAttnMetadata : public BaseAttnMetadata {
  bool is_prefill = false;
  std::vector<int> seq_lens, cached_lens;
  std::vector<int32_t> qo_indptr_host, kv_indptr_host;
  torch::Tensor indptr;  // qo_indptr (prefill) / kv_indptr (decode), device
  torch::Tensor last_rows;  // row of each request's last query token, device

  // Decode rows: every request of a decode batch, and the qo_len == 1
  // requests of a prefill-phase batch (mixed chunked-prefill + decode steps).
  int num_decode = 0;
  torch::Tensor dec_kv_indptr, dec_indices, dec_q_rows, dec_table_idx;
  sgl_decode_plan_t dec_plan{};
  // Mixed batches run as one launch (sgl_paged_mixed) with the decode rows
  // on dec_cus CUs; otherwise decode and prefill are separate launches.
  bool fused = false;
  int dec_cus = 0;

  // Prefill rows: requests of a prefill-phase batch with qo_len > 1.
  int num_prefill = 0;
  int max_qo_len = 0;
  torch::Tensor pre_qo_indptr, pre_kv_indptr, pre_indices, pre_q_start, pre_table_idx;

  bool use_capture_buffers = false;
  int64_t capture_tokens = 0;  // query rows of the captured step (replays may use fewer)
  std::vector<torch::Tensor> host_staging;  // pinned buffers of pending H2D copies

  torch::Tensor get_last_indices(int bs) const override;
  // Marks the device tensors as used on `stream` (the scheduler prepares
  // metadata on its own stream; scheduler.cc:152-179 does this by downcast).
  void record_stream(const c10::hip::HIPStream& stream) const;
};

class HipAttnBackend : public BaseAttnBackend {
 public:
  HipAttnBackend(std::shared_ptr<BaseKVCachePool> kv_cache, int num_qo_heads, int num_kv_heads,
                 int head_dim);
  ~HipAttnBackend() override;
  HipAttnBackend(const HipAttnBackend&) = delete;
  HipAttnBackend& operator=(const HipAttnBackend&) = delete;

  // Context::page_table (include/sglang/core/context.h:19-20): [rows, W] int32,
  // token-granular, device.
  void set_page_table(const torch::Tensor& page_table);

  void prepare_metadata(Batch& batch) override;
  torch::Tensor forward(const torch::Tensor& q, const torch::Tensor& k, const torch::Tensor& v,
                        int layer_id, Batch& batch) override;
  void init_capture_graph(int max_seq_len, const std::vector<int>& bs_list) override;
  // Fixed-address buffers for capturing mixed steps (prefill-phase batches:
  // qo_len == 1 rows beside chunked-prefill requests): up to max_decode_rows
  // decode rows and max_prefill_reqs prefill requests of at most
  // max_prefill_qo new tokens, every request at most max_seq_len long. After
  // this, prepare_for_capture / prepare_for_replay accept prefill-phase
  // batches; a graph replays any batch with the captured (decode rows,
  // prefill requests) counts and no more query rows than it was captured with.
  void init_mixed_capture_graph(int max_seq_len, int max_decode_rows, int max_prefill_reqs,
                                int max_prefill_qo);
  void prepare_for_capture(Batch& batch) override;
  void prepare_for_replay(Batch& batch) override;

  // GraphRunner::pad_batch (src/engine/engine.cc:628-645) for mixed steps:
  // appends copies of `dummy` (the reference's dummy_req_: table_idx the page
  // table's spare row, whose columns all hold the spare slot; cached_len 0,
  // device_len 1, hence one query row over the spare slot) until the
  // batch's decode rows reach the smallest captured mixed step with the same
  // number of prefill requests. The caller extends positions / out_loc with
  // one token per dummy (position 0, the spare slot), as the reference's
  // prepare_batch does over padded_reqs. Returns false, batch unchanged, when
  // no captured step fits.
  bool pad_mixed_batch(Batch& batch, const std::shared_ptr<Req>& dummy) const;

  // Attention over the pool only (K/V of the new tokens already stored, e.g.
  // by the fused norm + RoPE + store pass). q: [T, Hq, D] view; returns
  // [T, Hq * D].
  torch::Tensor attend(const torch::Tensor& q, int layer_id, Batch& batch);

  // Mixed batches: one launch with the decode rows on a share of the CUs and
  // the prefill rows on the others (default on, for kv-head counts dividing
  // 8); otherwise, with overlap_mixed, the prefill rows on a side stream
  // beside the decode launch (default on).
  void set_fused_mixed(bool on) { fused_mixed_ = on; }
  bool fused_mixed() const { return fused_mixed_; }
  void set_overlap_mixed(bool on) { overlap_mixed_ = on; }
  bool overlap_mixed() const { return overlap_mixed_; }

  int num_qo_heads() const { return num_qo_heads_; }
  int num_kv_heads() const { return num_kv_heads_; }
  int head_dim() const { return head_dim_; }
  const std::shared_ptr<BaseKVCachePool>& kv_cache() const { return kv_cache_; }

 private:
  std::shared_ptr<HipAttnMetadata> metadata_of(Batch& batch) const;
  torch::Tensor& workspace(int64_t bytes);
  torch::Tensor to_device(const std::vector<int32_t>& host, HipAttnMetadata& meta);

  void prepare_mixed_for_capture(Batch& batch);
  void prepare_mixed_for_replay(Batch& batch);
  void check_mixed_capacity(const HipAttnMetadata& m) const;
  void copy_contents(HipAttnMetadata& dst, const HipAttnMetadata& src);

  struct MixedCapture {
    int max_seq_len = 0, max_dec = 0, max_pre = 0, max_qo = 0;
    torch::Tensor qo_indptr;                                  // [max_dec + max_pre + 1]
    torch::Tensor dec_kv_indptr, dec_indices, dec_q_rows;     // decode rows
    torch::Tensor pre_qo_indptr, pre_kv_indptr, pre_q_start, pre_indices;  // prefill rows
    torch::Tensor workspace;  // decode split workspace of the largest plan
    std::map<std::pair<int, int>, std::shared_ptr<HipAttnMetadata>> metadata;
  };
  std::unique_ptr<MixedCapture> mixed_;

  struct CaptureState {
    int max_seq_len = 0;
    int max_bs = 0;
    torch::Tensor kv_indptr;  // [max_bs + 1]
    torch::Tensor indices;    // [max_bs * max_seq_len]
    torch::Tensor q_rows;     // [max_bs]: 0..max_bs-1
    torch::Tensor workspace;  // decode split workspace of the largest captured plan
    std::map<int, sgl_decode_plan_t> plans;
    std::map<int, std::shared_ptr<HipAttnMetadata>> metadata;
  };

  std::shared_ptr<BaseKVCachePool> kv_cache_;
  int num_qo_heads_, num_kv_heads_, head_dim_;
  torch::Tensor page_table_;
  torch::Tensor workspace_;
  // Set once the growable workspace has been recorded into a graph: growing
  // it then keeps the old buffer alive (a graph may still write to it) until
  // the next init_capture_graph / init_mixed_capture_graph, before which the
  // caller destroys the graphs it captured.
  bool workspace_captured_ = false;
  std::vector<torch::Tensor> retired_workspaces_;
  std::unique_ptr<CaptureState> capture_;
  // Side stream and fork/join events for mixed batches (created on first use).
  void* side_stream();
  void* side_stream_ = nullptr;
  bool overlap_mixed_ = true;
  bool fused_mixed_ = true;
  int device_cus_ = 256;
  hipEvent_t fork_event_ = nullptr;
  hipEvent_t join_event_ = nullptr;
};

// CacheManager::write_page_table (src/scheduler/prefill.cc:144-187): the
// scheduler's host list of allocated page starts and (table_idx, first_page,
// last_page) tuples go up in one pinned copy of num_pages + 3 n ints, and the
// device expands pages to token slots (sgl_write_page_table) -- instead of
// the reference's host loop and three token-sized copies. Same checks: the
// allocations take exactly the pages given.
void write_page_table(const torch::Tensor& page_table, const std::vector<int32_t>& allocated_pages,
                      const std::vector<std::tuple<int, int, int>>& allocation_info,
                      int page_size);

// RMSNorm module (weight [size], bf16 by default; fp16 weights serve fp16
// activations). The q/k path is bf16 only.
class RMSNorm {
 public:
  RMSNorm(int size, float eps, torch::Device device);
  torch::Tensor forward(const torch::Tensor& x) const;            // normalization.cu:236-241
  void forward_inplace(torch::Tensor& x) const;                   // normalization.cu:243-269
  void forward_inplace_3d_strided(torch::Tensor& x) const;        // normalization.cu:271-316
  void fused_add_forward_inplace(torch::Tensor& x, torch::Tensor& residual) const;  // :386-416
  float eps() const { return eps_; }
  torch::Tensor weight;

 private:
  float eps_;
};

// normalization.cu:318-384
void fused_qk_rmsnorm_inplace_3d_strided(torch::Tensor& q, torch::Tensor& k, const RMSNorm& q_norm,
                                         const RMSNorm& k_norm);

// Gated activations of the MLP: out [T, d] = act(input[:, :d]) * input[:, d:]
// (activation.cu:15-77), bf16 or fp16.
void silu_and_mul(torch::Tensor& out, const torch::Tensor& input);
void gelu_and_mul(torch::Tensor& out, const torch::Tensor& input);

// Sampling from probabilities, the reference's Sampler kernels
// (include/sglang/engine/sampling.h:7-36, src/engine/sampling.cu:65-194):
// same names, arguments and checks; the HIP kernels replace FlashInfer's.
struct FlashInferSamplingResult {
  torch::Tensor samples;
  torch::Tensor success;
};
torch::Tensor flashinfer_sample_from_probs(const torch::Tensor& probs,
                                           const torch::Tensor& uniform_samples, bool deterministic);
FlashInferSamplingResult flashinfer_top_k_sample_from_probs(const torch::Tensor& probs,
                                                            const torch::Tensor& uniform_samples,
                                                            const torch::Tensor& top_k,
                                                            int64_t top_k_value, bool deterministic);
FlashInferSamplingResult flashinfer_top_p_sample_from_probs(const torch::Tensor& probs,
                                                            const torch::Tensor& uniform_samples,
                                                            const torch::Tensor& top_p,
                                                            double top_p_value, bool deterministic);
FlashInferSamplingResult flashinfer_top_k_top_p_sample_from_probs(
    const torch::Tensor& probs, const torch::Tensor& uniform_samples, const torch::Tensor& top_k,
    double top_k_value, const torch::Tensor& top_p, double top_p_value, bool deterministic);

// The probabilities Sampler::sample hands to the draws above:
// softmax(logits.to(kFloat32) / temperatures, -1) (src/engine/engine.cc:306-308),
// one device pass (logits bf16, fp16 or fp32 [batch, vocab]; temperatures
// [batch] or [batch, 1], any floating type, on the logits' device).
torch::Tensor sampling_probs(const torch::Tensor& logits, const torch::Tensor& temperatures);

// Sampler::sample's probabilities and draw in one launch (engine.cc:306-333):
// the draw the reference picks from which of top_k / top_p are defined
// (both: top_k as int32; top_k only: as float32), uniform_samples [batch]
// for the plain draw or [rounds, batch] otherwise; the probabilities are
// sampling_probs' bits and are not stored. success is undefined for the
// plain draw.
FlashInferSamplingResult sample_from_logits(const torch::Tensor& logits,
                                            const torch::Tensor& temperatures,
                                            const torch::Tensor& uniform_samples,
                                            const torch::Tensor& top_k, const torch::Tensor& top_p);

// NeoX RoPE with a half-width fp32 cos/sin cache built on the device
// (rotary_embedding.cu:75-94 builds the same table with LibTorch-CPU ops).
class RotaryEmbedding {
 public:
  RotaryEmbedding(int head_size, int rotary_dim, int max_position_embeddings, float base,
                  torch::Device device);
  void forward_inplace(const torch::Tensor& positions, torch::Tensor& query,
                       torch::Tensor& key) const;
  const torch::Tensor& cos_cache() const { return cos_cache_; }
  const torch::Tensor& sin_cache() const { return sin_cache_; }
  int rotary_dim() const { return rotary_dim_; }

 private:
  int head_size_, rotary_dim_;
  torch::Tensor cos_cache_, sin_cache_;
};

// qkv [T, (Hq + 2 Hkv) D] -> o [T, Hq D]: qk-norm, RoPE and the KV store in
// one fused pass, then paged attention (attention_layer.cc:17-51).
class AttentionLayer {
 public:
  AttentionLayer(int layer_id, int num_qo_heads, int num_kv_heads, int head_dim,
                 std::shared_ptr<HipAttnBackend> backend, std::shared_ptr<RotaryEmbedding> rotary,
                 std::shared_ptr<RMSNorm> q_norm, std::shared_ptr<RMSNorm> k_norm);
  torch::Tensor forward(const torch::Tensor& qkv, const torch::Tensor& positions, Batch& batch);

 private:
  int layer_id_, num_qo_heads_, num_kv_heads_, head_dim_;
  std::shared_ptr<HipAttnBackend> backend_;
  std::shared_ptr<RotaryEmbedding> rotary_;
  std::shared_ptr<RMSNorm> q_norm_, k_norm_;
};

}  // namespace sglang
