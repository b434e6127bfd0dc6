// Host-side types of the attention boundary, mirroring the reference's
// interface so HipAttnBackend is a drop-in for its FlashInfer backend.
//
//   BaseAttnMetadata / BaseAttnBackend  include/sglang/attention/backend.h:16-41
//   BaseKVCachePool                     include/sglang/kvcache/base.h:78-90
//   Req (fields the backend reads)      include/sglang/core/req.h:13-58, src/core/req.cc:126-140
//   Batch / BatchPhase                  include/sglang/core/batch.h:11-37
//
// Only the members the attention path touches are declared. When the backend
// is linked into the reference's Engine, the reference's own headers take the
// place of this file (same names, same member meaning).
#pragma once

#include <torch/torch.h>

#include <cstdint>
#include <memory>
#include <vector>

namespace sglang {

struct Batch;

struct BaseAttnMetadata {
  virtual ~BaseAttnMetadata() = default;
  // Row of the last query token of each of the first bs requests
  // (lm-head selection, src/models/utils.cc:8-19).
  virtual torch::Tensor get_last_indices(int bs) const = 0;
};

class BaseAttnBackend {
 public:
  virtual ~BaseAttnBackend() = default;
  virtual torch::Tensor forward(const torch::Tensor& q, const torch::Tensor& k,
                                const torch::Tensor& v, int layer_id, Batch& batch) = 0;
  virtual void prepare_metadata(Batch& batch) = 0;
  virtual void init_capture_graph(int max_seq_len, const std::vector<int>& bs_list) = 0;
  virtual void prepare_for_capture(Batch& batch) = 0;
  virtual void prepare_for_replay(Batch& batch) = 0;
};

class BaseKVCachePool {
 public:
  virtual ~BaseKVCachePool() = default;
  virtual torch::Tensor k_cache(int layer_id) const = 0;
  virtual torch::Tensor v_cache(int layer_id) const = 0;
  virtual void store_kv(const torch::Tensor& key, const torch::Tensor& val,
                        const torch::Tensor& out_loc, int layer_id) = 0;
  virtual torch::Device device() const = 0;
  virtual torch::Dtype dtype() const = 0;
  virtual int num_layers() const = 0;
};

struct Req {
  int table_idx = -1;  // row of the page table
  int cached_len = 0;  // tokens already in the KV cache
  int device_len_ = 0; // tokens the request has on the device (cached + new)

  int device_len() const { return device_len_; }
  int extend_len() const { return device_len_ - cached_len; }
};

enum class BatchPhase : std::uint8_t { Prefill, Decode };

struct Batch {
  BatchPhase phase = BatchPhase::Prefill;
  std::vector<std::shared_ptr<Req>> padded_reqs;
  torch::Tensor positions;  // [T] int32, device
  torch::Tensor out_loc;    // [T] int32 / int64, device: KV slot of each new token
  std::shared_ptr<BaseAttnMetadata> attn_metadata;

  bool is_prefill() const { return phase == BatchPhase::Prefill; }
  bool is_decode() const { return phase == BatchPhase::Decode; }
  int padded_size() const { return static_cast<int>(padded_reqs.size()); }
};

}  // namespace sglang
