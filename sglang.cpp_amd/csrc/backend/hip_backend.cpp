// MI355X attention backend over libsgl_attn.so (see hip_backend.h).
#include "hip_backend.h"

#include <ATen/hip/HIPContext.h>
#include <c10/hip/HIPCachingAllocator.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>

namespace sglang {
namespace {

void* current_stream(const torch::Device& dev) {
  return static_cast<void*>(at::hip::getCurrentHIPStream(dev.index()).stream());
}

const torch::TensorOptions kI32 = torch::TensorOptions().dtype(torch::kInt32);

void check_bf16(const torch::Tensor& t, const char* what) {
  // The reference backend hard-codes bf16 and would reinterpret fp16 data;
  // this one refuses it instead.
  TORCH_CHECK(t.scalar_type() == torch::kBFloat16, what, " must be bf16, got ", t.scalar_type());
}

}  // namespace

void check_hip(hipError_t status, const char* what) {
  TORCH_CHECK(status == hipSuccess, what, " failed: ", hipGetErrorString(status));
}

void check_sgl(int status, const char* what) {
  TORCH_CHECK(status == SGL_OK, what, " failed: ", sgl_status_string(status), " (status ", status,
              ")");
}

// ---------------------------------------------------------------- KV pool

MHAKVCache::MHAKVCache(int num_kv_heads, int num_layers, int head_dim, int num_pages,
                       int page_size, torch::Dtype dtype, torch::Device device)
    : device_(device), num_layers_(num_layers), kv_heads_(num_kv_heads), head_dim_(head_dim) {
  TORCH_CHECK(num_kv_heads > 0 && num_layers > 0 && head_dim > 0 && num_pages > 0 &&
                  page_size > 0,
              "MHAKVCache: sizes must be positive");
  const int64_t slots = static_cast<int64_t>(num_pages) * page_size;
  kv_buffer_ = torch::empty({2, num_layers, slots, num_kv_heads, head_dim},
                            torch::TensorOptions().dtype(dtype).device(device));
}

torch::Tensor MHAKVCache::k_cache(int layer_id) const { return kv_buffer_[0][layer_id]; }
torch::Tensor MHAKVCache::v_cache(int layer_id) const { return kv_buffer_[1][layer_id]; }

void MHAKVCache::store_kv(const torch::Tensor& key, const torch::Tensor& val,
                          const torch::Tensor& out_loc, int layer_id) {
  // Same checks as the reference (src/kvcache/mha_kvcache.cu:111-141).
  TORCH_CHECK(key.is_cuda() && val.is_cuda() && out_loc.is_cuda(),
              "key, val and out_loc must be device tensors");
  TORCH_CHECK(key.scalar_type() == val.scalar_type(), "key and val dtype must match");
  TORCH_CHECK(key.scalar_type() == kv_buffer_.scalar_type(), "key dtype must match the pool");
  TORCH_CHECK(key.stride(-1) == 1 && val.stride(-1) == 1,
              "key and val last dimension must be contiguous");
  TORCH_CHECK(out_loc.dim() == 1, "out_loc must be rank 1");
  auto k = key.dim() == 2 ? key.view({-1, kv_heads_, head_dim_}) : key;
  auto v = val.dim() == 2 ? val.view({-1, kv_heads_, head_dim_}) : val;
  TORCH_CHECK(k.dim() == 3 && v.dim() == 3, "key and val must be rank 2 or 3");
  TORCH_CHECK(k.size(0) == v.size(0) && k.size(0) == out_loc.size(0),
              "key, val and out_loc token counts must match");
  TORCH_CHECK(k.size(1) == kv_heads_ && v.size(1) == kv_heads_ && k.size(2) == head_dim_ &&
                  v.size(2) == head_dim_,
              "key and val shape must match KV cache layout");
  TORCH_CHECK(layer_id >= 0 && layer_id < num_layers_, "layer_id out of range");
  const int64_t tokens = k.size(0);
  if (tokens == 0) return;
  int index_dtype;
  if (out_loc.scalar_type() == torch::kInt32) {
    index_dtype = SGL_INDEX_I32;
  } else {
    TORCH_CHECK(out_loc.scalar_type() == torch::kInt64, "out_loc must be int32 or int64");
    index_dtype = SGL_INDEX_I64;
  }
  auto kb = k_cache(layer_id);
  auto vb = v_cache(layer_id);
  check_sgl(sgl_store_kv(kb.data_ptr(), vb.data_ptr(), k.data_ptr(), v.data_ptr(),
                         out_loc.data_ptr(), index_dtype, tokens,
                         static_cast<int64_t>(kv_heads_) * head_dim_, k.stride(0), v.stride(0),
                         current_stream(device_)),
            "sgl_store_kv");
}

// ---------------------------------------------------------------- metadata

torch::Tensor HipAttnMetadata::get_last_indices(int bs) const {
  // Same as the reference (flashinfer_backend.cu:83-85): indptr[1 .. bs] - 1.
  return indptr.slice(0, 1, bs + 1) - 1;
}

void HipAttnMetadata::record_stream(const c10::hip::HIPStream& stream) const {
  for (const torch::Tensor* t : {&indptr, &last_rows, &dec_kv_indptr, &dec_indices, &dec_q_rows,
                                 &dec_table_idx, &pre_qo_indptr, &pre_kv_indptr, &pre_indices,
                                 &pre_q_start, &pre_table_idx}) {
    if (t->defined() && t->is_cuda() && t->numel() > 0)
      c10::hip::HIPCachingAllocator::recordStream(t->storage().data_ptr(), stream);
  }
}

// ---------------------------------------------------------------- backend

void* HipAttnBackend::side_stream() {
  if (!side_stream_) {
    // A pool stream at the default priority (streams of other priorities
    // are avoided on purpose).
    side_stream_ = at::hip::getStreamFromPool(/*isHighPriority=*/false,
                                              kv_cache_->device().index())
                       .stream();
    check_hip(hipEventCreateWithFlags(&fork_event_, hipEventDisableTiming), "hipEventCreate");
    check_hip(hipEventCreateWithFlags(&join_event_, hipEventDisableTiming), "hipEventCreate");
  }
  return side_stream_;
}

HipAttnBackend::~HipAttnBackend() {
  if (fork_event_) (void)hipEventDestroy(fork_event_);
  if (join_event_) (void)hipEventDestroy(join_event_);
}

HipAttnBackend::HipAttnBackend(std::shared_ptr<BaseKVCachePool> kv_cache, int num_qo_heads,
                               int num_kv_heads, int head_dim)
    : kv_cache_(std::move(kv_cache)),
      num_qo_heads_(num_qo_heads),
      num_kv_heads_(num_kv_heads),
      head_dim_(head_dim) {
  TORCH_CHECK(kv_cache_, "HipAttnBackend needs a KV pool");
  TORCH_CHECK(num_qo_heads > 0 && num_kv_heads > 0 && num_qo_heads % num_kv_heads == 0,
              "num_qo_heads must be a positive multiple of num_kv_heads");
  TORCH_CHECK(head_dim == 128, "HipAttnBackend is built for head_dim 128");
  TORCH_CHECK(kv_cache_->dtype() == torch::kBFloat16, "HipAttnBackend needs a bf16 KV pool");
  int cus = 0;
  if (kv_cache_->device().is_cuda() &&
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount,
                            kv_cache_->device().index()) == hipSuccess &&
      cus > 0)
    device_cus_ = cus;
}

void HipAttnBackend::set_page_table(const torch::Tensor& page_table) {
  TORCH_CHECK(page_table.dim() == 2 && page_table.scalar_type() == torch::kInt32 &&
                  page_table.stride(1) == 1,
              "page table must be a 2-D int32 tensor with unit column stride");
  TORCH_CHECK(page_table.device() == kv_cache_->device(), "page table must be on the pool device");
  page_table_ = page_table;
}

torch::Tensor& HipAttnBackend::workspace(int64_t bytes) {
  if (!workspace_.defined() || workspace_.numel() < bytes) {
    if (workspace_captured_ && workspace_.defined()) {
      retired_workspaces_.push_back(workspace_);
      workspace_captured_ = false;
    }
    workspace_ = torch::empty({std::max<int64_t>(bytes, 256)},
                              torch::TensorOptions().dtype(torch::kUInt8).device(
                                  kv_cache_->device()));
  }
  return workspace_;
}

std::shared_ptr<HipAttnMetadata> HipAttnBackend::metadata_of(Batch& batch) const {
  auto meta = std::dynamic_pointer_cast<HipAttnMetadata>(batch.attn_metadata);
  TORCH_CHECK(meta, "HipAttnBackend requires HipAttnMetadata (call prepare_metadata first)");
  return meta;
}

namespace {

// Fields of one upload start at multiples of 64 int32 (256 bytes).
constexpr int64_t kFieldAlign = 64;
int64_t align_field(int64_t n) { return (n + kFieldAlign - 1) / kFieldAlign * kFieldAlign; }

// One step's host int32 metadata, gathered so that it reaches the device in
// a single pinned copy; the device tensor continues past the uploaded
// fields with room the kernels fill (the index arrays).
class PackedUpload {
 public:
  // Appends v and returns its offset; pad = false lets the next field
  // follow it directly (two fields then read as one array).
  int64_t add(const std::vector<int32_t>& v, bool pad = true) {
    const int64_t off = static_cast<int64_t>(host_.size());
    host_.insert(host_.end(), v.begin(), v.end());
    if (pad) host_.resize(align_field(static_cast<int64_t>(host_.size())), 0);
    return off;
  }
  int64_t size() const { return static_cast<int64_t>(host_.size()); }
  // [uploaded fields | device_only entries] on dev; the pinned source stays
  // alive in `staging` until the copy has run (the pinned allocator also
  // records the copy's stream).
  torch::Tensor send(int64_t device_only, const torch::Device& dev,
                     std::vector<torch::Tensor>& staging) {
    const int64_t n = size();
    auto out = torch::empty({std::max<int64_t>(n + device_only, 1)}, kI32.device(dev));
    if (n > 0) {
      auto pinned = torch::empty({n}, kI32.pinned_memory(true));
      std::memcpy(pinned.data_ptr<int32_t>(), host_.data(), sizeof(int32_t) * n);
      out.slice(0, 0, n).copy_(pinned, /*non_blocking=*/true);
      staging.push_back(std::move(pinned));
    }
    return out;
  }

 private:
  std::vector<int32_t> host_;
};

}  // namespace

torch::Tensor HipAttnBackend::to_device(const std::vector<int32_t>& host, HipAttnMetadata& meta) {
  PackedUpload up;
  up.add(host, false);
  return up.send(0, kv_cache_->device(), meta.host_staging).slice(0, 0, host.size());
}

void HipAttnBackend::prepare_metadata(Batch& batch) {
  TORCH_CHECK(page_table_.defined(), "HipAttnBackend: set_page_table() first");
  auto meta = std::make_shared<HipAttnMetadata>();
  meta->is_prefill = batch.is_prefill();
  const int bs = batch.padded_size();
  meta->seq_lens.resize(bs);
  meta->cached_lens.resize(bs);
  meta->kv_indptr_host.assign(bs + 1, 0);
  for (int i = 0; i < bs; ++i) {
    const auto& req = batch.padded_reqs[i];
    meta->seq_lens[i] = req->device_len();
    meta->cached_lens[i] = req->cached_len;
    meta->kv_indptr_host[i + 1] = meta->kv_indptr_host[i] + req->device_len();
  }

  // Which requests go to which kernel. Decode batches (flashinfer_backend.cu:
  // 408-464): every request, query row i. Prefill batches (:466-519):
  // qo_len = max(1, extend), kv_len = device_len, and with no cache hit
  // anywhere qo_indptr = kv_indptr; one-token requests go to the split-KV
  // decode kernel, the rest to the causal prefill kernel (each writes its
  // own rows of o).
  std::vector<int> dec, pre;
  if (batch.is_decode()) {
    dec.resize(bs);
    for (int i = 0; i < bs; ++i) dec[i] = i;
    meta->qo_indptr_host.resize(bs + 1);
    for (int i = 0; i <= bs; ++i) meta->qo_indptr_host[i] = i;
  } else {
    bool all_no_cache_hit = true;
    for (int i = 0; i < bs; ++i) all_no_cache_hit = all_no_cache_hit && batch.padded_reqs[i]->cached_len == 0;
    if (all_no_cache_hit) {
      meta->qo_indptr_host = meta->kv_indptr_host;
    } else {
      meta->qo_indptr_host.assign(bs + 1, 0);
      for (int i = 0; i < bs; ++i)
        meta->qo_indptr_host[i + 1] =
            meta->qo_indptr_host[i] + std::max(1, batch.padded_reqs[i]->extend_len());
    }
    for (int i = 0; i < bs; ++i)
      (meta->qo_indptr_host[i + 1] - meta->qo_indptr_host[i] == 1 ? dec : pre).push_back(i);
  }
  const int nd = static_cast<int>(dec.size()), np = static_cast<int>(pre.size());

  // Both kinds of rows: one launch with the decode rows on the CU share
  // their K/V bytes need next to the prefill's flops.
  if (nd > 0 && np > 0 && fused_mixed_ && num_kv_heads_ <= 8 && 8 % num_kv_heads_ == 0) {
    int64_t dec_tokens = 0;
    for (int i : dec) dec_tokens += batch.padded_reqs[i]->device_len();
    double flops = 0.0;
    for (int i : pre) {
      const double qo = meta->qo_indptr_host[i + 1] - meta->qo_indptr_host[i];
      const double kv = batch.padded_reqs[i]->device_len();
      flops += qo * (kv - qo) + qo * (qo + 1) / 2;
    }
    flops *= 4.0 * head_dim_ * num_qo_heads_;
    const int h = sgl_mixed_decode_cus(dec_tokens, num_kv_heads_, head_dim_, flops);
    if (h < device_cus_) {
      meta->fused = true;
      meta->dec_cus = h;
    }
  }

  // Host fields of both kinds of rows, then one upload.
  std::vector<int32_t> dec_ip(nd + 1, 0), dec_rows(nd), pre_qo(np + 1, 0), pre_ip(np + 1, 0),
      pre_start(np), table(nd + np);
  for (int i = 0; i < nd; ++i) {
    const auto& req = batch.padded_reqs[dec[i]];
    dec_ip[i + 1] = dec_ip[i] + req->device_len();
    dec_rows[i] = meta->qo_indptr_host[dec[i]];
    table[i] = req->table_idx;
  }
  int max_qo = 0;
  for (int i = 0; i < np; ++i) {
    const int r = pre[i];
    const auto& req = batch.padded_reqs[r];
    const int q_len = meta->qo_indptr_host[r + 1] - meta->qo_indptr_host[r];
    pre_qo[i + 1] = pre_qo[i] + q_len;
    pre_ip[i + 1] = pre_ip[i] + req->device_len();
    pre_start[i] = meta->qo_indptr_host[r];
    table[nd + i] = req->table_idx;
    max_qo = std::max(max_qo, q_len);
  }
  // The index arrays: decode rows' indices, then (from a 256-byte boundary)
  // the prefill rows'. One gather fills both: its kv_indptr runs over the
  // decode rows and continues at the prefill base, so the last decode row's
  // gather also fills the padding gap (page-table values, never read).
  const int64_t dec_total = dec_ip[nd], pre_total = pre_ip[np];
  const int64_t pre_base = nd > 0 ? align_field(std::max<int64_t>(dec_total, 1)) : 0;
  TORCH_CHECK(pre_base + pre_total <= 0x7fffffff, "batch KV tokens exceed int32 offsets");
  PackedUpload up;
  const int64_t o_qo = batch.is_prefill() ? up.add(meta->qo_indptr_host) : -1;
  const int64_t o_dip = up.add(dec_ip), o_drows = up.add(dec_rows);
  const int64_t o_pqo = up.add(pre_qo), o_pip = up.add(pre_ip), o_pstart = up.add(pre_start);
  const int64_t o_table = up.add(table);
  int64_t o_gather_ip = o_dip;  // decode rows only
  if (np > 0 && nd == 0) o_gather_ip = o_pip;
  if (np > 0 && nd > 0) {
    std::vector<int32_t> both(nd + np + 1);
    for (int i = 0; i < nd; ++i) both[i] = dec_ip[i];
    for (int i = 0; i <= np; ++i) both[nd + i] = static_cast<int32_t>(pre_base + pre_ip[i]);
    o_gather_ip = up.add(both);
  }
  const int64_t o_ind = up.size();
  const int64_t ind_len = pre_base + (np > 0 ? std::max<int64_t>(pre_total, 1) : 0);
  auto dev = up.send(std::max<int64_t>(ind_len, 1), kv_cache_->device(), meta->host_staging);
  auto field = [&](int64_t off, int64_t n) { return dev.slice(0, off, off + n); };
  if (nd + np > 0)
    check_sgl(sgl_build_decode_indices(page_table_.data_ptr<int32_t>(), page_table_.size(0),
                                       page_table_.stride(0), page_table_.size(1),
                                       dev.data_ptr<int32_t>() + o_table,
                                       dev.data_ptr<int32_t>() + o_gather_ip,
                                       dev.data_ptr<int32_t>() + o_ind, nd + np,
                                       current_stream(kv_cache_->device())),
              "sgl_build_decode_indices");

  if (nd > 0 || batch.is_decode()) {
    meta->num_decode = nd;
    meta->dec_kv_indptr = field(o_dip, nd + 1);
    meta->dec_q_rows = field(o_drows, nd);
    meta->dec_table_idx = field(o_table, nd);
    meta->dec_indices = field(o_ind, std::max<int64_t>(dec_total, 1));
    if (meta->fused)
      check_sgl(sgl_decode_plan_cus(dec_ip.data(), nd, num_qo_heads_, num_kv_heads_, head_dim_,
                                    meta->dec_cus, &meta->dec_plan),
                "sgl_decode_plan_cus");
    else
      check_sgl(sgl_decode_plan(dec_ip.data(), nd, num_qo_heads_, num_kv_heads_, head_dim_,
                                &meta->dec_plan),
                "sgl_decode_plan");
    // The split workspace grows in forward, on the stream that uses it: a
    // scheduler that prepares step n + 1 on its own stream while step n's
    // forward runs must not free the buffer that forward is using.
  }
  if (np > 0) {
    meta->num_prefill = np;
    meta->max_qo_len = max_qo;
    meta->pre_qo_indptr = field(o_pqo, np + 1);
    meta->pre_kv_indptr = field(o_pip, np + 1);
    meta->pre_q_start = field(o_pstart, np);
    meta->pre_table_idx = field(o_table + nd, np);
    meta->pre_indices = field(o_ind + pre_base, std::max<int64_t>(pre_total, 1));
  }
  meta->indptr = batch.is_prefill() ? field(o_qo, bs + 1) : meta->dec_kv_indptr;
  batch.attn_metadata = meta;
}

torch::Tensor HipAttnBackend::forward(const torch::Tensor& q, const torch::Tensor& k,
                                      const torch::Tensor& v, int layer_id, Batch& batch) {
  // Reference: FlashInferBackend::forward (flashinfer_backend.cu:522-681):
  // store the new tokens' K/V, then paged attention over the pool. A batch
  // without metadata is refused before the store.
  metadata_of(batch);
  auto k_3d = k.dim() == 2 ? k.view({-1, num_kv_heads_, head_dim_}) : k;
  auto v_3d = v.dim() == 2 ? v.view({-1, num_kv_heads_, head_dim_}) : v;
  kv_cache_->store_kv(k_3d, v_3d, batch.out_loc, layer_id);
  return attend(q.view({-1, num_qo_heads_, head_dim_}), layer_id, batch);
}

torch::Tensor HipAttnBackend::attend(const torch::Tensor& q_in, int layer_id, Batch& batch) {
  auto meta = metadata_of(batch);
  auto q = q_in.dim() == 2 ? q_in.view({-1, num_qo_heads_, head_dim_}) : q_in;
  check_bf16(q, "q");
  TORCH_CHECK(q.dim() == 3 && q.size(1) == num_qo_heads_ && q.size(2) == head_dim_ &&
                  q.stride(2) == 1,
              "q must be [T, num_qo_heads, head_dim] with a contiguous last dim");
  auto o = torch::empty({q.size(0), num_qo_heads_, head_dim_}, q.options());
  auto kc = kv_cache_->k_cache(layer_id).view({-1, num_kv_heads_, head_dim_});
  auto vc = kv_cache_->v_cache(layer_id).view({-1, num_kv_heads_, head_dim_});
  void* stream = current_stream(kv_cache_->device());
  const float sm_scale = 1.0f / std::sqrt(static_cast<float>(head_dim_));
  if (meta->fused) {
    // Decode units and prefill items in one launch (decode on dec_cus CUs).
    torch::Tensor& ws = !meta->use_capture_buffers ? workspace(meta->dec_plan.workspace_bytes)
                                                   : mixed_->workspace;
    if (!meta->use_capture_buffers) {
      hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
      check_hip(hipStreamIsCapturing(static_cast<hipStream_t>(stream), &cs),
                "hipStreamIsCapturing");
      if (cs != hipStreamCaptureStatusNone) workspace_captured_ = true;
    }
    TORCH_CHECK(ws.numel() >= meta->dec_plan.workspace_bytes, "decode workspace too small");
    check_sgl(sgl_paged_mixed(&meta->dec_plan, q.data_ptr(), q.stride(0), q.stride(1),
                              kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1),
                              meta->dec_indices.data_ptr<int32_t>(),
                              meta->dec_kv_indptr.data_ptr<int32_t>(),
                              meta->dec_q_rows.data_ptr<int32_t>(), meta->num_decode,
                              meta->pre_indices.data_ptr<int32_t>(),
                              meta->pre_qo_indptr.data_ptr<int32_t>(),
                              meta->pre_kv_indptr.data_ptr<int32_t>(),
                              meta->pre_q_start.data_ptr<int32_t>(), meta->num_prefill,
                              meta->max_qo_len, num_qo_heads_, num_kv_heads_, head_dim_, sm_scale,
                              o.data_ptr(), o.stride(0), o.stride(1), ws.data_ptr(), ws.numel(),
                              stream),
              "sgl_paged_mixed");
    return o.view({-1, num_qo_heads_ * head_dim_});
  }
  // Otherwise a mixed batch runs the prefill rows on a side stream next to
  // the decode rows (they write disjoint rows of o): the MFMA-bound prefill
  // and the HBM-bound decode then share the GPU. Fork and join are event
  // edges, so this also holds inside a captured graph. The persistent decode
  // launch goes first so its workgroups are resident before the prefill
  // tiles take the remaining slots (the other order measured no gain).
  const bool fork = overlap_mixed_ && meta->num_decode > 0 && meta->num_prefill > 0;
  void* pre_stream = stream;
  if (fork) {
    pre_stream = side_stream();
    check_hip(hipEventRecord(fork_event_, static_cast<hipStream_t>(stream)), "hipEventRecord");
    check_hip(hipStreamWaitEvent(static_cast<hipStream_t>(pre_stream), fork_event_, 0),
              "hipStreamWaitEvent");
  }
  if (meta->num_decode > 0) {
    // Graph-captured launches use the capture workspace, whose address never
    // changes; eager launches use the growable one, which is kept alive if a
    // graph records it anyway (capture of eagerly prepared metadata).
    torch::Tensor& ws = !meta->use_capture_buffers ? workspace(meta->dec_plan.workspace_bytes)
                        : meta->is_prefill         ? mixed_->workspace
                                                   : capture_->workspace;
    if (!meta->use_capture_buffers) {
      hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
      check_hip(hipStreamIsCapturing(static_cast<hipStream_t>(stream), &cs),
                "hipStreamIsCapturing");
      if (cs != hipStreamCaptureStatusNone) workspace_captured_ = true;
    }
    TORCH_CHECK(ws.numel() >= meta->dec_plan.workspace_bytes, "decode workspace too small");
    check_sgl(sgl_paged_decode(&meta->dec_plan, q.data_ptr(), q.stride(0), q.stride(1),
                               kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1),
                               meta->dec_indices.data_ptr<int32_t>(),
                               meta->dec_kv_indptr.data_ptr<int32_t>(),
                               meta->dec_q_rows.data_ptr<int32_t>(), meta->num_decode,
                               num_qo_heads_, num_kv_heads_, head_dim_, sm_scale, o.data_ptr(),
                               o.stride(0), o.stride(1), ws.data_ptr(), ws.numel(), stream),
              "sgl_paged_decode");
  }
  if (meta->num_prefill > 0) {
    check_sgl(sgl_paged_prefill(q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(),
                                vc.data_ptr(), kc.stride(0), kc.stride(1),
                                meta->pre_indices.data_ptr<int32_t>(),
                                meta->pre_qo_indptr.data_ptr<int32_t>(),
                                meta->pre_kv_indptr.data_ptr<int32_t>(),
                                meta->pre_q_start.data_ptr<int32_t>(), meta->num_prefill,
                                meta->max_qo_len, num_qo_heads_, num_kv_heads_, head_dim_,
                                sm_scale, o.data_ptr(), o.stride(0), o.stride(1), pre_stream),
              "sgl_paged_prefill");
  }
  if (fork) {
    check_hip(hipEventRecord(join_event_, static_cast<hipStream_t>(pre_stream)), "hipEventRecord");
    check_hip(hipStreamWaitEvent(static_cast<hipStream_t>(stream), join_event_, 0),
              "hipStreamWaitEvent");
  }
  return o.view({-1, num_qo_heads_ * head_dim_});
}

// ---------------------------------------------------------------- graphs
//
// Capture buffers have fixed addresses sized at init (the reference's
// DecodeCaptureData, flashinfer_backend.cu:193-219). A decode plan per batch
// size is built once for the worst case (every request at max_seq_len); the
// decode kernel sizes its work units on the device from kv_indptr, so replay
// only refreshes buffer contents — no host split planning, no pinned ring
// (replaces flashinfer_backend.cu:267-352).

void HipAttnBackend::init_capture_graph(int max_seq_len, const std::vector<int>& bs_list) {
  capture_.reset();
  // Graphs of the previous capture set are retired with it (the caller
  // destroys them before capturing again), and so are the grown-out
  // workspaces they may have recorded.
  retired_workspaces_.clear();
  if (bs_list.empty()) return;
  TORCH_CHECK(max_seq_len > 0, "max_seq_len must be positive");
  auto cap = std::make_unique<CaptureState>();
  cap->max_seq_len = max_seq_len;
  cap->max_bs = *std::max_element(bs_list.begin(), bs_list.end());
  TORCH_CHECK(*std::min_element(bs_list.begin(), bs_list.end()) > 0,
              "batch sizes must be positive");
  TORCH_CHECK(static_cast<int64_t>(cap->max_bs) * max_seq_len <= 0x7fffffff,
              "max batch size x max_seq_len must fit int32 token offsets");
  const auto dev = kI32.device(kv_cache_->device());
  cap->kv_indptr = torch::zeros({cap->max_bs + 1}, dev);
  cap->indices = torch::zeros({static_cast<int64_t>(cap->max_bs) * max_seq_len}, dev);
  cap->q_rows = torch::arange(cap->max_bs, dev);
  int64_t ws_bytes = 0;
  for (int bs : bs_list) {
    std::vector<int32_t> worst(bs + 1);
    for (int i = 0; i <= bs; ++i) worst[i] = i * max_seq_len;
    sgl_decode_plan_t plan;
    check_sgl(sgl_decode_plan(worst.data(), bs, num_qo_heads_, num_kv_heads_, head_dim_, &plan),
              "sgl_decode_plan");
    cap->plans[bs] = plan;
    ws_bytes = std::max<int64_t>(ws_bytes, plan.workspace_bytes);
  }
  cap->workspace = torch::empty({std::max<int64_t>(ws_bytes, 256)},
                                torch::TensorOptions().dtype(torch::kUInt8).device(
                                    kv_cache_->device()));
  capture_ = std::move(cap);
}

void HipAttnBackend::prepare_for_capture(Batch& batch) {
  if (batch.is_prefill()) {
    prepare_mixed_for_capture(batch);
    return;
  }
  TORCH_CHECK(capture_, "Decode capture state is not initialized");
  TORCH_CHECK(page_table_.defined(), "HipAttnBackend: set_page_table() first");
  const int bs = batch.padded_size();
  auto it = capture_->plans.find(bs);
  TORCH_CHECK(it != capture_->plans.end(), "No decode capture plan for batch size ", bs);
  auto meta = std::make_shared<HipAttnMetadata>();
  meta->use_capture_buffers = true;
  meta->num_decode = bs;
  meta->dec_plan = it->second;
  meta->dec_kv_indptr = capture_->kv_indptr.slice(0, 0, bs + 1);
  meta->dec_indices = capture_->indices.slice(0, 0, static_cast<int64_t>(bs) * capture_->max_seq_len);
  meta->dec_q_rows = capture_->q_rows.slice(0, 0, bs);
  meta->indptr = meta->dec_kv_indptr;
  // Worst-case contents: every request at max_seq_len over its own row.
  std::vector<int32_t> worst(bs + 1), table_idx(bs);
  for (int i = 0; i <= bs; ++i) worst[i] = i * capture_->max_seq_len;
  for (int i = 0; i < bs; ++i) table_idx[i] = batch.padded_reqs[i]->table_idx;
  meta->kv_indptr_host = worst;
  meta->dec_kv_indptr.copy_(to_device(worst, *meta));
  meta->dec_table_idx = to_device(table_idx, *meta);
  check_sgl(sgl_build_decode_indices(page_table_.data_ptr<int32_t>(), page_table_.size(0),
                                     page_table_.stride(0), page_table_.size(1),
                                     meta->dec_table_idx.data_ptr<int32_t>(),
                                     meta->dec_kv_indptr.data_ptr<int32_t>(),
                                     meta->dec_indices.data_ptr<int32_t>(), bs,
                                     current_stream(kv_cache_->device())),
            "sgl_build_decode_indices");
  capture_->metadata[bs] = meta;
  batch.attn_metadata = meta;
}

void HipAttnBackend::prepare_for_replay(Batch& batch) {
  if (batch.is_prefill()) {
    prepare_mixed_for_replay(batch);
    return;
  }
  TORCH_CHECK(capture_, "Decode capture state is not initialized");
  auto meta = metadata_of(batch);
  const int bs = batch.padded_size();
  auto it = capture_->metadata.find(bs);
  TORCH_CHECK(it != capture_->metadata.end(), "No decode capture metadata for batch size ", bs);
  auto& cap = it->second;
  TORCH_CHECK(static_cast<int>(meta->kv_indptr_host.size()) == bs + 1,
              "Invalid kv_indptr size for replay");
  for (int i = 0; i < bs; ++i) {
    TORCH_CHECK(meta->kv_indptr_host[i + 1] - meta->kv_indptr_host[i] <= capture_->max_seq_len,
                "request longer than the captured max_seq_len");
  }
  check_sgl(sgl_decode_plan_check(&cap->dec_plan, meta->kv_indptr_host.data(), bs),
            "sgl_decode_plan_check");
  // kv_indptr and indices into the capture buffers: one launch on the
  // engine stream, after the previous replay's reads of them.
  const sgl_i32_copy_t copies[2] = {
      {meta->dec_kv_indptr.data_ptr<int32_t>(), cap->dec_kv_indptr.data_ptr<int32_t>(), bs + 1},
      {meta->dec_indices.data_ptr<int32_t>(), cap->dec_indices.data_ptr<int32_t>(),
       meta->kv_indptr_host[bs]}};
  check_sgl(sgl_copy_i32(copies, 2, current_stream(kv_cache_->device())), "sgl_copy_i32");
  cap->kv_indptr_host = meta->kv_indptr_host;
  cap->host_staging = meta->host_staging;  // the source's pending H2D copy stays alive
  batch.attn_metadata = cap;
}


// Mixed steps. The reference captures decode batches only
// (flashinfer_backend.cu:193-219,267-352); the same contract -- fixed
// addresses sized at init, replay rewrites contents only -- is extended here
// to prefill-phase batches whose qo_len == 1 rows go to the split-KV decode
// kernel and whose chunks go to the prefill kernel. Capture metadata is keyed
// by (decode rows, prefill requests); the decode rows use a worst-case plan
// (every row at max_seq_len, units sized on the device at replay) and the
// prefill launch is sized for max_prefill_qo (tiles past a request's rows
// exit at once), so both launches stay valid for any replayed lengths.

void HipAttnBackend::init_mixed_capture_graph(int max_seq_len, int max_decode_rows,
                                              int max_prefill_reqs, int max_prefill_qo) {
  mixed_.reset();
  retired_workspaces_.clear();  // as in init_capture_graph
  TORCH_CHECK(max_seq_len > 0 && max_decode_rows >= 0 && max_prefill_reqs > 0 &&
                  max_prefill_qo > 1 && max_prefill_qo <= max_seq_len,
              "init_mixed_capture_graph: need max_seq_len > 0, max_decode_rows >= 0, "
              "max_prefill_reqs > 0 and 1 < max_prefill_qo <= max_seq_len");
  TORCH_CHECK(static_cast<int64_t>(max_decode_rows) * max_seq_len <= 0x7fffffff &&
                  static_cast<int64_t>(max_prefill_reqs) * max_seq_len <= 0x7fffffff,
              "init_mixed_capture_graph: rows x max_seq_len must fit int32 token offsets");
  auto m = std::make_unique<MixedCapture>();
  m->max_seq_len = max_seq_len;
  m->max_dec = max_decode_rows;
  m->max_pre = max_prefill_reqs;
  m->max_qo = max_prefill_qo;
  const auto dev = kI32.device(kv_cache_->device());
  const int64_t L = max_seq_len;
  m->qo_indptr = torch::zeros({max_decode_rows + max_prefill_reqs + 1}, dev);
  m->dec_kv_indptr = torch::zeros({max_decode_rows + 1}, dev);
  m->dec_indices = torch::zeros({std::max<int64_t>(max_decode_rows * L, 1)}, dev);
  m->dec_q_rows = torch::zeros({std::max(max_decode_rows, 1)}, dev);
  m->pre_qo_indptr = torch::zeros({max_prefill_reqs + 1}, dev);
  m->pre_kv_indptr = torch::zeros({max_prefill_reqs + 1}, dev);
  m->pre_q_start = torch::zeros({max_prefill_reqs}, dev);
  m->pre_indices = torch::zeros({max_prefill_reqs * L}, dev);
  // Workspace for the largest worst-case decode plan of any row count: the
  // plan of a two-launch step, or of a one-launch step, whose units are at
  // most max(decode CUs x 8 / hkv, tokens / the fused launch's unit cap) --
  // largest at the whole device's CUs.
  const bool fusable = num_kv_heads_ <= 8 && 8 % num_kv_heads_ == 0;
  int64_t ws_bytes = 256;
  std::vector<int32_t> worst(1, 0);
  for (int n = 1; n <= max_decode_rows; ++n) {
    worst.push_back(static_cast<int32_t>(n * L));
    sgl_decode_plan_t plan;
    check_sgl(sgl_decode_plan(worst.data(), n, num_qo_heads_, num_kv_heads_, head_dim_, &plan),
              "sgl_decode_plan");
    ws_bytes = std::max<int64_t>(ws_bytes, plan.workspace_bytes);
    if (fusable) {
      check_sgl(sgl_decode_plan_cus(worst.data(), n, num_qo_heads_, num_kv_heads_, head_dim_,
                                    device_cus_, &plan),
                "sgl_decode_plan_cus");
      ws_bytes = std::max<int64_t>(ws_bytes, plan.workspace_bytes);
    }
  }
  m->workspace = torch::empty({ws_bytes}, torch::TensorOptions().dtype(torch::kUInt8).device(
                                              kv_cache_->device()));
  mixed_ = std::move(m);
}

bool HipAttnBackend::pad_mixed_batch(Batch& batch, const std::shared_ptr<Req>& dummy) const {
  TORCH_CHECK(batch.is_prefill(), "pad_mixed_batch pads prefill-phase (mixed) batches");
  TORCH_CHECK(dummy && dummy->cached_len == 0 && dummy->device_len() == 1,
              "the dummy request has cached_len 0 and device_len 1");
  if (!mixed_) return false;
  // Query rows as prepare_metadata counts them: qo_len = max(1, extend),
  // or device_len when no request has a cache hit.
  const int bs = batch.padded_size();
  bool all_no_cache_hit = true;
  for (const auto& r : batch.padded_reqs) all_no_cache_hit = all_no_cache_hit && r->cached_len == 0;
  int n_dec = 0;
  for (const auto& r : batch.padded_reqs)
    n_dec += (all_no_cache_hit ? r->device_len() : std::max(1, r->extend_len())) == 1;
  const int n_pre = bs - n_dec;
  int best = -1;
  for (const auto& kv : mixed_->metadata)
    if (kv.first.second == n_pre && kv.first.first >= n_dec &&
        (best < 0 || kv.first.first < best))
      best = kv.first.first;
  if (best < 0) return false;
  batch.padded_reqs.insert(batch.padded_reqs.end(), static_cast<size_t>(best - n_dec), dummy);
  return true;
}

void HipAttnBackend::check_mixed_capacity(const HipAttnMetadata& m) const {
  TORCH_CHECK(m.num_decode <= mixed_->max_dec, "mixed step has ", m.num_decode,
              " decode rows; capture capacity is ", mixed_->max_dec);
  TORCH_CHECK(m.num_prefill <= mixed_->max_pre, "mixed step has ", m.num_prefill,
              " prefill requests; capture capacity is ", mixed_->max_pre);
  TORCH_CHECK(m.max_qo_len <= mixed_->max_qo, "prefill chunk of ", m.max_qo_len,
              " tokens exceeds the captured max_prefill_qo ", mixed_->max_qo);
  for (size_t i = 0; i + 1 < m.kv_indptr_host.size(); ++i)
    TORCH_CHECK(m.kv_indptr_host[i + 1] - m.kv_indptr_host[i] <= mixed_->max_seq_len,
                "request longer than the captured max_seq_len");
}

// A batch's metadata contents into capture buffers: every field in one
// device launch (sgl_copy_i32) on the current stream.
void HipAttnBackend::copy_contents(HipAttnMetadata& dst, const HipAttnMetadata& src) {
  const int bs = static_cast<int>(src.qo_indptr_host.size()) - 1;
  std::vector<sgl_i32_copy_t> c;
  auto add = [&](const torch::Tensor& from, torch::Tensor& to, int64_t n) {
    if (n > 0) c.push_back({from.data_ptr<int32_t>(), to.data_ptr<int32_t>(), n});
  };
  add(src.indptr, dst.indptr, bs + 1);
  if (src.num_decode > 0) {
    const int n = src.num_decode;
    add(src.dec_kv_indptr, dst.dec_kv_indptr, n + 1);
    add(src.dec_q_rows, dst.dec_q_rows, n);
    add(src.dec_indices, dst.dec_indices, src.dec_indices.numel());
  }
  if (src.num_prefill > 0) {
    const int n = src.num_prefill;
    add(src.pre_qo_indptr, dst.pre_qo_indptr, n + 1);
    add(src.pre_kv_indptr, dst.pre_kv_indptr, n + 1);
    add(src.pre_q_start, dst.pre_q_start, n);
    add(src.pre_indices, dst.pre_indices, src.pre_indices.numel());
  }
  check_sgl(sgl_copy_i32(c.data(), static_cast<int>(c.size()),
                         current_stream(src.indptr.device())),
            "sgl_copy_i32");
  dst.seq_lens = src.seq_lens;
  dst.cached_lens = src.cached_lens;
  dst.qo_indptr_host = src.qo_indptr_host;
  dst.kv_indptr_host = src.kv_indptr_host;
}

void HipAttnBackend::prepare_mixed_for_capture(Batch& batch) {
  TORCH_CHECK(mixed_, "prefill-phase capture needs init_mixed_capture_graph() first");
  prepare_metadata(batch);  // this batch's contents, then moved into the fixed buffers
  auto src = metadata_of(batch);
  check_mixed_capacity(*src);
  const int bs = batch.padded_size();
  const int n_dec = src->num_decode, n_pre = src->num_prefill;
  const int64_t L = mixed_->max_seq_len;
  auto meta = std::make_shared<HipAttnMetadata>();
  meta->is_prefill = true;
  meta->use_capture_buffers = true;
  meta->indptr = mixed_->qo_indptr.slice(0, 0, bs + 1);
  meta->num_decode = n_dec;
  // The one-launch split is fixed at capture, from the captured batch's sizes.
  meta->fused = src->fused;
  meta->dec_cus = src->dec_cus;
  if (n_dec > 0) {
    std::vector<int32_t> worst(n_dec + 1);
    for (int i = 0; i <= n_dec; ++i) worst[i] = static_cast<int32_t>(i * L);
    if (meta->fused)
      check_sgl(sgl_decode_plan_cus(worst.data(), n_dec, num_qo_heads_, num_kv_heads_, head_dim_,
                                    meta->dec_cus, &meta->dec_plan),
                "sgl_decode_plan_cus");
    else
      check_sgl(sgl_decode_plan(worst.data(), n_dec, num_qo_heads_, num_kv_heads_, head_dim_,
                                &meta->dec_plan),
                "sgl_decode_plan");
    TORCH_CHECK(meta->dec_plan.workspace_bytes <= mixed_->workspace.numel(),
                "mixed capture workspace too small");
    meta->dec_kv_indptr = mixed_->dec_kv_indptr.slice(0, 0, n_dec + 1);
    meta->dec_indices = mixed_->dec_indices.slice(0, 0, n_dec * L);
    meta->dec_q_rows = mixed_->dec_q_rows.slice(0, 0, n_dec);
  }
  meta->num_prefill = n_pre;
  meta->max_qo_len = mixed_->max_qo;
  if (n_pre > 0) {
    meta->pre_qo_indptr = mixed_->pre_qo_indptr.slice(0, 0, n_pre + 1);
    meta->pre_kv_indptr = mixed_->pre_kv_indptr.slice(0, 0, n_pre + 1);
    meta->pre_q_start = mixed_->pre_q_start.slice(0, 0, n_pre);
    meta->pre_indices = mixed_->pre_indices.slice(0, 0, n_pre * L);
  }
  copy_contents(*meta, *src);
  meta->capture_tokens = src->qo_indptr_host[bs];
  meta->host_staging = src->host_staging;  // pending H2D copies of the source stay alive
  mixed_->metadata[{n_dec, n_pre}] = meta;
  batch.attn_metadata = meta;
}

void HipAttnBackend::prepare_mixed_for_replay(Batch& batch) {
  TORCH_CHECK(mixed_, "prefill-phase replay needs init_mixed_capture_graph() first");
  auto src = metadata_of(batch);
  TORCH_CHECK(!src->use_capture_buffers, "prepare_for_replay expects prepare_metadata() first");
  auto it = mixed_->metadata.find({src->num_decode, src->num_prefill});
  TORCH_CHECK(it != mixed_->metadata.end(), "no captured mixed step with ", src->num_decode,
              " decode rows and ", src->num_prefill, " prefill requests");
  auto& cap = it->second;
  check_mixed_capacity(*src);
  const int bs = batch.padded_size();
  TORCH_CHECK(static_cast<int>(cap->indptr.numel()) == bs + 1,
              "replayed batch size differs from the captured one");
  TORCH_CHECK(src->qo_indptr_host[bs] <= cap->capture_tokens, "replayed step has ",
              src->qo_indptr_host[bs], " query rows; the graph was captured with ",
              cap->capture_tokens);
  if (src->num_decode > 0) {
    std::vector<int32_t> dec_ip(src->num_decode + 1, 0);
    int i = 0;
    for (int r = 0; r < bs; ++r)
      if (src->qo_indptr_host[r + 1] - src->qo_indptr_host[r] == 1) {
        dec_ip[i + 1] = dec_ip[i] + (src->kv_indptr_host[r + 1] - src->kv_indptr_host[r]);
        ++i;
      }
    check_sgl(sgl_decode_plan_check(&cap->dec_plan, dec_ip.data(), src->num_decode),
              "sgl_decode_plan_check");
  }
  copy_contents(*cap, *src);
  cap->host_staging = src->host_staging;
  batch.attn_metadata = cap;
}

// ---------------------------------------------------------------- page table

void write_page_table(const torch::Tensor& page_table, const std::vector<int32_t>& allocated_pages,
                      const std::vector<std::tuple<int, int, int>>& allocation_info,
                      int page_size) {
  if (allocated_pages.empty()) return;
  TORCH_CHECK(page_size > 0, "page_size must be positive");
  TORCH_CHECK(page_table.is_cuda() && page_table.dim() == 2 &&
                  page_table.scalar_type() == torch::kInt32 && page_table.stride(1) == 1,
              "page table must be a 2-D int32 device tensor with unit column stride");
  const int64_t npages = static_cast<int64_t>(allocated_pages.size());
  const int64_t nalloc = static_cast<int64_t>(allocation_info.size());
  int64_t taken = 0;
  for (const auto& [table_idx, first_page, last_page] : allocation_info) {
    (void)table_idx;
    if (last_page > first_page) taken += last_page - first_page;
  }
  TORCH_CHECK(taken == npages, "Allocated page count mismatch");
  auto staging = torch::empty({npages + 3 * nalloc}, kI32.pinned_memory(true));
  int32_t* h = staging.data_ptr<int32_t>();
  std::memcpy(h, allocated_pages.data(), sizeof(int32_t) * npages);
  int32_t* ai = h + npages;
  for (const auto& [table_idx, first_page, last_page] : allocation_info) {
    *ai++ = table_idx;
    *ai++ = first_page;
    *ai++ = last_page;
  }
  auto dev = staging.to(page_table.device(), /*non_blocking=*/true);
  check_sgl(sgl_write_page_table(page_table.data_ptr<int32_t>(), page_table.size(0),
                                 page_table.stride(0), page_table.size(1),
                                 dev.data_ptr<int32_t>(), npages, dev.data_ptr<int32_t>() + npages,
                                 static_cast<int>(nalloc), page_size,
                                 current_stream(page_table.device())),
            "sgl_write_page_table");
}

// ---------------------------------------------------------------- layers

namespace {
// SGL_DTYPE_* of a 16-bit floating tensor; the reference's kernels take
// fp16 and bf16 (normalization.cu:253-268,346-372, activation.cu:25-44,
// rotary_embedding.cu:124-168).
int half_dtype(const torch::Tensor& t, const char* what) {
  if (t.scalar_type() == torch::kBFloat16) return SGL_DTYPE_BF16;
  TORCH_CHECK(t.scalar_type() == torch::kFloat16, what, " must be bf16 or fp16");
  return SGL_DTYPE_F16;
}

void check_same_dtype(const torch::Tensor& a, const torch::Tensor& b, const char* what) {
  TORCH_CHECK(a.scalar_type() == b.scalar_type(), what, " must share one dtype");
}
}  // namespace

RMSNorm::RMSNorm(int size, float eps, torch::Device device) : eps_(eps) {
  weight = torch::ones({size}, torch::TensorOptions().dtype(torch::kBFloat16).device(device));
}

void RMSNorm::forward_inplace_3d_strided(torch::Tensor& x) const {
  TORCH_CHECK(x.is_cuda() && x.dim() == 3 && x.stride(2) == 1,
              "Strided RMSNorm expects a rank-3 device tensor with a contiguous last dim");
  const int dt = half_dtype(x, "x");
  check_same_dtype(x, weight, "x and the RMSNorm weight");
  TORCH_CHECK(weight.size(0) == x.size(2), "RMSNorm weight size must match last dimension");
  check_sgl(sgl_qk_rmsnorm(x.data_ptr(), nullptr, weight.data_ptr(), nullptr, x.size(0), x.size(1),
                           0, x.size(2), x.stride(0), x.stride(1), 0, 0, eps_, dt,
                           current_stream(x.device())),
            "sgl_qk_rmsnorm");
}

namespace {
// [rows, d] view of a tensor whose rows are contiguous: rank 2 with any row
// stride, or a contiguous tensor of higher rank.
void rows_view(const torch::Tensor& t, int64_t& rows, int64_t& d, int64_t& stride,
               const char* what) {
  TORCH_CHECK(t.is_cuda() && t.dim() >= 2 && t.stride(-1) == 1, what,
              " must be a device tensor of rank >= 2 with a contiguous last dim");
  d = t.size(-1);
  rows = d > 0 ? t.numel() / d : 0;
  if (t.dim() == 2) {
    stride = t.stride(0);
  } else {
    TORCH_CHECK(t.is_contiguous(), what, " of rank > 2 must be contiguous");
    stride = d;
  }
}
}  // namespace

torch::Tensor RMSNorm::forward(const torch::Tensor& x) const {
  auto out = torch::empty_like(x, x.options().memory_format(torch::MemoryFormat::Contiguous));
  int64_t rows, d, xs, os, r2, d2;
  rows_view(x, rows, d, xs, "x");
  rows_view(out, r2, d2, os, "out");
  TORCH_CHECK(weight.size(0) == d, "RMSNorm weight size must match last dimension");
  const int dt = half_dtype(x, "x");
  TORCH_CHECK(weight.scalar_type() == x.scalar_type(), "RMSNorm weight dtype must match x");
  check_sgl(sgl_rmsnorm(out.data_ptr(), x.data_ptr(), weight.data_ptr(), rows, d, xs, os, dt, eps_,
                        current_stream(x.device())),
            "sgl_rmsnorm");
  return out;
}

void RMSNorm::forward_inplace(torch::Tensor& x) const {
  int64_t rows, d, xs;
  rows_view(x, rows, d, xs, "x");
  TORCH_CHECK(weight.size(0) == d, "RMSNorm weight size must match last dimension");
  const int dt = half_dtype(x, "x");
  TORCH_CHECK(weight.scalar_type() == x.scalar_type(), "RMSNorm weight dtype must match x");
  check_sgl(sgl_rmsnorm(x.data_ptr(), x.data_ptr(), weight.data_ptr(), rows, d, xs, xs, dt, eps_,
                        current_stream(x.device())),
            "sgl_rmsnorm");
}

void RMSNorm::fused_add_forward_inplace(torch::Tensor& x, torch::Tensor& residual) const {
  TORCH_CHECK(x.is_cuda() && residual.is_cuda(), "x and residual must be device tensors");
  TORCH_CHECK(x.dim() == 2 && residual.dim() == 2, "FusedAddRMSNorm expects rank-2 tensors");
  TORCH_CHECK(x.sizes() == residual.sizes(), "x and residual shapes must match");
  TORCH_CHECK(x.size(-1) > 0, "RMSNorm last dimension must be positive");
  TORCH_CHECK(weight.size(0) == x.size(1), "RMSNorm weight size must match last dimension");
  TORCH_CHECK(x.stride(1) == 1 && residual.stride(1) == 1, "rows must be contiguous");
  const int dt = half_dtype(x, "x");
  TORCH_CHECK(residual.scalar_type() == x.scalar_type() && weight.scalar_type() == x.scalar_type(),
              "x, residual and weight must share a dtype");
  check_sgl(sgl_fused_add_rmsnorm(x.data_ptr(), residual.data_ptr(), weight.data_ptr(), x.size(0),
                                  x.size(1), x.stride(0), residual.stride(0), dt, eps_,
                                  current_stream(x.device())),
            "sgl_fused_add_rmsnorm");
}

static void act_and_mul(bool gelu, torch::Tensor& out, const torch::Tensor& input) {
  TORCH_CHECK(input.is_cuda() && out.is_cuda(), "Inputs must be device tensors");
  TORCH_CHECK(input.dim() == 2 && out.dim() == 2 && input.stride(1) == 1 && out.stride(1) == 1,
              "input / out must be rank-2 with contiguous rows");
  const int64_t d = input.size(1) / 2;
  TORCH_CHECK(input.size(1) == 2 * d && out.size(0) == input.size(0) && out.size(1) == d,
              "input must be [T, 2d] and out [T, d]");
  const int dt = half_dtype(input, "input");
  TORCH_CHECK(out.scalar_type() == input.scalar_type(), "out dtype must match input");
  auto fn = gelu ? sgl_gelu_and_mul : sgl_silu_and_mul;
  check_sgl(fn(out.data_ptr(), input.data_ptr(), input.size(0), d, input.stride(0), out.stride(0),
               dt, current_stream(input.device())),
            gelu ? "sgl_gelu_and_mul" : "sgl_silu_and_mul");
}

void silu_and_mul(torch::Tensor& out, const torch::Tensor& input) { act_and_mul(false, out, input); }
void gelu_and_mul(torch::Tensor& out, const torch::Tensor& input) { act_and_mul(true, out, input); }

// ---------------------------------------------------------------- sampling

namespace {
void check_probs(const torch::Tensor& probs) {
  TORCH_CHECK(probs.defined(), "probs must be defined");
  TORCH_CHECK(probs.is_cuda(), "sampling requires device probs");
  TORCH_CHECK(probs.is_contiguous(), "sampling requires contiguous probs");
  TORCH_CHECK(probs.scalar_type() == torch::kFloat32, "sampling expects float32 probs");
  TORCH_CHECK(probs.dim() == 2, "probs must have shape [batch, vocab]");
}

void check_uniform(const torch::Tensor& probs, const torch::Tensor& u, int64_t dims) {
  TORCH_CHECK(u.defined() && u.is_cuda() && u.is_contiguous() && u.scalar_type() == torch::kFloat32,
              "uniform_samples must be a contiguous device float32 tensor");
  TORCH_CHECK(u.device() == probs.device(), "uniform_samples must be on the same device as probs");
  TORCH_CHECK(u.dim() == dims, "uniform_samples has unexpected dimensions");
  TORCH_CHECK(u.size(dims - 1) == probs.size(0), dims == 1
                  ? "uniform_samples must have shape [batch]"
                  : "uniform_samples must have shape [max_rounds, batch]");
}

void check_row_arg(const torch::Tensor& t, const torch::Tensor& probs, c10::ScalarType st,
                   const char* what) {
  TORCH_CHECK(!t.defined() || (t.is_cuda() && t.is_contiguous() && t.scalar_type() == st &&
                               t.device() == probs.device() && t.numel() == probs.size(0)),
              what, " must be a contiguous device tensor of the documented dtype with shape [batch]");
}

FlashInferSamplingResult sampling_outputs(const torch::Tensor& probs) {
  auto opts = probs.options();
  return {torch::empty({probs.size(0)}, opts.dtype(torch::kInt32)),
          torch::empty({probs.size(0)}, opts.dtype(torch::kBool))};
}

int32_t narrow_dim(int64_t v, const char* what) {
  TORCH_CHECK(v >= 0 && v <= 0x7fffffff, what, " out of range");
  return static_cast<int32_t>(v);
}
}  // namespace

torch::Tensor sampling_probs(const torch::Tensor& logits, const torch::Tensor& temperatures) {
  TORCH_CHECK(logits.is_cuda() && logits.dim() == 2 && logits.stride(1) == 1,
              "logits must be a [batch, vocab] device tensor with contiguous rows");
  int dtype = SGL_DTYPE_F32;
  if (logits.scalar_type() == torch::kBFloat16) dtype = SGL_DTYPE_BF16;
  else if (logits.scalar_type() == torch::kFloat16) dtype = SGL_DTYPE_F16;
  else TORCH_CHECK(logits.scalar_type() == torch::kFloat32, "logits must be bf16, fp16 or float32");
  const int64_t batch = logits.size(0);
  TORCH_CHECK(temperatures.numel() == batch, "one temperature per row");
  auto temps = temperatures.to(logits.device()).to(torch::kFloat32).reshape({batch}).contiguous();
  auto probs = torch::empty({batch, logits.size(1)}, logits.options().dtype(torch::kFloat32));
  check_sgl(sgl_softmax_temperature(probs.data_ptr<float>(), probs.stride(0), logits.data_ptr(),
                                    logits.stride(0), dtype, temps.data_ptr<float>(), 1.0f, batch,
                                    logits.size(1), current_stream(logits.device())),
            "sgl_softmax_temperature");
  return probs;
}

FlashInferSamplingResult sample_from_logits(const torch::Tensor& logits,
                                            const torch::Tensor& temperatures,
                                            const torch::Tensor& uniform_samples,
                                            const torch::Tensor& top_k, const torch::Tensor& top_p) {
  TORCH_CHECK(logits.is_cuda() && logits.dim() == 2 && logits.stride(1) == 1,
              "logits must be a [batch, vocab] device tensor with contiguous rows");
  int dtype = SGL_DTYPE_F32;
  if (logits.scalar_type() == torch::kBFloat16) dtype = SGL_DTYPE_BF16;
  else if (logits.scalar_type() == torch::kFloat16) dtype = SGL_DTYPE_F16;
  else TORCH_CHECK(logits.scalar_type() == torch::kFloat32, "logits must be bf16, fp16 or float32");
  const int64_t batch = logits.size(0);
  TORCH_CHECK(temperatures.numel() == batch, "one temperature per row");
  auto temps = temperatures.to(logits.device()).to(torch::kFloat32).reshape({batch}).contiguous();
  const bool has_k = top_k.defined(), has_p = top_p.defined();
  const int mode = has_k && has_p ? 3 : has_k ? 1 : has_p ? 2 : 0;
  TORCH_CHECK(uniform_samples.is_cuda() && uniform_samples.scalar_type() == torch::kFloat32 &&
                  uniform_samples.is_contiguous() && uniform_samples.dim() == (mode == 0 ? 1 : 2) &&
                  uniform_samples.size(-1) == batch,
              "uniform_samples must be contiguous float32 [batch] (plain draw) or [rounds, batch]");
  torch::Tensor k_f, k_i, p_f;
  if (mode == 1) k_f = top_k.to(logits.device()).to(torch::kFloat32).reshape({batch}).contiguous();
  if (mode == 3) k_i = top_k.to(logits.device()).to(torch::kInt32).reshape({batch}).contiguous();
  if (mode >= 2) p_f = top_p.to(logits.device()).to(torch::kFloat32).reshape({batch}).contiguous();
  FlashInferSamplingResult r;
  r.samples = torch::empty({batch}, logits.options().dtype(torch::kInt32));
  if (mode != 0) r.success = torch::empty({batch}, logits.options().dtype(torch::kBool));
  check_sgl(sgl_sampling_from_logits(
                logits.data_ptr(), logits.stride(0), dtype, temps.data_ptr<float>(), 1.0f,
                uniform_samples.data_ptr<float>(), mode,
                k_f.defined() ? k_f.data_ptr<float>() : nullptr,
                k_i.defined() ? k_i.data_ptr<int32_t>() : nullptr, 0,
                p_f.defined() ? p_f.data_ptr<float>() : nullptr, 0.0f, r.samples.data_ptr<int32_t>(),
                mode != 0 ? reinterpret_cast<uint8_t*>(r.success.data_ptr<bool>()) : nullptr,
                narrow_dim(batch, "batch"), narrow_dim(logits.size(1), "vocab"),
                mode == 0 ? 1 : narrow_dim(uniform_samples.size(0), "rounds"),
                current_stream(logits.device())),
            "sgl_sampling_from_logits");
  return r;
}

torch::Tensor flashinfer_sample_from_probs(const torch::Tensor& probs,
                                           const torch::Tensor& uniform_samples, bool deterministic) {
  check_probs(probs);
  check_uniform(probs, uniform_samples, 1);
  auto samples = torch::empty({probs.size(0)}, probs.options().dtype(torch::kInt32));
  check_sgl(sgl_sampling_from_probs(probs.data_ptr<float>(), uniform_samples.data_ptr<float>(),
                                    samples.data_ptr<int32_t>(), narrow_dim(probs.size(0), "batch"),
                                    narrow_dim(probs.size(1), "vocab"), deterministic ? 1 : 0,
                                    current_stream(probs.device())),
            "sgl_sampling_from_probs");
  return samples;
}

FlashInferSamplingResult flashinfer_top_k_sample_from_probs(const torch::Tensor& probs,
                                                            const torch::Tensor& uniform_samples,
                                                            const torch::Tensor& top_k,
                                                            int64_t top_k_value, bool deterministic) {
  check_probs(probs);
  check_uniform(probs, uniform_samples, 2);
  check_row_arg(top_k, probs, torch::kFloat32, "top_k");
  auto r = sampling_outputs(probs);
  check_sgl(sgl_top_k_sampling_from_probs(
                probs.data_ptr<float>(), uniform_samples.data_ptr<float>(), r.samples.data_ptr<int32_t>(),
                reinterpret_cast<uint8_t*>(r.success.data_ptr<bool>()),
                top_k.defined() ? top_k.data_ptr<float>() : nullptr,
                narrow_dim(probs.size(0), "batch"), static_cast<int>(top_k_value),
                narrow_dim(probs.size(1), "vocab"), narrow_dim(uniform_samples.size(0), "rounds"),
                deterministic ? 1 : 0, current_stream(probs.device())),
            "sgl_top_k_sampling_from_probs");
  return r;
}

FlashInferSamplingResult flashinfer_top_p_sample_from_probs(const torch::Tensor& probs,
                                                            const torch::Tensor& uniform_samples,
                                                            const torch::Tensor& top_p,
                                                            double top_p_value, bool deterministic) {
  check_probs(probs);
  check_uniform(probs, uniform_samples, 2);
  check_row_arg(top_p, probs, torch::kFloat32, "top_p");
  auto r = sampling_outputs(probs);
  check_sgl(sgl_top_p_sampling_from_probs(
                probs.data_ptr<float>(), uniform_samples.data_ptr<float>(), r.samples.data_ptr<int32_t>(),
                reinterpret_cast<uint8_t*>(r.success.data_ptr<bool>()),
                top_p.defined() ? top_p.data_ptr<float>() : nullptr,
                narrow_dim(probs.size(0), "batch"), static_cast<float>(top_p_value),
                narrow_dim(probs.size(1), "vocab"), narrow_dim(uniform_samples.size(0), "rounds"),
                deterministic ? 1 : 0, current_stream(probs.device())),
            "sgl_top_p_sampling_from_probs");
  return r;
}

FlashInferSamplingResult flashinfer_top_k_top_p_sample_from_probs(
    const torch::Tensor& probs, const torch::Tensor& uniform_samples, const torch::Tensor& top_k,
    double top_k_value, const torch::Tensor& top_p, double top_p_value, bool deterministic) {
  check_probs(probs);
  check_uniform(probs, uniform_samples, 2);
  check_row_arg(top_k, probs, torch::kInt32, "top_k");
  check_row_arg(top_p, probs, torch::kFloat32, "top_p");
  auto r = sampling_outputs(probs);
  check_sgl(sgl_top_k_top_p_sampling_from_probs(
                probs.data_ptr<float>(), uniform_samples.data_ptr<float>(),
                top_k.defined() ? top_k.data_ptr<int32_t>() : nullptr,
                top_p.defined() ? top_p.data_ptr<float>() : nullptr, r.samples.data_ptr<int32_t>(),
                reinterpret_cast<uint8_t*>(r.success.data_ptr<bool>()),
                narrow_dim(probs.size(0), "batch"), static_cast<int>(top_k_value),
                static_cast<float>(top_p_value), narrow_dim(probs.size(1), "vocab"),
                narrow_dim(uniform_samples.size(0), "rounds"), deterministic ? 1 : 0,
                current_stream(probs.device())),
            "sgl_top_k_top_p_sampling_from_probs");
  return r;
}

void fused_qk_rmsnorm_inplace_3d_strided(torch::Tensor& q, torch::Tensor& k, const RMSNorm& q_norm,
                                         const RMSNorm& k_norm) {
  TORCH_CHECK(q.is_cuda() && k.is_cuda(), "q and k must be device tensors");
  TORCH_CHECK(q.dim() == 3 && k.dim() == 3, "Fused QK RMSNorm expects rank-3 tensors");
  TORCH_CHECK(q.stride(2) == 1 && k.stride(2) == 1, "Last dimension must be contiguous");
  TORCH_CHECK(q.size(0) == k.size(0) && q.size(2) == k.size(2), "q / k shapes must agree");
  TORCH_CHECK(q_norm.eps() == k_norm.eps(), "Q and K RMSNorm eps must match");
  const int dt = half_dtype(q, "q");
  check_same_dtype(q, k, "q and k");
  check_same_dtype(q, q_norm.weight, "q and the q-norm weight");
  check_same_dtype(q, k_norm.weight, "q and the k-norm weight");
  check_sgl(sgl_qk_rmsnorm(q.data_ptr(), k.data_ptr(), q_norm.weight.data_ptr(),
                           k_norm.weight.data_ptr(), q.size(0), q.size(1), k.size(1), q.size(2),
                           q.stride(0), q.stride(1), k.stride(0), k.stride(1), q_norm.eps(), dt,
                           current_stream(q.device())),
            "sgl_qk_rmsnorm");
}

RotaryEmbedding::RotaryEmbedding(int head_size, int rotary_dim, int max_position_embeddings,
                                 float base, torch::Device device)
    : head_size_(head_size), rotary_dim_(rotary_dim) {
  TORCH_CHECK(rotary_dim > 0 && rotary_dim % 2 == 0 && rotary_dim <= head_size,
              "rotary_dim must be even and <= head_size");
  auto opts = torch::TensorOptions().dtype(torch::kFloat32).device(device);
  cos_cache_ = torch::empty({max_position_embeddings, rotary_dim / 2}, opts);
  sin_cache_ = torch::empty_like(cos_cache_);
  check_sgl(sgl_rope_cos_sin_cache(cos_cache_.data_ptr<float>(), sin_cache_.data_ptr<float>(),
                                   max_position_embeddings, rotary_dim, base,
                                   current_stream(device)),
            "sgl_rope_cos_sin_cache");
}

void RotaryEmbedding::forward_inplace(const torch::Tensor& positions, torch::Tensor& query,
                                      torch::Tensor& key) const {
  TORCH_CHECK(query.is_cuda() && key.is_cuda() && positions.is_cuda(),
              "Inputs must be device tensors");
  TORCH_CHECK(positions.scalar_type() == torch::kInt32, "positions must be int32");
  const int dt = half_dtype(query, "query");
  check_same_dtype(query, key, "query and key");
  check_sgl(sgl_rope(query.data_ptr(), key.data_ptr(), cos_cache_.data_ptr<float>(),
                     sin_cache_.data_ptr<float>(), positions.data_ptr<int32_t>(),
                     positions.size(0), query.size(1), key.size(1), rotary_dim_, query.size(2),
                     cos_cache_.size(1), query.stride(0), query.stride(1), key.stride(0),
                     key.stride(1), dt, current_stream(query.device())),
            "sgl_rope");
}

AttentionLayer::AttentionLayer(int layer_id, int num_qo_heads, int num_kv_heads, int head_dim,
                               std::shared_ptr<HipAttnBackend> backend,
                               std::shared_ptr<RotaryEmbedding> rotary,
                               std::shared_ptr<RMSNorm> q_norm, std::shared_ptr<RMSNorm> k_norm)
    : layer_id_(layer_id),
      num_qo_heads_(num_qo_heads),
      num_kv_heads_(num_kv_heads),
      head_dim_(head_dim),
      backend_(std::move(backend)),
      rotary_(std::move(rotary)),
      q_norm_(std::move(q_norm)),
      k_norm_(std::move(k_norm)) {
  TORCH_CHECK(backend_ && rotary_, "AttentionLayer needs a backend and a rotary embedding");
  TORCH_CHECK(static_cast<bool>(q_norm_) == static_cast<bool>(k_norm_),
              "the fused pass needs both q and k norms or neither");
  TORCH_CHECK(rotary_->rotary_dim() == head_dim, "the fused pass uses full-width rotary");
}

torch::Tensor AttentionLayer::forward(const torch::Tensor& qkv, const torch::Tensor& positions,
                                      Batch& batch) {
  // Missing context fails before anything is written (the reference's
  // layer throws on a missing context, tests/layers/test_attention_layer.cpp:7-22).
  TORCH_CHECK(batch.attn_metadata,
              "AttentionLayer: the batch has no attention metadata (call prepare_metadata first)");
  TORCH_CHECK(qkv.dim() == 2 && qkv.stride(1) == 1, "qkv must be [T, (Hq + 2 Hkv) D]");
  check_bf16(qkv, "qkv");
  TORCH_CHECK(qkv.size(1) == (num_qo_heads_ + 2 * num_kv_heads_) * head_dim_,
              "qkv width does not match the head counts");
  TORCH_CHECK(positions.scalar_type() == torch::kInt32 && batch.out_loc.scalar_type() == torch::kInt32,
              "positions and out_loc must be int32 for the fused pass");
  TORCH_CHECK(batch.out_loc.size(0) == qkv.size(0) && positions.size(0) == qkv.size(0),
              "positions and out_loc need one entry per token");
  auto kc = backend_->kv_cache()->k_cache(layer_id_);
  auto vc = backend_->kv_cache()->v_cache(layer_id_);
  check_sgl(sgl_fused_qknorm_rope_store(
                qkv.data_ptr(), qkv.stride(0), kc.data_ptr(), vc.data_ptr(),
                q_norm_ ? q_norm_->weight.data_ptr() : nullptr,
                k_norm_ ? k_norm_->weight.data_ptr() : nullptr, rotary_->cos_cache().data_ptr<float>(),
                rotary_->sin_cache().data_ptr<float>(), positions.data_ptr<int32_t>(),
                batch.out_loc.data_ptr<int32_t>(), qkv.size(0), num_qo_heads_, num_kv_heads_,
                head_dim_, q_norm_ ? q_norm_->eps() : 0.f,
                // k is read from the pool from here on; qkv's k part is dead
                SGL_FUSED_NO_K_WRITEBACK, current_stream(qkv.device())),
            "sgl_fused_qknorm_rope_store");
  auto q = qkv.narrow(1, 0, num_qo_heads_ * head_dim_).view({-1, num_qo_heads_, head_dim_});
  return backend_->attend(q, layer_id_, batch);
}

}  // namespace sglang
