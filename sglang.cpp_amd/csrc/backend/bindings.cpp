// Python bindings of the C++ attention backend (module sgl_backend). The
// classes keep the reference's names so a test reads like the reference's
// own use of them (src/engine/engine.cc, src/layers/attention_layer.cc).
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>
#include <torch/extension.h>

#include "hip_backend.h"

namespace py = pybind11;
using namespace sglang;

namespace {

torch::Device cuda(int index) { return torch::Device(torch::kCUDA, static_cast<c10::DeviceIndex>(index)); }

torch::Dtype parse_dtype(const std::string& name) {
  if (name == "bfloat16" || name == "bf16") return torch::kBFloat16;
  if (name == "float16" || name == "fp16") return torch::kFloat16;
  throw std::invalid_argument("unsupported KV dtype: " + name);
}

std::shared_ptr<HipAttnMetadata> hip_meta(const Batch& b) {
  auto m = std::dynamic_pointer_cast<HipAttnMetadata>(b.attn_metadata);
  if (!m) throw std::runtime_error("batch has no HipAttnMetadata");
  return m;
}

py::dict plan_dict(const sgl_decode_plan_t& p) {
  py::dict d;
  d["kv_chunk_size"] = p.kv_chunk_size;
  d["min_chunk_size"] = p.min_chunk_size;
  d["max_total_tokens"] = p.max_total_tokens;
  d["split_kv"] = p.split_kv;
  d["num_units"] = p.num_units;
  d["batch_size"] = p.batch_size;
  d["workspace_bytes"] = p.workspace_bytes;
  return d;
}

}  // namespace

PYBIND11_MODULE(sgl_backend, m) {
  m.doc() = "gfx950 attention backend (BaseAttnBackend contract over libsgl_attn)";

  py::class_<Req, std::shared_ptr<Req>>(m, "Req")
      .def(py::init([](int table_idx, int cached_len, int device_len) {
             auto r = std::make_shared<Req>();
             r->table_idx = table_idx;
             r->cached_len = cached_len;
             r->device_len_ = device_len;
             return r;
           }),
           py::arg("table_idx"), py::arg("cached_len"), py::arg("device_len"))
      .def_readwrite("table_idx", &Req::table_idx)
      .def_readwrite("cached_len", &Req::cached_len)
      .def_readwrite("device_len_", &Req::device_len_)
      .def("device_len", &Req::device_len)
      .def("extend_len", &Req::extend_len);

  py::class_<Batch, std::shared_ptr<Batch>>(m, "Batch")
      .def(py::init([](bool is_prefill, std::vector<std::shared_ptr<Req>> reqs,
                       torch::Tensor positions, torch::Tensor out_loc) {
             auto b = std::make_shared<Batch>();
             b->phase = is_prefill ? BatchPhase::Prefill : BatchPhase::Decode;
             b->padded_reqs = std::move(reqs);
             b->positions = std::move(positions);
             b->out_loc = std::move(out_loc);
             return b;
           }),
           py::arg("is_prefill"), py::arg("reqs"), py::arg("positions"), py::arg("out_loc"))
      .def_readwrite("padded_reqs", &Batch::padded_reqs)
      .def_readwrite("positions", &Batch::positions)
      .def_readwrite("out_loc", &Batch::out_loc)
      .def("is_prefill", &Batch::is_prefill)
      .def("is_decode", &Batch::is_decode)
      .def("padded_size", &Batch::padded_size)
      .def("has_metadata", [](const Batch& b) { return static_cast<bool>(b.attn_metadata); })
      .def("get_last_indices",
           [](const Batch& b, int bs) { return hip_meta(b)->get_last_indices(bs); })
      .def("num_decode_rows", [](const Batch& b) { return hip_meta(b)->num_decode; })
      .def("num_prefill_rows", [](const Batch& b) { return hip_meta(b)->num_prefill; })
      .def("fused_mixed_cus",  // CUs of the decode rows in a one-launch mixed step, else 0
           [](const Batch& b) { return hip_meta(b)->fused ? hip_meta(b)->dec_cus : 0; })
      .def("decode_plan", [](const Batch& b) { return plan_dict(hip_meta(b)->dec_plan); })
      .def("uses_capture_buffers",
           [](const Batch& b) { return hip_meta(b)->use_capture_buffers; })
      .def("qo_indptr_host", [](const Batch& b) { return hip_meta(b)->qo_indptr_host; })
      .def("kv_indptr_host", [](const Batch& b) { return hip_meta(b)->kv_indptr_host; })
      .def("record_metadata_stream",  // HipAttnMetadata::record_stream (scheduler.cc:152-179)
           [](const Batch& b, int64_t stream_id, int device_index) {
             // torch.cuda.Stream's (stream_id, device_index) name a HIP stream
             hip_meta(b)->record_stream(c10::hip::HIPStream(c10::Stream::unpack3(
                 stream_id, static_cast<c10::DeviceIndex>(device_index), c10::DeviceType::HIP)));
           },
           py::arg("stream_id"), py::arg("device_index"));

  py::class_<BaseKVCachePool, std::shared_ptr<BaseKVCachePool>>(m, "BaseKVCachePool");
  py::class_<MHAKVCache, BaseKVCachePool, std::shared_ptr<MHAKVCache>>(m, "MHAKVCache")
      .def(py::init([](int hkv, int layers, int head_dim, int pages, int page_size, int device,
                       const std::string& dtype) {
             return std::make_shared<MHAKVCache>(hkv, layers, head_dim, pages, page_size,
                                                 parse_dtype(dtype), cuda(device));
           }),
           py::arg("num_kv_heads"), py::arg("num_layers"), py::arg("head_dim"),
           py::arg("num_pages"), py::arg("page_size"), py::arg("device") = 0,
           py::arg("dtype") = "bfloat16")
      .def("k_cache", &MHAKVCache::k_cache)
      .def("v_cache", &MHAKVCache::v_cache)
      .def("store_kv", &MHAKVCache::store_kv, py::arg("key"), py::arg("val"), py::arg("out_loc"),
           py::arg("layer_id"))
      .def("buffer", &MHAKVCache::buffer);

  py::class_<HipAttnBackend, std::shared_ptr<HipAttnBackend>>(m, "HipAttnBackend")
      .def(py::init<std::shared_ptr<BaseKVCachePool>, int, int, int>(), py::arg("kv_cache"),
           py::arg("num_qo_heads"), py::arg("num_kv_heads"), py::arg("head_dim"))
      .def("set_page_table", &HipAttnBackend::set_page_table)
      .def("set_fused_mixed", &HipAttnBackend::set_fused_mixed)
      .def("fused_mixed", &HipAttnBackend::fused_mixed)
      .def("set_overlap_mixed", &HipAttnBackend::set_overlap_mixed)
      .def("overlap_mixed", &HipAttnBackend::overlap_mixed)
      .def("prepare_metadata", &HipAttnBackend::prepare_metadata)
      .def("forward", &HipAttnBackend::forward, py::arg("q"), py::arg("k"), py::arg("v"),
           py::arg("layer_id"), py::arg("batch"))
      .def("attend", &HipAttnBackend::attend, py::arg("q"), py::arg("layer_id"), py::arg("batch"))
      .def("init_capture_graph", &HipAttnBackend::init_capture_graph, py::arg("max_seq_len"),
           py::arg("bs_list"))
      .def("init_mixed_capture_graph", &HipAttnBackend::init_mixed_capture_graph,
           py::arg("max_seq_len"), py::arg("max_decode_rows"), py::arg("max_prefill_reqs"),
           py::arg("max_prefill_qo"))
      .def("prepare_for_capture", &HipAttnBackend::prepare_for_capture)
      .def("prepare_for_replay", &HipAttnBackend::prepare_for_replay)
      .def("pad_mixed_batch", &HipAttnBackend::pad_mixed_batch, py::arg("batch"),
           py::arg("dummy"));

  m.def("write_page_table", &write_page_table, py::arg("page_table"),
        py::arg("allocated_pages"), py::arg("allocation_info"), py::arg("page_size"),
        "CacheManager::write_page_table (prefill.cc:144-187) on the device");

  py::class_<RMSNorm, std::shared_ptr<RMSNorm>>(m, "RMSNorm")
      .def(py::init([](int size, float eps, int device) {
             return std::make_shared<RMSNorm>(size, eps, cuda(device));
           }),
           py::arg("size"), py::arg("eps"), py::arg("device") = 0)
      .def_readwrite("weight", &RMSNorm::weight)
      .def("eps", &RMSNorm::eps)
      .def("forward", &RMSNorm::forward)
      .def("forward_inplace", [](const RMSNorm& n, torch::Tensor x) { n.forward_inplace(x); })
      .def("forward_inplace_3d_strided", [](const RMSNorm& n, torch::Tensor x) {
        n.forward_inplace_3d_strided(x);
      })
      .def("fused_add_forward_inplace", [](const RMSNorm& n, torch::Tensor x, torch::Tensor r) {
        n.fused_add_forward_inplace(x, r);
      });

  m.def("sampling_probs", &sampling_probs, py::arg("logits"), py::arg("temperatures"));
  m.def("sample_from_logits",
        [](torch::Tensor logits, torch::Tensor temps, torch::Tensor u,
           c10::optional<torch::Tensor> k, c10::optional<torch::Tensor> p) {
          auto r = sample_from_logits(logits, temps, u, k.value_or(torch::Tensor()),
                                      p.value_or(torch::Tensor()));
          return py::make_tuple(r.samples, r.success);
        },
        py::arg("logits"), py::arg("temperatures"), py::arg("uniform_samples"),
        py::arg("top_k") = py::none(), py::arg("top_p") = py::none());
  m.def("flashinfer_sample_from_probs", &flashinfer_sample_from_probs, py::arg("probs"),
        py::arg("uniform_samples"), py::arg("deterministic") = false);
  auto pair = [](const FlashInferSamplingResult& r) { return py::make_tuple(r.samples, r.success); };
  m.def("flashinfer_top_k_sample_from_probs",
        [pair](torch::Tensor p, torch::Tensor u, c10::optional<torch::Tensor> k, int64_t kv, bool det) {
          return pair(flashinfer_top_k_sample_from_probs(p, u, k.value_or(torch::Tensor()), kv, det));
        },
        py::arg("probs"), py::arg("uniform_samples"), py::arg("top_k"), py::arg("top_k_value") = 0,
        py::arg("deterministic") = false);
  m.def("flashinfer_top_p_sample_from_probs",
        [pair](torch::Tensor p, torch::Tensor u, c10::optional<torch::Tensor> t, double tv, bool det) {
          return pair(flashinfer_top_p_sample_from_probs(p, u, t.value_or(torch::Tensor()), tv, det));
        },
        py::arg("probs"), py::arg("uniform_samples"), py::arg("top_p"), py::arg("top_p_value") = 0.0,
        py::arg("deterministic") = false);
  m.def("flashinfer_top_k_top_p_sample_from_probs",
        [pair](torch::Tensor p, torch::Tensor u, c10::optional<torch::Tensor> k, double kv,
               c10::optional<torch::Tensor> t, double tv, bool det) {
          return pair(flashinfer_top_k_top_p_sample_from_probs(p, u, k.value_or(torch::Tensor()), kv,
                                                               t.value_or(torch::Tensor()), tv, det));
        },
        py::arg("probs"), py::arg("uniform_samples"), py::arg("top_k"), py::arg("top_k_value"),
        py::arg("top_p"), py::arg("top_p_value"), py::arg("deterministic") = false);
  m.def("silu_and_mul", [](torch::Tensor out, torch::Tensor input) { silu_and_mul(out, input); });
  m.def("gelu_and_mul", [](torch::Tensor out, torch::Tensor input) { gelu_and_mul(out, input); });

  m.def("fused_qk_rmsnorm_inplace_3d_strided",
        [](torch::Tensor q, torch::Tensor k, const RMSNorm& qn, const RMSNorm& kn) {
          fused_qk_rmsnorm_inplace_3d_strided(q, k, qn, kn);
        });

  py::class_<RotaryEmbedding, std::shared_ptr<RotaryEmbedding>>(m, "RotaryEmbedding")
      .def(py::init([](int head_size, int rotary_dim, int max_pos, float base, int device) {
             return std::make_shared<RotaryEmbedding>(head_size, rotary_dim, max_pos, base,
                                                      cuda(device));
           }),
           py::arg("head_size"), py::arg("rotary_dim"), py::arg("max_position_embeddings"),
           py::arg("base"), py::arg("device") = 0)
      .def("forward_inplace",
           [](const RotaryEmbedding& r, const torch::Tensor& pos, torch::Tensor q,
              torch::Tensor k) { r.forward_inplace(pos, q, k); })
      .def("cos_cache", &RotaryEmbedding::cos_cache)
      .def("sin_cache", &RotaryEmbedding::sin_cache);

  py::class_<AttentionLayer, std::shared_ptr<AttentionLayer>>(m, "AttentionLayer")
      .def(py::init<int, int, int, int, std::shared_ptr<HipAttnBackend>,
                    std::shared_ptr<RotaryEmbedding>, std::shared_ptr<RMSNorm>,
                    std::shared_ptr<RMSNorm>>(),
           py::arg("layer_id"), py::arg("num_qo_heads"), py::arg("num_kv_heads"),
           py::arg("head_dim"), py::arg("backend"), py::arg("rotary"),
           py::arg("q_norm") = nullptr, py::arg("k_norm") = nullptr)
      .def("forward", &AttentionLayer::forward, py::arg("qkv"), py::arg("positions"),
           py::arg("batch"));
}
