"""The measurement contract of bench.py, checked on the CPU.

The algorithmic work behind every roofline figure is pinned to figures
derived by hand for the benchmark configurations (bytes and flops per
launch, the derivation in each test's comments), so a wrong term in a
formula shows up here rather than as a plausible-looking fraction. The per-kernel
HBM traffic keys bench.py reads must exist in profiles/traffic.json, each
with its rocprof summary, and a multi-GPU request must be refused.
"""
import json
import subprocess
import sys
from pathlib import Path

import numpy as np

import __graft_entry__ as entry

REPO = Path(__file__).resolve().parents[1]
wl = entry.load_package().workloads


def test_cfg1_decode_bytes():
    w = wl.cfg1_decode_small()
    b = w.batch
    # K+V 8,388,608 + Q/O 32,768 + one index per page (P = 1) 8,192
    assert wl.attention_bytes(w.shape, b.qo_lens, b.kv_lens, b.page_size) == 8_429_568


def test_cfg2_prefill_work():
    w = wl.cfg2_prefill_prefix()
    b = w.batch
    # 41,024 visible pairs per head and request: sum over i < 128 of 256 + i + 1
    assert wl.causal_pairs(128, 384) == 41_024
    assert wl.attention_flops(w.shape, b.qo_lens, b.kv_lens, True) == 2_688_548_864
    # K+V 12,582,912 + Q/O 8,388,608 + 24 pages x 8 requests x 4 B
    assert wl.attention_bytes(w.shape, b.qo_lens, b.kv_lens, b.page_size) == 20_972_288


def test_cfg3_fused_store_bytes():
    w = wl.cfg3_fused_store()
    assert wl.fused_store_bytes(w.shape, 8192) == 138_477_568


def test_cfg5_prefill_chunk_flops():
    w = wl.cfg5_prefill_chunk()
    b = w.batch
    assert list(b.qo_lens) == [2048] and list(b.kv_lens) == [6144]
    # 4 D Hq pairs: pairs = sum over i < 2048 of 4096 + i + 1 = 10,486,784
    assert wl.causal_pairs(2048, 6144) == 10_486_784
    assert wl.attention_flops(w.shape, b.qo_lens, b.kv_lens, True) == 4 * 128 * 32 * 10_486_784


def test_causal_pairs_brute_force():
    rng = np.random.default_rng(3)
    for _ in range(20):
        qo = int(rng.integers(1, 50))
        kv = qo + int(rng.integers(0, 50))
        off = kv - qo
        want = sum(1 for i in range(qo) for j in range(kv) if j <= i + off)
        assert wl.causal_pairs(qo, kv) == want


def test_traffic_keys_have_profiles():
    traffic = json.loads((REPO / "profiles" / "traffic.json").read_text())
    src = (REPO / "bench.py").read_text()
    keys = ["paged_decode_cfg1", "paged_decode_cfg4", "paged_prefill_cfg2",
            "paged_prefill_cfg5_chunk", "fused_qknorm_rope_store_cfg3",
            "fused_add_rmsnorm_qwen3_8b", "silu_and_mul_qwen3_8b", "sampling_top_k_top_p",
            "softmax_temperature_sampler", "sampler_step_top_k_top_p"]
    for k in keys:
        assert k in traffic and traffic[k] > 0, k
        assert (REPO / "profiles" / f"{k}.md").exists(), k
    # every key bench.py names literally is one of them
    for k in ("paged_prefill_cfg2", "paged_prefill_cfg5_chunk", "fused_qknorm_rope_store_cfg3",
              "sampling_top_k_top_p", "softmax_temperature_sampler", "sampler_step_top_k_top_p"):
        assert f'"{k}"' in src, k


def test_sampler_softmax_bytes():
    # one read of bf16 logits, one write of fp32 probabilities, the temperatures
    bench = _bench_module()
    assert 256 * 151936 * (2 + 4) + 4 * 256 == 233374720
    assert bench.SAMPLING_BATCH == 256 and bench.QWEN3_VOCAB == 151936


def test_multi_gpu_request_is_refused():
    res = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode != 0
    assert "one GPU" in res.stderr


def _bench_module():
    import importlib.util
    spec = importlib.util.spec_from_file_location("_bench", REPO / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_probe_library_exports_its_entry_points():
    """The ceiling probes the bench reports are built beside the attention
    library and export what bench.py binds (no GPU call)."""
    import ctypes
    path = REPO / "sglang.cpp_amd" / "libsgl_probes.so"
    if not path.exists():
        import pytest
        pytest.skip("libsgl_probes.so not built")
    lib = ctypes.CDLL(str(path))
    for name in ("sgl_probe_stream_read", "sgl_probe_page_read", "sgl_probe_decode_read",
                 "sgl_probe_mfma_bf16", "sgl_probe_empty", "sgl_probe_stream_copy"):
        assert hasattr(lib, name), name
    bench = _bench_module()
    assert bench.load_probes() is not None


def test_ceiling_fractions_use_the_bound_of_each_kernel():
    bench = _bench_module()
    ceil = {"stream_read": {"GB/s": 7000.0}, "mfma_random": {"TFLOP/s": 1800.0}}
    extra = {"cfg4": {"roofline": {"bound": "hbm", "achieved": 6300.0}},
             "prefill_chunk": {"roofline": {"bound": "mfma", "achieved": 900.0}},
             "cfg5": {"graph_ms": 21.0}}
    fr = bench.ceiling_fracs(extra, ceil)
    assert fr == {"cfg4": 0.9, "prefill_chunk": 0.5}
    # a kernel that writes as much as it reads: against the copy ceiling
    ceil["stream_copy"] = {"GB/s": 5000.0}
    extra["cfg3"] = {"roofline": {"bound": "hbm", "achieved": 4500.0}}
    fr = bench.ceiling_fracs(extra, ceil)
    assert fr == {"cfg4": 0.9, "prefill_chunk": 0.5, "cfg3": 0.9}
    # one MFMA of the probe: 32 x 32 x 16 multiply-adds
    assert bench.MFMA_FLOPS == 32768
