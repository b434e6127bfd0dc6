"""Benchmark of the MI355X attention hot path (one GPU).

Default workload (the headline line): benchmark configuration 4 — ragged paged
decode at the Qwen3-8B attention shape (32 q / 8 kv heads, head_dim 128,
bf16), batch 256, kv lengths ~ U[128, 4096], page_size 16, seeded random
page table, split-KV. One step = one sgl_paged_decode call (the decode
kernel plus its split merge) over the whole batch, inputs resident in HBM.

The other configs are reported under "extra" (and as their own lines with
--workload): cfg1 small decode, cfg2 prefill with prefix hits, cfg3 fused
RoPE + qk-norm + KV store, cfg5 mixed 48-layer step replayed as a hipGraph,
prefill_chunk (cfg5's 2048-token prefill chunk on its 4096-token prefix, one
layer, alone: the prefill kernel's MFMA fraction); and the residual path around attention at the Qwen3-8B shape for an
8192-token chunk: resid_norm (fused add + RMSNorm, hidden 4096) and
resid_act (SiLU-and-mul, intermediate 12288); sampling (top-k + top-p
draw for 256 rows over the Qwen3 vocabulary, as the Sampler runs it); and
sampler_softmax (the Sampler's probabilities from bf16 logits and per-row
temperatures for those rows, beside LibTorch's own path on the device);
and sampler_step (that softmax and the top-k + top-p draw in one launch,
beside our two launches and LibTorch's probabilities followed by our draw).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload cfgN]
                       [--no-extra] [--no-cpu] [--min-warm-seconds S]

Each workload is warmed for W steps and then until at least S seconds
(default 0.5) have passed, because the GPU clock ramps under sustained
load; the timed region is exactly K steps.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

METRIC = "paged decode attn GB/s & prefill TFLOP/s (% MI355X peak), 1 GPU"
HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, AMD published
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense bf16 MFMA, AMD published
PROFILE_TRAFFIC = REPO / "profiles" / "traffic.json"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--min-warm-seconds", type=float, default=0.5,
                    help="keep warming each workload until this much time has passed "
                         "(after the W warm-up steps; the timed region is still K steps)")
    ap.add_argument("--workload", default="cfg4",
                    choices=["cfg1", "cfg2", "cfg3", "cfg4", "cfg5", "prefill_chunk", "resid_norm",
                             "resid_act", "sampling", "sampler_softmax", "sampler_step"])
    ap.add_argument("--no-extra", action="store_true", help="headline workload only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--cfg5-layers", type=int, default=48)
    ap.add_argument("--ceilings-only", action="store_true",
                    help="only measure the practical ceilings of this GPU (stream read, MFMA "
                         "issue on random and constant bf16 operands, empty launch) and print them")
    ap.add_argument("--no-resident-leg", action="store_true",
                    help="time rotated (HBM-resident) buffer sets only, without the one-set "
                         "cache-resident leg (profiler runs)")
    ap.add_argument("--replay-host-only", action="store_true",
                    help="only measure the host cost of prepare_metadata + prepare_for_replay "
                         "per serving step (configurations 4 and 5)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB (steps times): "
                         "the known-size reference for rocprofv3 FETCH_SIZE / WRITE_SIZE")
    return ap.parse_args()


# ------------------------------------------------------------------ helpers

class Timer:
    """Times K launches of fn: wall clock around the loop (synchronized on
    both sides) and one pair of HIP events recorded on the stream the kernels
    run on, bracketing the same K steps (per-step event pairs would add a
    queue barrier between steps)."""

    def __init__(self, torch, min_warm_s=0.0):
        self.torch = torch
        self.min_warm_s = min_warm_s

    def run(self, fn, steps, warmup):
        """W warm-up steps, continued (in batches of 8) until at least
        min_warm_s seconds have passed: the GPU clock ramps under sustained
        load, and a few warm-up steps leave a short kernel timed below its
        steady-state clock. Then exactly K timed steps."""
        torch = self.torch
        stream = torch.cuda.current_stream()
        w0 = time.perf_counter()
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        while time.perf_counter() - w0 < self.min_warm_s:
            for _ in range(8):
                fn()
            torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        start.record(stream)
        for _ in range(steps):
            fn()
        end.record(stream)
        torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - t0) * 1e3 / steps
        ev_ms = start.elapsed_time(end) / steps
        return wall_ms, ev_ms


    def run_graph(self, fn, steps, warmup):
        """The same K steps captured as one hipGraph of K back-to-back calls
        and replayed once (after warm-up replays), so that for calls shorter
        than the host's per-call launch cost (a Python ctypes call and a
        kernel launch) the events time the kernels and not the gaps between
        them. Returns (wall ms, event ms) per step."""
        torch = self.torch
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(steps):
                fn()
        w0 = time.perf_counter()
        graph.replay()
        torch.cuda.synchronize()
        while time.perf_counter() - w0 < self.min_warm_s:
            graph.replay()
            torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        start.record(stream)
        graph.replay()
        end.record(stream)
        torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - t0) * 1e3 / steps
        ev_ms = start.elapsed_time(end) / steps
        del graph
        return wall_ms, ev_ms


def load_traffic(key):
    try:
        return json.loads(PROFILE_TRAFFIC.read_text()).get(key)
    except (OSError, ValueError):
        return None


# ------------------------------------------------------------------ workloads

# The MI355X's last-level (Infinity) cache holds 256 MB: a workload whose
# buffers fit in it and are re-run back to back is partly served from that
# cache, not HBM. HBM-bound workloads below this size are therefore timed
# over several independent buffer sets used in turn, enough that the bytes
# touched between two uses of one set exceed ROTATE_BYTES; the figure on one
# set (cache-resident) is reported beside it.
ROTATE_BYTES = 512 << 20


def rotation_sets(set_bytes):
    """Buffer sets so that the other sets touch >= ROTATE_BYTES between two
    uses of one set."""
    return max(1, -(-ROTATE_BYTES // max(1, int(set_bytes))) + 1)


def rotating(steps):
    """One step function that runs the given steps in turn (under graph
    capture each captured call keeps the set it was captured on)."""
    if len(steps) == 1:
        return steps[0]
    state = {"i": 0}

    def step():
        i = state["i"]
        state["i"] = (i + 1) % len(steps)
        steps[i]()

    return step



def setup_decode(torch, capi, wl, w, dev, seed=0):
    b, s = w.batch, w.shape
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    hq, hkv, D = s.num_qo_heads, s.num_kv_heads, s.head_dim
    kc = torch.randn((b.num_slots, hkv, D), device=dev, generator=g).to(torch.bfloat16)
    vc = torch.randn((b.num_slots, hkv, D), device=dev, generator=g).to(torch.bfloat16)
    qkv = torch.randn((b.batch_size, s.qkv_width), device=dev, generator=g).to(torch.bfloat16)
    q = qkv[:, :hq * D].view(-1, hq, D)
    o = torch.empty((b.batch_size, hq, D), device=dev, dtype=torch.bfloat16)
    plan = capi.decode_plan(b.kv_indptr, hq, hkv, D)
    ws = capi.decode_workspace(plan, dev)
    idx = torch.from_numpy(b.indices).to(dev)
    kvp = torch.from_numpy(b.kv_indptr).to(dev)
    scale = 1.0 / math.sqrt(D)

    def step():
        capi.paged_decode(plan, q, kc, vc, idx, kvp, o, ws, scale)

    nbytes = wl.attention_bytes(s, b.qo_lens, b.kv_lens, b.page_size)
    flops = wl.attention_flops(s, b.qo_lens, b.kv_lens, causal=False)
    return step, nbytes, flops, dict(q=q, kc=kc, vc=vc, plan=plan)


def setup_prefill(torch, capi, wl, w, dev, seed=0, sets=1):
    b, s = w.batch, w.shape
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    hq, hkv, D = s.num_qo_heads, s.num_kv_heads, s.head_dim
    rows = int(b.qo_indptr[-1])
    idx = torch.from_numpy(b.indices).to(dev)
    qop = torch.from_numpy(b.qo_indptr).to(dev)
    kvp = torch.from_numpy(b.kv_indptr).to(dev)
    scale = 1.0 / math.sqrt(D)
    max_qo = int(b.qo_lens.max())

    def one_set():
        kc = torch.randn((b.num_slots, hkv, D), device=dev, generator=g).to(torch.bfloat16)
        vc = torch.randn((b.num_slots, hkv, D), device=dev, generator=g).to(torch.bfloat16)
        qkv = torch.randn((rows, s.qkv_width), device=dev, generator=g).to(torch.bfloat16)
        q = qkv[:, :hq * D].view(-1, hq, D)
        o = torch.empty((rows, hq, D), device=dev, dtype=torch.bfloat16)

        def step():
            capi.paged_prefill(q, kc, vc, idx, qop, kvp, max_qo, o, scale)
        return step

    nbytes = wl.attention_bytes(s, b.qo_lens, b.kv_lens, b.page_size)
    flops = wl.attention_flops(s, b.qo_lens, b.kv_lens, causal=True)
    return rotating([one_set() for _ in range(sets)]), nbytes, flops


def setup_fused(torch, capi, wl, w, dev, seed=0, sets=1):
    b, s = w.batch, w.shape
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    hq, hkv, D = s.num_qo_heads, s.num_kv_heads, s.head_dim
    T = int(b.qo_indptr[-1])
    qw = (torch.rand(D, device=dev, generator=g) + 0.5).to(torch.bfloat16)
    kw = (torch.rand(D, device=dev, generator=g) + 0.5).to(torch.bfloat16)
    cos, sin = capi.rope_cos_sin_cache(w.extra["max_pos"], D, w.extra["theta"], dev)
    pos = torch.from_numpy(b.positions).to(dev)
    loc = torch.from_numpy(b.out_loc).to(dev)
    eps = w.extra["eps"]
    # The pass is in place; repeated steps re-normalise already-normalised
    # rows, which costs the same bytes and keeps values finite.

    def one_set():
        qkv = torch.randn((T, s.qkv_width), device=dev, generator=g).to(torch.bfloat16)
        kc = torch.empty((T, hkv, D), device=dev, dtype=torch.bfloat16)
        vc = torch.empty_like(kc)

        def step():
            # The pass as the attention layer runs it: k goes to the pool only
            # (the algorithmic byte count has no k write-back into qkv).
            capi.fused_qknorm_rope_store(qkv, kc, vc, qw, kw, cos, sin, pos, loc, hq, hkv, D,
                                         eps, write_k_back=False)
        return step

    return rotating([one_set() for _ in range(sets)]), wl.fused_store_bytes(s, T)


def setup_mixed(torch, wl, w, dev, layers, seed=0):
    """Config 5 through the C++ backend (HipAttnBackend over an MHAKVCache
    [2, L, slots, Hkv, D]): one prefill-phase batch of 64 qo=1 requests and a
    2048-token chunk; per layer, forward = KV store of the new tokens, the
    split-KV decode kernel on the qo=1 rows and the causal prefill kernel on
    the chunk. The 48-layer step is captured once on the backend's
    fixed-address mixed-step buffers (init_mixed_capture_graph /
    prepare_for_capture) and replayed as a hipGraph. Warm-up alternates
    prepare_metadata + prepare_for_replay between a second batch of new
    lengths and the benchmark batch, so the timed replays run on metadata a
    serving loop would have rewritten; the timed step is the replay."""
    import __graft_entry__ as entry
    sb = entry.load_package().backend.load()
    b, s = w.batch, w.shape
    hq, hkv, D = s.num_qo_heads, s.num_kv_heads, s.head_dim
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    cache = sb.MHAKVCache(hkv, layers, D, b.num_pages + 1, b.page_size, dev.index or 0)
    pool = cache.buffer()
    for l in range(layers):
        pool[0, l].normal_(generator=g)
        pool[1, l].normal_(generator=g)
    backend = sb.HipAttnBackend(cache, hq, hkv, D)
    # A/B switches: the one-launch mixed step (default) and, without it, the
    # side-stream overlap of separate launches (default).
    backend.set_fused_mixed(os.environ.get("SGL_FUSED_MIXED", "1") != "0")
    backend.set_overlap_mixed(os.environ.get("SGL_OVERLAP_MIXED", "1") != "0")
    page_table = torch.from_numpy(b.page_table).to(dev)
    backend.set_page_table(page_table)
    qo, kvl = b.qo_lens, b.kv_lens
    dec = np.nonzero(qo == 1)[0]
    pre = np.nonzero(qo > 1)[0]
    max_seq = int(b.page_table.shape[1])
    backend.init_mixed_capture_graph(max_seq, len(dec), len(pre), int(qo[pre].max()))

    def make_batch(cached, device):
        reqs = [sb.Req(int(b.table_idx[i]), int(cached[i]), int(device[i]))
                for i in range(b.batch_size)]
        return sb.Batch(True, reqs, torch.from_numpy(b.positions).to(dev),
                        torch.from_numpy(b.out_loc).to(dev))

    batch = make_batch(b.cached_lens, b.device_lens)
    # A second step of the same shape with other lengths: every request one
    # token shorter (its page-table row still holds it).
    alt = make_batch(b.cached_lens - 1, b.device_lens - 1)
    rows = int(b.qo_indptr[-1])
    qkv = torch.randn((rows, s.qkv_width), device=dev, generator=g).to(torch.bfloat16)
    q = qkv[:, :hq * D]
    k = qkv[:, hq * D:(hq + hkv) * D]
    v = qkv[:, (hq + hkv) * D:]
    backend.prepare_for_capture(batch)
    assert batch.uses_capture_buffers()

    def layer_pass():
        for l in range(layers):
            backend.forward(q, k, v, l, batch)

    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        layer_pass()  # warm the capture stream
    torch.cuda.current_stream().wait_stream(cap)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        layer_pass()
    torch.cuda.synchronize()
    for nb in (alt, batch):  # serving-loop metadata updates, ending on the benchmark batch
        backend.prepare_metadata(nb)
        backend.prepare_for_replay(nb)
        graph.replay()
    torch.cuda.synchronize()

    assert batch.num_decode_rows() == len(dec) and batch.num_prefill_rows() == len(pre)
    dec_bytes = wl.attention_bytes(s, qo[dec], kvl[dec], b.page_size) * layers
    pre_flops = wl.attention_flops(s, qo[pre], kvl[pre], causal=True) * layers
    pre_bytes = wl.attention_bytes(s, qo[pre], kvl[pre], b.page_size) * layers
    return graph.replay, dec_bytes, pre_flops, pre_bytes, (graph, cache, backend, batch, alt, qkv)


def measure_replay_host(torch, wl, dev, iters=200):
    """Host cost of one serving step's metadata on the graph-replay path:
    prepare_metadata (the scheduler's per-step call, scheduler.cc:338) plus
    prepare_for_replay (GraphRunner::replay, engine.cc:732-743), CPU wall
    clock per step, at configuration 4's decode batch (256 requests, one
    captured batch size) and configuration 5's mixed step (64 decode rows +
    a 2048-token chunk). Each step's calls are timed alone (the device
    synchronised before them); reported as the median and 90th percentile
    over `iters` steps, plus each call's median."""
    import __graft_entry__ as entry
    sb = entry.load_package().backend.load()
    out = {}
    for name, w in (("cfg4", wl.cfg4_decode_large()), ("cfg5", wl.cfg5_mixed(layers=1))):
        b, sh = w.batch, w.shape
        cache = sb.MHAKVCache(sh.num_kv_heads, 1, sh.head_dim, b.num_pages + 1, b.page_size,
                              dev.index or 0)
        backend = sb.HipAttnBackend(cache, sh.num_qo_heads, sh.num_kv_heads, sh.head_dim)
        backend.set_page_table(torch.from_numpy(b.page_table).to(dev))
        max_seq = int(b.page_table.shape[1])
        decode = name == "cfg4"
        if decode:
            backend.init_capture_graph(max_seq, [b.batch_size])
        else:
            qo = b.qo_lens
            backend.init_mixed_capture_graph(max_seq, int((qo == 1).sum()), int((qo > 1).sum()),
                                             int(qo[qo > 1].max()))
        pos = torch.from_numpy(b.positions).to(dev)
        loc = torch.from_numpy(b.out_loc).to(dev)

        def batch_of(shift):
            reqs = [sb.Req(int(b.table_idx[i]), int(b.cached_lens[i]) - shift,
                           int(b.device_lens[i]) - shift) for i in range(b.batch_size)]
            return sb.Batch(not decode, reqs, pos, loc)

        cap = batch_of(0)
        backend.prepare_for_capture(cap)
        t_meta, t_rep, t_all = [], [], []
        for i in range(iters + 20):
            nb = batch_of(i % 2)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            backend.prepare_metadata(nb)
            t1 = time.perf_counter()
            backend.prepare_for_replay(nb)
            t2 = time.perf_counter()
            if i >= 20:
                t_meta.append(t1 - t0)
                t_rep.append(t2 - t1)
                t_all.append(t2 - t0)
        torch.cuda.synchronize()
        us = lambda v, q=50: round(float(np.percentile(np.asarray(v) * 1e6, q)), 1)
        out[name] = {"step_us_median": us(t_all), "step_us_p90": us(t_all, 90),
                     "prepare_metadata_us": us(t_meta), "prepare_for_replay_us": us(t_rep),
                     "requests": int(b.batch_size), "iters": iters}
        del backend, cache
    return out


# ------------------------------------------------------------------ CPU baseline

def _cpu_threads(torch):
    """LibTorch threads for the CPU legs: the host's CPU share (OMP_NUM_THREADS
    when set, else the process's CPU affinity)."""
    n = int(os.environ.get("OMP_NUM_THREADS") or len(os.sched_getaffinity(0)))
    torch.set_num_threads(max(1, n))
    return torch.get_num_threads()


def _cpu_pool(torch, slots, hkv, D, seed):
    g = torch.Generator()
    g.manual_seed(seed)
    kc = torch.randn((slots, hkv, D), generator=g).to(torch.bfloat16)
    vc = torch.randn((slots, hkv, D), generator=g).to(torch.bfloat16)
    return kc, vc, g


def cpu_baseline_decode(torch, wl, w, target_s=1.0):
    """LibTorch-CPU fp32 decode (oracle/torch_cpu.py) on the first n requests
    of the same workload, n grown until one run takes about target_s;
    median of 5 runs after a warm-up."""
    from oracle import torch_cpu as tc
    b, s = w.batch, w.shape
    threads = _cpu_threads(torch)
    hkv, hq, D = s.num_kv_heads, s.num_qo_heads, s.head_dim
    scale = 1.0 / math.sqrt(D)
    lens_all = b.kv_lens.astype(np.int64)
    n = min(32, b.batch_size)
    while True:
        lens = lens_all[:n]
        ip = torch.from_numpy(np.concatenate([[0], np.cumsum(lens)]))
        slots = int(ip[-1])
        kc, vc, g = _cpu_pool(torch, slots, hkv, D, 3)
        idx = torch.randperm(slots, generator=g)
        q = torch.randn((n, hq, D), generator=g).to(torch.bfloat16)
        t0 = time.perf_counter()
        tc.decode(q, kc, vc, idx, ip, scale)
        el = time.perf_counter() - t0
        if el >= target_s / 2 or n == b.batch_size:
            break
        n = min(b.batch_size, max(n + 1, int(n * target_s / max(el, 1e-3))))
    med, runs = tc.median_time(lambda: tc.decode(q, kc, vc, idx, ip, scale))
    nbytes = wl.attention_bytes(s, np.ones(n, np.int64), lens, b.page_size)
    info = tc.host_info()
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port", "cpu_model": info["cpu_model"], "median_s": round(med, 4),
            "runs_s": [round(t, 4) for t in runs],
            "sample": f"LibTorch-CPU fp32 decode (oracle/torch_cpu.py) on the first {n} of "
                      f"{b.batch_size} requests of {w.name} (sum kv {slots} tokens), median "
                      f"of 5 runs after 1 warm-up, {threads} threads"}


def cpu_baseline_prefill(torch, wl, w):
    """LibTorch-CPU fp32 causal prefill on the whole workload, median of 5."""
    from oracle import torch_cpu as tc
    b, s = w.batch, w.shape
    threads = _cpu_threads(torch)
    hkv, hq, D = s.num_kv_heads, s.num_qo_heads, s.head_dim
    kc, vc, g = _cpu_pool(torch, b.num_slots, hkv, D, 4)
    q = torch.randn((int(b.qo_indptr[-1]), hq, D), generator=g).to(torch.bfloat16)
    idx = torch.from_numpy(b.indices.astype(np.int64))
    qip, kip = b.qo_indptr.astype(np.int64), b.kv_indptr.astype(np.int64)
    scale = 1.0 / math.sqrt(D)
    med, runs = tc.median_time(lambda: tc.prefill(q, kc, vc, idx, qip, kip, scale))
    flops = wl.attention_flops(s, b.qo_lens, b.kv_lens, causal=True)
    return {"value": round(flops / med / 1e12, 5), "unit": "TFLOP/s", "cores": threads,
            "kind": "port", "cpu_model": tc.host_info()["cpu_model"], "median_s": round(med, 4),
            "runs_s": [round(t, 4) for t in runs],
            "sample": f"LibTorch-CPU fp32 causal prefill (oracle/torch_cpu.py), all of {w.name}, "
                      f"median of 5 runs after 1 warm-up, {threads} threads"}


def cpu_baseline_fused(torch, wl, w):
    """LibTorch-CPU fused qk-norm + RoPE + KV store (oracle/torch_cpu.py) on the
    whole config 3 workload, median of 5 runs after a warm-up."""
    from oracle import torch_cpu as tc
    b, s = w.batch, w.shape
    threads = _cpu_threads(torch)
    hq, hkv, D = s.num_qo_heads, s.num_kv_heads, s.head_dim
    T = int(b.qo_indptr[-1])
    g = torch.Generator()
    g.manual_seed(6)
    qkv = torch.randn((T, s.qkv_width), generator=g).to(torch.bfloat16)
    kc = torch.zeros((T, hkv, D), dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    qw = (torch.rand(D, generator=g) + 0.5).to(torch.bfloat16)
    kw = (torch.rand(D, generator=g) + 0.5).to(torch.bfloat16)
    # the reference's table (rotary_embedding.cu:80-93), built once, not timed
    inv_freq = 1.0 / (w.extra["theta"] ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    freqs = torch.outer(torch.arange(w.extra["max_pos"], dtype=torch.float32), inv_freq)
    cos, sin = freqs.cos(), freqs.sin()
    pos = torch.from_numpy(b.positions.astype(np.int64))
    loc = torch.from_numpy(b.out_loc.astype(np.int64))
    eps = w.extra["eps"]

    def once():
        tc.fused_qknorm_rope_store(qkv, kc, vc, qw, kw, cos, sin, pos, loc, hq, hkv, eps)

    # One pass takes tens of milliseconds, where scheduler noise is large:
    # each timed run repeats the pass until it lasts about half a second.
    once()
    t0 = time.perf_counter()
    once()
    reps = max(1, int(0.5 / max(time.perf_counter() - t0, 1e-3)))

    def timed():
        for _ in range(reps):
            once()

    med, runs = tc.median_time(timed, runs=7)
    med, runs = med / reps, [t / reps for t in runs]
    nbytes = wl.fused_store_bytes(s, T)
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port", "cpu_model": tc.host_info()["cpu_model"], "median_s": round(med, 4),
            "runs_s": [round(t, 4) for t in runs],
            "sample": f"LibTorch-CPU fused qk-norm + RoPE + KV store (oracle/torch_cpu.py), all "
                      f"{T} tokens of {w.name}, {reps} passes per timed run, median of 7 runs "
                      f"after 1 warm-up, {threads} threads"}


def cpu_baseline_mixed(torch, wl, w):
    """Config 5 on the CPU: ONE layer (the 64 decode rows and the 2048-token
    chunk, LibTorch-CPU fp32), median of 5, scaled x layers as stated."""
    from oracle import torch_cpu as tc
    b, s = w.batch, w.shape
    threads = _cpu_threads(torch)
    hkv, hq, D = s.num_kv_heads, s.num_qo_heads, s.head_dim
    kc, vc, g = _cpu_pool(torch, b.num_slots, hkv, D, 5)
    rows = int(b.qo_indptr[-1])
    q = torch.randn((rows, hq, D), generator=g).to(torch.bfloat16)
    qo, kvl = b.qo_lens, b.kv_lens
    dec = np.nonzero(qo == 1)[0]
    pre = np.nonzero(qo > 1)[0]
    idx = torch.from_numpy(b.indices.astype(np.int64))
    kip = b.kv_indptr.astype(np.int64)
    scale = 1.0 / math.sqrt(D)
    # decode rows keep their own kv ranges; the chunk is a one-request prefill
    dec_ip = np.concatenate([[0], np.cumsum(kvl[dec])]).astype(np.int64)
    dec_idx = torch.cat([idx[kip[r]:kip[r + 1]] for r in dec])
    dec_q = q[torch.from_numpy(b.qo_indptr[dec].astype(np.int64))]
    pre_rows = [(int(b.qo_indptr[r]), int(b.qo_indptr[r + 1])) for r in pre]

    def layer():
        tc.decode(dec_q, kc, vc, dec_idx, dec_ip, scale)
        for (q0, q1), r in zip(pre_rows, pre):
            tc.prefill(q[q0:q1], kc, vc, idx[kip[r]:kip[r + 1]], np.array([0, q1 - q0]),
                       np.array([0, kvl[r]]), scale)

    med, runs = tc.median_time(layer)
    return {"ms_per_step": round(med * 1e3 * w.layers, 2), "unit": "ms per 48-layer step",
            "ms_per_layer": round(med * 1e3, 2), "cores": threads, "kind": "port",
            "cpu_model": tc.host_info()["cpu_model"], "runs_s": [round(t, 4) for t in runs],
            "sample": f"LibTorch-CPU fp32, one layer of {w.name} (64 decode rows + the "
                      f"2048-token chunk), median of 5 runs after 1 warm-up, scaled x{w.layers} "
                      f"layers, {threads} threads"}


# ------------------------------------------------------------------ main

def roofline_hbm(nbytes, kernel_ms, traffic_key):
    achieved = nbytes / (kernel_ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": load_traffic(traffic_key)}


def roofline_mfma(flops, kernel_ms, traffic_key):
    achieved = flops / (kernel_ms * 1e-3) / 1e12
    return {"bound": "mfma", "achieved": round(achieved, 2), "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": round(achieved / BF16_PEAK_TFLOPS, 4),
            "traffic": load_traffic(traffic_key)}


RESID_TOKENS, RESID_HIDDEN, RESID_INTER = 8192, 4096, 12288  # Qwen3-8B, one 8192-token chunk


def setup_resid(torch, capi, name, dev, seed=0, sets=1):
    """Residual-path kernels at the Qwen3-8B shape (qwen3.cc:24-31 and
    utils.cc:49 call them once per layer). Algorithmic bytes: fused add +
    RMSNorm reads x and residual and writes both (8 T d) plus the weight;
    SiLU-and-mul reads [T, 2d] and writes [T, d] (6 T d)."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    T = RESID_TOKENS
    if name == "resid_norm":
        d = RESID_HIDDEN
        w = (torch.rand(d, device=dev, generator=g) + 0.5).to(torch.bfloat16)

        def one_set():
            x = torch.randn((T, d), device=dev, generator=g).to(torch.bfloat16)
            r = torch.randn((T, d), device=dev, generator=g).to(torch.bfloat16)

            def step():
                # in place on x and r; repeated steps keep values finite (x is
                # renormalised each time, r grows by at most ~|x| per step)
                capi.fused_add_rmsnorm(x, r, w, 1e-6)
            return step

        return (rotating([one_set() for _ in range(sets)]), 8 * T * d + 2 * d,
                {"tokens": T, "hidden": d})
    d = RESID_INTER

    def one_set():
        inp = torch.randn((T, 2 * d), device=dev, generator=g).to(torch.bfloat16)
        out = torch.empty((T, d), device=dev, dtype=torch.bfloat16)

        def step():
            capi.silu_and_mul(out, inp)
        return step

    return rotating([one_set() for _ in range(sets)]), 6 * T * d, {"tokens": T, "intermediate": d}


SAMPLING_BATCH, QWEN3_VOCAB = 256, 151936


def setup_sampling(torch, capi, dev, seed=0, sets=1):
    """Top-k + top-p draw as the reference's Sampler::sample runs it
    (engine.cc:300-345): probs = softmax(logits / T) fp32 [256, 151936],
    uniform [32, 256], per-row top_k int32 and top_p. Algorithmic bytes: one
    read of probs (the rejection rounds re-read rows from L2)."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    B, V = SAMPLING_BATCH, QWEN3_VOCAB
    temp = torch.linspace(0.6, 1.2, B, device=dev).view(B, 1)
    u = torch.rand((32, B), device=dev, generator=g)
    k = torch.full((B,), 50, dtype=torch.int32, device=dev)
    tp = torch.full((B,), 0.9, dtype=torch.float32, device=dev)

    def one_set():
        logits = torch.randn((B, V), device=dev, generator=g) * 3
        probs = torch.softmax(logits / temp, -1).contiguous()
        del logits

        def step():
            capi.top_k_top_p_sampling_from_probs(probs, u, k, 0, tp, 0.0)
        return step

    return rotating([one_set() for _ in range(sets)]), B * V * 4 + 32 * B * 4 + B * 5, {
        "batch": B, "vocab": V, "top_k": 50, "top_p": 0.9}


# ------------------------------------------------------------------ ceilings

def load_probes():
    """libsgl_probes.so (sglang.cpp_amd/csrc/probes/ceilings.hip): raises if
    it is not built."""
    import ctypes
    path = REPO / "sglang.cpp_amd" / "libsgl_probes.so"
    if not path.exists():
        raise RuntimeError(f"{path} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(str(path))
    vp, i64, i32, u32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_uint32
    lib.sgl_probe_stream_read.argtypes = [vp, i64, i32, i32, vp, vp]
    lib.sgl_probe_mfma_bf16.argtypes = [i32, i32, i32, u32, vp, vp, vp]
    lib.sgl_probe_empty.argtypes = [i32, i32, vp]
    lib.sgl_probe_page_read.argtypes = [vp, vp, i32, i64, i32, i32, vp, vp]
    lib.sgl_probe_page_read.restype = i32
    lib.sgl_probe_decode_read.argtypes = [vp, vp, vp, i32, i32, i32, i32, i32, vp, vp]
    lib.sgl_probe_decode_read.restype = i32
    lib.sgl_probe_stream_copy.argtypes = [vp, vp, i64, i32, i32, vp]
    lib.sgl_probe_stream_copy.restype = i32
    for f in (lib.sgl_probe_stream_read, lib.sgl_probe_mfma_bf16, lib.sgl_probe_empty):
        f.restype = i32
    return lib


def _probe_ok(st, what):
    if st != 0:
        raise RuntimeError(f"{what} failed: status {st}")


MFMA_FLOPS = 32 * 32 * 16 * 2  # one v_mfma_f32_32x32x16_bf16


def measure_ceilings(torch, dev, min_warm_s=0.5, sweep=None):
    """Practical ceilings of this GPU, measured in this process:
    stream_read: best GB/s of a plain 16-byte streaming read of 2 GiB over
    grid sizes, loads in flight per lane (4, 8, 16), cached/non-temporal
    loads and grid-stride/block-contiguous order; mfma_random / mfma_const: TFLOP/s of back-to-back 32x32x16
    bf16 MFMAs (2 waves per SIMD on every CU) on random / constant operands,
    with the shader clock (MHz) each ran at; empty_launch_us: per-launch time
    of an empty 256-workgroup kernel, as a graph of 200 launches and eagerly."""
    lib = load_probes()
    s = torch.cuda.current_stream()
    sp = s.cuda_stream
    out = {}
    # stream read
    nbytes = 2 << 30
    buf = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    buf.random_(0, 256)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    best = (0.0, 0, 0)
    for variant, grid in [(v | b, g) for b in (0, 8) for v in range(6)
                          for g in (1024, 2048, 4096, 8192)]:
        def go():
            _probe_ok(lib.sgl_probe_stream_read(buf.data_ptr(), nbytes, grid, variant,
                                                sink.data_ptr(), sp), "sgl_probe_stream_read")
        for _ in range(3):
            go()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(10):
            go()
        e1.record(s)
        torch.cuda.synchronize()
        gbs = nbytes / (e0.elapsed_time(e1) / 10 * 1e-3) / 1e9
        if sweep is not None:
            sweep.append({"probe": "stream_read", "variant": variant, "grid": grid,
                          "GB/s": round(gbs, 1)})
        if gbs > best[0]:
            best = (gbs, grid, variant)
    # paged read: 32 KiB pages in a seeded random order
    page = 32 << 10
    npages = nbytes // page
    g = torch.Generator(device="cpu")
    g.manual_seed(0)
    order = torch.randperm(npages, generator=g).to(torch.int32).to(dev)
    pbest = (0.0, 0, 0)
    for pif, pgrid in [(f, gr) for f in (1, 2) for gr in (256, 512, 1024, 2048, 4096)]:
        def gop():
            _probe_ok(lib.sgl_probe_page_read(buf.data_ptr(), order.data_ptr(), npages, page, pgrid,
                                              pif, sink.data_ptr(), sp), "sgl_probe_page_read")
        for _ in range(3):
            gop()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(10):
            gop()
        e1.record(s)
        torch.cuda.synchronize()
        gbs = nbytes / (e0.elapsed_time(e1) / 10 * 1e-3) / 1e9
        if sweep is not None:
            sweep.append({"probe": "page_read", "pages_in_flight": pif, "grid": pgrid,
                          "GB/s": round(gbs, 1)})
        if gbs > pbest[0]:
            pbest = (gbs, pgrid, pif)
    out["page_read_32k"] = {"GB/s": round(pbest[0], 1),
                            "frac_of_published": round(pbest[0] / HBM_PEAK_GBS, 4),
                            "grid": pbest[1], "pages_in_flight": pbest[2], "page_bytes": page,
                            "bytes": nbytes}
    # the paged decode's load pattern: K and V pools of 2^19 2-KiB slots
    # (1 GiB each), 16-slot pages in a seeded random order
    slots = nbytes // 2 // 2048
    pages = torch.randperm(slots // 16, generator=g)
    tok_order = (pages.view(-1, 1) * 16 + torch.arange(16).view(1, 16)).reshape(-1)
    tok_order = tok_order.to(torch.int32).to(dev)
    kpool, vpool = buf[: nbytes // 2], buf[nbytes // 2:]
    dbest = {}
    for kmode, dgrid, bar, depth in [(m, gr, br, dp) for m in range(4) for gr in (256, 512, 1024)
                                     for br in (1, 0) for dp in (2, 3)]:
        def god():
            _probe_ok(lib.sgl_probe_decode_read(kpool.data_ptr(), vpool.data_ptr(),
                                                tok_order.data_ptr(), slots, dgrid, kmode, bar,
                                                depth, sink.data_ptr(), sp),
                      "sgl_probe_decode_read")
        for _ in range(3):
            god()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(10):
            god()
        e1.record(s)
        torch.cuda.synchronize()
        gbs = nbytes / (e0.elapsed_time(e1) / 10 * 1e-3) / 1e9
        if sweep is not None:
            sweep.append({"probe": "decode_read", "kmode": kmode, "grid": dgrid,
                          "barrier": bar, "depth": depth, "GB/s": round(gbs, 1)})
        key = ("k_operand_cached", "k_operand_nt", "k_rows_nt", "k_rows_cached")[kmode]
        if gbs > dbest.get(key, 0.0):
            dbest[key] = round(gbs, 1)
    out["decode_read_pattern"] = {"GB/s": dbest, "bytes": nbytes, "page_slots": 16,
                                  "slot_bytes": 2048}
    # read + write streams: a copy of 1 GiB into another 1 GiB, the same in
    # place, and a 2 GiB fill (bytes counted: everything read plus written)
    half = nbytes // 2
    a_, b_ = buf[:half], buf[half:]
    for key, src_, dst_, n_, counted, vars_ in (
            ("stream_copy", a_, b_, half, 2 * half, (0, 1, 2, 3, 4, 5, 6, 7)),
            ("stream_copy_inplace", a_, a_, half, 2 * half, (0, 1, 2, 3, 4, 5, 6, 7)),
            ("stream_write", None, buf, nbytes, nbytes, (8, 10, 12, 14))):
        cbest = (0.0, 0, 0)
        for variant, cgrid in [(v, gr) for v in vars_ for gr in (1024, 2048, 4096, 8192)]:
            def goc():
                _probe_ok(lib.sgl_probe_stream_copy(
                    None if src_ is None else src_.data_ptr(), dst_.data_ptr(), n_, cgrid,
                    variant, sp), "sgl_probe_stream_copy")
            for _ in range(3):
                goc()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for _ in range(10):
                goc()
            e1.record(s)
            torch.cuda.synchronize()
            gbs = counted / (e0.elapsed_time(e1) / 10 * 1e-3) / 1e9
            if sweep is not None:
                sweep.append({"probe": key, "variant": variant, "grid": cgrid,
                              "GB/s": round(gbs, 1)})
            if gbs > cbest[0]:
                cbest = (gbs, cgrid, variant)
        out[key] = {"GB/s": round(cbest[0], 1), "frac_of_published": round(cbest[0] / HBM_PEAK_GBS, 4),
                    "grid": cbest[1], "nt_loads": bool(cbest[2] & 1),
                    "nt_stores": bool(cbest[2] & 2), "in_flight": 16 if cbest[2] & 4 else 8,
                    "bytes": counted}
    del buf
    out["stream_read"] = {"GB/s": round(best[0], 1), "frac_of_published": round(best[0] / HBM_PEAK_GBS, 4),
                          "grid": best[1], "loads_in_flight": 4 << ((best[2] >> 1) & 3),
                          "non_temporal": bool(best[2] & 1),
                          "order": "block-contiguous" if best[2] & 8 else "grid-stride",
                          "bytes": nbytes}
    # MFMA issue
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    grid = 2 * cus
    iters = 20000
    fsink = torch.zeros(grid, dtype=torch.float32, device=dev)
    clocks = torch.zeros(grid * 4, dtype=torch.int64, device=dev)
    for kind, rnd in (("mfma_random", 1), ("mfma_const", 0)):
        def go():
            _probe_ok(lib.sgl_probe_mfma_bf16(grid, iters, rnd, 12345, fsink.data_ptr(),
                                              clocks.data_ptr(), sp), "sgl_probe_mfma_bf16")
        t0 = time.perf_counter()
        go()
        torch.cuda.synchronize()
        while time.perf_counter() - t0 < min_warm_s:
            go()
            torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(5):
            go()
        e1.record(s)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / 5
        flops = grid * 4 * iters * 4 * MFMA_FLOPS
        c = clocks.view(grid, 4).cpu().numpy().astype(np.float64)
        mhz = np.median((c[:, 1] - c[:, 0]) / np.maximum(c[:, 3] - c[:, 2], 1) * 100.0)
        tf = flops / (ms * 1e-3) / 1e12
        out[kind] = {"TFLOP/s": round(tf, 1), "frac_of_published": round(tf / BF16_PEAK_TFLOPS, 4),
                     "shader_clock_MHz": round(float(mhz), 0), "ms": round(ms, 4),
                     "waves_per_simd": 2, "workgroups": grid}
    # empty launch
    def empty():
        _probe_ok(lib.sgl_probe_empty(256, 256, torch.cuda.current_stream().cuda_stream),
                  "sgl_probe_empty")
    timer = Timer(torch, 0.1)
    wall, ev = timer.run_graph(empty, 200, 10)
    ewall, eev = timer.run(empty, 200, 10)
    out["empty_launch_us"] = {"graph": round(ev * 1e3, 2), "eager": round(eev * 1e3, 2),
                              "workgroups": 256}
    return out


# HBM-bound workloads that write half or more of their bytes: held against
# the streaming copy's ceiling (read and write together), the others
# against the streaming read's.
WRITE_HEAVY = ("cfg3", "resid_norm", "sampler_softmax")


def ceiling_fracs(extra, ceil):
    """Each kernel's achieved rate over the practical ceiling of its bound."""
    sr = ceil["stream_read"]["GB/s"]
    cr = ceil.get("stream_copy", {}).get("GB/s", sr)
    mr = ceil["mfma_random"]["TFLOP/s"]
    fr = {}
    for name, rec in extra.items():
        rl = rec.get("roofline") if isinstance(rec, dict) else None
        if not rl:
            continue
        if rl["bound"] == "hbm":
            c = cr if name in WRITE_HEAVY else sr
        else:
            c = mr
        fr[name] = round(rl["achieved"] / c, 4)
    return fr


def setup_sampler_softmax(torch, capi, dev, seed=0, sets=1):
    """The probabilities of Sampler::sample (engine.cc:306-308) for the
    sampling workload's batch: bf16 logits [256, 151936] (the LM head's
    output), per-row temperatures. Algorithmic bytes: one read of the
    logits, one write of the fp32 probabilities, the temperatures. Also
    returns the reference's own statements on the same device
    (logits.to(float32) / temperatures, torch.softmax) for comparison."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    B, V = SAMPLING_BATCH, QWEN3_VOCAB
    temps = torch.linspace(0.6, 1.2, B, device=dev)

    def one_set():
        logits = (torch.randn((B, V), device=dev, generator=g) * 3).to(torch.bfloat16)
        out = torch.empty((B, V), device=dev)

        def step():
            capi.softmax_temperature(logits, temps, out=out)

        def torch_step():
            torch.softmax(logits.to(torch.float32) / temps.view(B, 1), -1)
        return step, torch_step

    pairs = [one_set() for _ in range(sets)]
    return (rotating([p[0] for p in pairs]), rotating([p[1] for p in pairs]),
            B * V * (2 + 4) + 4 * B, {"batch": B, "vocab": V, "logits": "bf16"})


def setup_sampler_step(torch, capi, dev, seed=0, sets=1):
    """The whole Sampler step as engine.cc:306-333 runs it for the sampling
    workload's rows: bf16 logits [256, 151936], per-row temperatures,
    top-k 50 + top-p 0.9, uniform [32, 256]. Returns the fused launch
    (probabilities computed inside the draw, never stored), our two launches
    (softmax_temperature, then the draw) and the reference's statements for
    the probabilities (LibTorch) followed by our draw. Algorithmic bytes of
    the step: one read of the logits."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    B, V = SAMPLING_BATCH, QWEN3_VOCAB
    temps = torch.linspace(0.6, 1.2, B, device=dev)
    u = torch.rand((32, B), device=dev, generator=g)
    k = torch.full((B,), 50, dtype=torch.int32, device=dev)
    tp = torch.full((B,), 0.9, dtype=torch.float32, device=dev)
    probs = torch.empty((B, V), device=dev)

    def one_set():
        logits = (torch.randn((B, V), device=dev, generator=g) * 3).to(torch.bfloat16)

        def fused():
            capi.sampling_from_logits(logits, u, "top_k_top_p", temps, top_k=k, top_p=tp)

        def two():
            capi.softmax_temperature(logits, temps, out=probs)
            capi.top_k_top_p_sampling_from_probs(probs, u, k, 0, tp, 0.0)

        def torch_probs():
            p = torch.softmax(logits.to(torch.float32) / temps.view(B, 1), -1).contiguous()
            capi.top_k_top_p_sampling_from_probs(p, u, k, 0, tp, 0.0)
        return fused, two, torch_probs

    trip = [one_set() for _ in range(sets)]
    return (rotating([t[0] for t in trip]), rotating([t[1] for t in trip]),
            rotating([t[2] for t in trip]), B * V * 2 + 4 * B + 32 * B * 4, {
                "batch": B, "vocab": V, "logits": "bf16", "top_k": 50, "top_p": 0.9})


# Whether rotated workloads also time their one-set (cache-resident) leg;
# off for profiler runs, whose summaries then hold the rotated launches only.
RESIDENT_LEG = True


def _resident_leg(run, step, steps, warmup):
    return run(step, steps, warmup)[1] if RESIDENT_LEG else None


def _resident(rec_rot, ev_1, nbytes=None, flops=None, sets=1):
    """The one-set (cache-resident) figure beside a rotated-buffer record."""
    rec_rot["buffer_sets"] = sets
    rec_rot["rotated_bytes"] = ROTATE_BYTES
    if ev_1 is None:
        return rec_rot
    out = {"kernel_ms": ev_1}
    if nbytes:
        out["GB/s"] = nbytes / (ev_1 * 1e-3) / 1e9
        out["hbm_frac"] = round(out["GB/s"] / HBM_PEAK_GBS, 4)
    if flops:
        out["TFLOP/s"] = flops / (ev_1 * 1e-3) / 1e12
        out["mfma_frac"] = round(out["TFLOP/s"] / BF16_PEAK_TFLOPS, 4)
    rec_rot["cache_resident"] = out
    return rec_rot


def run_workload(name, torch, capi, wl, dev, steps, warmup, cfg5_layers, min_warm_s=0.0):
    timer = Timer(torch, min_warm_s)
    if name == "sampler_step":
        fused, two, torch_probs, nbytes, shape = setup_sampler_step(torch, capi, dev)
        ev1 = _resident_leg(timer.run_graph, fused, steps, warmup)
        del fused, two, torch_probs
        sets = rotation_sets(nbytes)
        fused, two, torch_probs, nbytes, shape = setup_sampler_step(torch, capi, dev, sets=sets)
        ewall, eev = timer.run(fused, steps, warmup)
        wall, ev = timer.run_graph(fused, steps, warmup)
        _, two_ev = timer.run_graph(two, steps, warmup)
        _, tp_ev = timer.run_graph(torch_probs, steps, warmup)
        rec = {"workload": f"sampler_step_top_k_top_p_b{SAMPLING_BATCH}_v{QWEN3_VOCAB}", **shape,
               "ms_per_step": wall, "kernel_ms": ev, "eager_ms_per_step": ewall,
               "eager_kernel_ms": eev, "timing": "graph", "bytes": nbytes,
               "GB/s": nbytes / (wall * 1e-3) / 1e9,
               "two_launch_ms": two_ev, "torch_probs_then_draw_ms": tp_ev,
               "speedup_vs_torch_probs_then_draw": tp_ev / ev,
               "roofline": roofline_hbm(nbytes, ev, "sampler_step_top_k_top_p")}
        return None, _resident(rec, ev1, nbytes, sets=sets)
    if name == "sampler_softmax":
        step, torch_step, nbytes, shape = setup_sampler_softmax(torch, capi, dev)
        ev1 = _resident_leg(timer.run_graph, step, steps, warmup)
        del step, torch_step
        torch.cuda.empty_cache()
        sets = rotation_sets(nbytes)
        step, torch_step, nbytes, shape = setup_sampler_softmax(torch, capi, dev, sets=sets)
        ewall, eev = timer.run(step, steps, warmup)
        wall, ev = timer.run_graph(step, steps, warmup)
        _, tev = timer.run_graph(torch_step, steps, warmup)
        rec = {"workload": f"sampler_softmax_b{SAMPLING_BATCH}_v{QWEN3_VOCAB}", **shape,
               "ms_per_step": wall, "kernel_ms": ev, "eager_ms_per_step": ewall,
               "eager_kernel_ms": eev, "timing": "graph", "bytes": nbytes,
               "GB/s": nbytes / (wall * 1e-3) / 1e9,
               "torch_path_ms": tev, "speedup_vs_torch_path": tev / ev,
               "roofline": roofline_hbm(nbytes, ev, "softmax_temperature_sampler")}
        return None, _resident(rec, ev1, nbytes, sets=sets)
    if name == "sampling":
        step, nbytes, shape = setup_sampling(torch, capi, dev)
        ev1 = _resident_leg(timer.run, step, steps, warmup)
        del step
        torch.cuda.empty_cache()
        sets = rotation_sets(nbytes)
        step, nbytes, shape = setup_sampling(torch, capi, dev, sets=sets)
        wall, ev = timer.run(step, steps, warmup)
        rec = {"workload": f"sampling_top_k_top_p_b{SAMPLING_BATCH}_v{QWEN3_VOCAB}", **shape,
               "ms_per_step": wall, "kernel_ms": ev, "bytes": nbytes,
               "GB/s": nbytes / (wall * 1e-3) / 1e9,
               "roofline": roofline_hbm(nbytes, ev, "sampling_top_k_top_p")}
        return None, _resident(rec, ev1, nbytes, sets=sets)
    if name in ("resid_norm", "resid_act"):
        step, nbytes, shape = setup_resid(torch, capi, name, dev)
        ev1 = _resident_leg(timer.run, step, steps, warmup)
        del step
        torch.cuda.empty_cache()
        sets = rotation_sets(nbytes)
        step, nbytes, shape = setup_resid(torch, capi, name, dev, sets=sets)
        wall, ev = timer.run(step, steps, warmup)
        kname = "fused_add_rmsnorm" if name == "resid_norm" else "silu_and_mul"
        rec = {"workload": f"{name}_qwen3_8b_t{RESID_TOKENS}_bf16", **shape, "ms_per_step": wall,
               "kernel_ms": ev, "bytes": nbytes, "GB/s": nbytes / (wall * 1e-3) / 1e9,
               "roofline": roofline_hbm(nbytes, ev, f"{kname}_qwen3_8b")}
        return None, _resident(rec, ev1, nbytes, sets=sets)
    # Configurations 1, 2 and 3 are single calls of 10-25 us, within a few us
    # of the host's per-call launch cost from Python: they are timed as a
    # captured graph of the K calls (the eager figures are kept beside them).
    if name in ("cfg1", "cfg4"):
        w = wl.cfg1_decode_small() if name == "cfg1" else wl.cfg4_decode_large()
        step, nbytes, flops, _ = setup_decode(torch, capi, wl, w, dev)
        wall, ev = timer.run(step, steps, warmup)
        eager = {}
        if name == "cfg1":
            eager = {"eager_ms_per_step": wall, "eager_kernel_ms": ev, "timing": "graph"}
            wall, ev = timer.run_graph(step, steps, warmup)
        rec = {"workload": w.name, "ms_per_step": wall, "kernel_ms": ev, **eager, "bytes": nbytes,
               "GB/s": nbytes / (wall * 1e-3) / 1e9,
               "roofline": roofline_hbm(nbytes, ev, "paged_decode_" + name)}
        return w, rec
    if name in ("cfg2", "prefill_chunk"):
        w = wl.cfg2_prefill_prefix() if name == "cfg2" else wl.cfg5_prefill_chunk()
        key = "paged_prefill_cfg2" if name == "cfg2" else "paged_prefill_cfg5_chunk"
        step, nbytes, flops = setup_prefill(torch, capi, wl, w, dev)
        if name == "cfg2":
            # 21 MB, latency-bound: timed on one set, as a graph of the K calls
            wall, ev = timer.run(step, steps, warmup)
            eager = {"eager_ms_per_step": wall, "eager_kernel_ms": ev, "timing": "graph"}
            wall, ev = timer.run_graph(step, steps, warmup)
            sets, ev1 = 1, None
        else:
            ev1 = _resident_leg(timer.run, step, steps, warmup)
            del step
            sets = rotation_sets(nbytes)
            step, nbytes, flops = setup_prefill(torch, capi, wl, w, dev, sets=sets)
            wall, ev = timer.run(step, steps, warmup)
            eager = {}
        rec = {"workload": w.name, "ms_per_step": wall, "kernel_ms": ev, **eager, "flops": flops,
               "bytes": nbytes, "TFLOP/s": flops / (wall * 1e-3) / 1e12,
               "GB/s": nbytes / (wall * 1e-3) / 1e9,
               "roofline": roofline_mfma(flops, ev, key),
               "roofline_hbm": roofline_hbm(nbytes, ev, None)}
        if name != "cfg2":
            rec = _resident(rec, ev1, nbytes, flops, sets=sets)
        return w, rec
    if name == "cfg3":
        w = wl.cfg3_fused_store()
        step, nbytes = setup_fused(torch, capi, wl, w, dev)
        ev1 = _resident_leg(timer.run_graph, step, steps, warmup)
        del step
        torch.cuda.empty_cache()
        sets = rotation_sets(nbytes)
        step, nbytes = setup_fused(torch, capi, wl, w, dev, sets=sets)
        wall, ev = timer.run(step, steps, warmup)
        eager = {"eager_ms_per_step": wall, "eager_kernel_ms": ev, "timing": "graph"}
        wall, ev = timer.run_graph(step, steps, warmup)
        rec = {"workload": w.name, "ms_per_step": wall, "kernel_ms": ev, **eager, "bytes": nbytes,
               "GB/s": nbytes / (wall * 1e-3) / 1e9,
               "roofline": roofline_hbm(nbytes, ev, "fused_qknorm_rope_store_cfg3")}
        return w, _resident(rec, ev1, nbytes, sets=sets)
    if name == "cfg5":
        w = wl.cfg5_mixed(layers=cfg5_layers)
        step, dec_bytes, pre_flops, pre_bytes, keep = setup_mixed(torch, wl, w, dev, cfg5_layers)
        wall, ev = timer.run(step, max(2, steps // 4), max(1, warmup // 2))
        t_roof = dec_bytes / (HBM_PEAK_GBS * 1e9) + pre_flops / (BF16_PEAK_TFLOPS * 1e12)
        rec = {"workload": w.name, "layers": cfg5_layers, "ms_per_step": wall, "graph_ms": ev,
               "decode_bytes": dec_bytes, "prefill_flops": pre_flops,
               "t_roofline_ms": t_roof * 1e3, "roofline_frac": t_roof * 1e3 / ev}
        del keep
        return w, rec
    raise ValueError(name)


def main():
    args = parse()
    global RESIDENT_LEG
    RESIDENT_LEG = not args.no_resident_leg
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the attention hot "
              "path is single-GPU in this build — run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    import __graft_entry__ as entry
    pkg = entry.load_package()
    capi, wl = pkg.capi, pkg.workloads
    capi.lib()
    if not torch.cuda.is_available():
        print("bench.py needs a HIP GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": n, "steps": args.steps}))
        return

    if args.replay_host_only:
        print(json.dumps({"replay_host": measure_replay_host(torch, wl, dev)}), flush=True)
        return

    if args.ceilings_only:
        sweep = []
        ceil = measure_ceilings(torch, dev, args.min_warm_seconds, sweep)
        print(json.dumps({"ceilings": ceil, "sweep": sweep}), flush=True)
        return

    w, head = run_workload(args.workload, torch, capi, wl, dev, args.steps, args.warmup,
                           args.cfg5_layers, args.min_warm_seconds)
    extra = {}
    if not args.no_extra:
        for name in ("cfg1", "cfg2", "cfg3", "cfg4", "cfg5", "prefill_chunk", "resid_norm",
                     "resid_act", "sampling", "sampler_softmax", "sampler_step"):
            if name == args.workload:
                continue
            try:
                _, rec = run_workload(name, torch, capi, wl, dev, args.steps, args.warmup,
                                      args.cfg5_layers, args.min_warm_seconds)
                extra[name] = rec
            except Exception as e:  # report, keep the headline line
                extra[name] = {"error": repr(e)}
            torch.cuda.empty_cache()
            print(f"[bench] {name}: {json.dumps(extra[name])}", file=sys.stderr, flush=True)

    if not args.no_extra:
        try:
            extra["replay_host"] = measure_replay_host(torch, wl, dev)
        except Exception as e:  # report, keep the headline line
            extra["replay_host"] = {"error": repr(e)}
        print(f"[bench] replay_host: {json.dumps(extra['replay_host'])}", file=sys.stderr,
              flush=True)
        try:
            ceil = measure_ceilings(torch, dev, args.min_warm_seconds)
            extra["ceilings"] = ceil
            extra["ceiling_frac"] = ceiling_fracs({args.workload: head, **extra}, ceil)
        except Exception as e:  # report, keep the headline line
            extra["ceilings"] = {"error": repr(e)}
        print(f"[bench] ceilings: {json.dumps(extra['ceilings'])}", file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu:
        if args.workload in ("cfg1", "cfg4"):
            cpu = cpu_baseline_decode(torch, wl, w)
        elif args.workload == "cfg2":
            cpu = cpu_baseline_prefill(torch, wl, w)
        elif args.workload == "cfg3":
            cpu = cpu_baseline_fused(torch, wl, w)
        elif args.workload == "cfg5":
            cpu = cpu_baseline_mixed(torch, wl, w)
        if args.workload == "cfg4" and not args.no_extra:
            # the other CPU legs of the plan, beside their GPU lines in extra
            for name, fn in (("cfg2", lambda: cpu_baseline_prefill(torch, wl,
                                                                   wl.cfg2_prefill_prefix())),
                             ("cfg3", lambda: cpu_baseline_fused(torch, wl, wl.cfg3_fused_store())),
                             ("cfg5", lambda: cpu_baseline_mixed(torch, wl,
                                                                 wl.cfg5_mixed(layers=48)))):
                try:
                    rec = fn()
                except Exception as e:  # report, keep the headline line
                    rec = {"error": repr(e)}
                if name in extra:
                    extra[name]["cpu_baseline"] = rec
                print(f"[bench] cpu {name}: {json.dumps(rec)}", file=sys.stderr, flush=True)

    if "GB/s" in head and args.workload != "cfg2":
        value, unit = head["GB/s"], "GB/s"
    elif args.workload == "cfg2":
        value, unit = head["TFLOP/s"], "TFLOP/s"
    else:
        value, unit = head["decode_bytes"] / (head["ms_per_step"] * 1e-3) / 1e9, "GB/s"
    if w is None:
        config = {"workload": head["workload"], "parallelism": "single GPU",
                  **{k: head[k] for k in ("tokens", "hidden", "intermediate", "batch", "vocab",
                                          "top_k", "top_p", "logits") if k in head}}
    else:
        s = w.shape
        config = {"workload": head["workload"], "batch": w.batch.batch_size,
                  "num_qo_heads": s.num_qo_heads, "num_kv_heads": s.num_kv_heads,
                  "head_dim": s.head_dim, "page_size": w.batch.page_size,
                  "sum_kv": int(w.batch.kv_lens.sum()), "parallelism": "single GPU"}
    if head.get("timing") == "graph":
        config["timing"] = "one hipGraph of the K calls (eager figures in extra)"
        extra.setdefault(args.workload, {k: head[k] for k in ("eager_ms_per_step", "eager_kernel_ms",
                                                              "torch_path_ms",
                                                              "speedup_vs_torch_path",
                                                              "two_launch_ms",
                                                              "torch_probs_then_draw_ms")
                                         if k in head})
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "min_warm_seconds": args.min_warm_seconds,
        "ms_per_step": round(head["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) bf16 Q/K/V, seeded random page permutation",
        "config": config,
        "roofline": head.get("roofline"),
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
