"""Benchmark configuration 5 at its own shape, through HipAttnBackend:
64 decode rows with kv ~ U[1024, 32768] beside one 2048-token prefill chunk
on a 4096-token cached prefix, Qwen3-30B-A3B attention (32q/4kv, d128),
page_size 16 -- eagerly, then through one captured graph replayed with new
lengths (the mixed-step extension of the reference's capture contract,
src/attention/flashinfer_backend.cu:193-219,267-352; GraphRunner,
src/engine/engine.cc:670-743).

The oracle checks every decode row of the eager step, a sample of decode
rows that always holds the longest request on each replay, and 256 (eager) or
128 (replay) rows of the chunk including its first and last tokens. A chunk
row i sees the kv prefix [0, kv - qo + i] of its request, so each sampled
row is one oracle decode over that prefix (the causal prefill's definition,
src/attention/flashinfer_backend.cu:596-679, bottom-right alignment).
"""
import math
import sys

import numpy as np
import pytest
import torch

from conftest import pkg, wl
from helpers import assert_attn_close, u16

pytestmark = pytest.mark.gpu

D = 128
HQ, HKV, P = 32, 4, 16
L = 32768          # longest request (page-table row width)
N_DEC = 64
CHUNK = 2048       # captured prefill chunk capacity
SCALE = 1 / math.sqrt(D)


def note(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


class Cfg5:
    """Pool with a full page-table row per request (64 decode + 1 prefill),
    the spare page as the padding slot."""

    def __init__(self, sb, dev):
        rng = np.random.default_rng(70)
        self.full = wl.make_paged_batch(rng, [L - 1] * (N_DEC + 1), [L] * (N_DEC + 1),
                                        page_size=P)
        self.pt = self.full.page_table
        self.dummy_slot = int(self.pt[N_DEC + 1, 0])
        self.cache = sb.MHAKVCache(HKV, 1, D, self.full.num_pages + 1, P, 0)
        g = torch.Generator(device=dev)
        g.manual_seed(71)
        buf = self.cache.buffer()
        for i in range(2):  # K then V, in two draws to bound the temporary
            buf[i].copy_(torch.randn(tuple(buf[i].shape), device=dev, generator=g)
                         .to(torch.bfloat16))
        self.backend = sb.HipAttnBackend(self.cache, HQ, HKV, D)
        self.backend.set_page_table(torch.from_numpy(self.pt).to(dev))
        self.g = g
        self.sb, self.dev = sb, dev
        torch.cuda.synchronize()
        # host mirror of the pool (the oracle's inputs), updated with every store
        self.kc = u16(self.cache.k_cache(0))
        self.vc = u16(self.cache.v_cache(0))

    def step(self, dec_lens, cached, dev_len):
        """A mixed batch: decode requests i < 64 (row i), then the chunk (row 64)."""
        sb = self.sb
        reqs = [sb.Req(i, int(n) - 1, int(n)) for i, n in enumerate(dec_lens)]
        reqs.append(sb.Req(N_DEC, int(cached), int(dev_len)))
        pos = np.concatenate([np.asarray(dec_lens) - 1,
                              np.arange(cached, dev_len)]).astype(np.int32)
        rows = np.concatenate([np.arange(N_DEC), np.full(dev_len - cached, N_DEC)])
        loc = self.pt[rows, pos].astype(np.int32)
        T = len(pos)
        q = torch.randn((T, HQ * D), device=self.dev, generator=self.g).to(torch.bfloat16)
        k = torch.randn((T, HKV * D), device=self.dev, generator=self.g).to(torch.bfloat16)
        v = torch.randn((T, HKV * D), device=self.dev, generator=self.g).to(torch.bfloat16)
        batch = sb.Batch(True, reqs, torch.from_numpy(pos).to(self.dev),
                         torch.from_numpy(loc).to(self.dev))
        return dict(batch=batch, q=q, k=k, v=v, loc=loc, T=T, dec_lens=np.asarray(dec_lens),
                    cached=cached, dev_len=dev_len)

    def apply_store(self, st):
        T = st["T"]
        self.kc[st["loc"]] = u16(st["k"]).reshape(T, HKV, D)
        self.vc[st["loc"]] = u16(st["v"]).reshape(T, HKV, D)

    def check(self, oracle, st, o, dec_sample, chunk_sample, what):
        got = o.float().cpu().numpy().reshape(-1, HQ, D)
        qh = u16(st["q"]).reshape(st["T"], HQ, D)
        lens = st["dec_lens"]
        # decode rows
        ip = np.concatenate([[0], np.cumsum(lens[dec_sample])]).astype(np.int32)
        idx = np.concatenate([self.pt[r, :lens[r]] for r in dec_sample]).astype(np.int32)
        ref = oracle.decode(qh[dec_sample].copy(), self.kc, self.vc, idx, ip, SCALE)
        assert_attn_close(got[dec_sample], ref, what=f"{what}: decode rows")
        # chunk rows: row i sees the prefix [0, cached + i]
        cached = st["cached"]
        ip = np.concatenate([[0], np.cumsum(cached + chunk_sample + 1)]).astype(np.int32)
        idx = np.concatenate([self.pt[N_DEC, :cached + i + 1] for i in chunk_sample])
        ref = oracle.decode(qh[N_DEC + chunk_sample].copy(), self.kc, self.vc,
                            idx.astype(np.int32), ip, SCALE)
        assert_attn_close(got[N_DEC + chunk_sample], ref, what=f"{what}: chunk rows")


def chunk_rows(rng, qo, n):
    edge = np.array([0, 1, 2, qo - 3, qo - 2, qo - 1])
    mid = rng.choice(np.arange(3, qo - 3), n - len(edge), replace=False)
    return np.unique(np.concatenate([edge, mid]))


def test_cfg5_mixed_eager_and_graph_replay(oracle, dev):
    sb = pkg.backend.load()
    note("cfg5 at its own shape: eager step")
    c = Cfg5(sb, dev)
    # the benchmark workload's own lengths (seeded draw of wl.cfg5_mixed)
    w = wl.cfg5_mixed(layers=1)
    dec0 = w.batch.device_lens[:N_DEC].astype(np.int64)
    assert (w.batch.cached_lens[N_DEC], w.batch.device_lens[N_DEC]) == (4096, 6144)
    assert (w.shape.num_qo_heads, w.shape.num_kv_heads, w.batch.page_size) == (HQ, HKV, P)
    st = c.step(dec0, 4096, 6144)
    b = st["batch"]
    c.backend.prepare_metadata(b)
    assert b.num_decode_rows() == N_DEC and b.num_prefill_rows() == 1
    # the one-launch mixed path: decode rows on a share of the CUs
    assert 8 <= b.fused_mixed_cus() < 256
    o = c.backend.forward(st["q"], st["k"], st["v"], 0, b)
    torch.cuda.synchronize()
    c.apply_store(st)
    # the store is bit-exact at the new tokens' slots
    np.testing.assert_array_equal(u16(c.cache.k_cache(0)[torch.from_numpy(st["loc"]).to(dev)]),
                                  c.kc[st["loc"]])
    rng = np.random.default_rng(72)
    c.check(oracle, st, o, np.arange(N_DEC), chunk_rows(rng, 2048, 256), "eager cfg5")
    note(f"cfg5 eager ok; longest decode row {int(dec0.max())}")

    # capture the step once (fixed-address metadata), then replay new lengths
    be = c.backend
    be.init_mixed_capture_graph(L, N_DEC, 1, CHUNK)
    T_cap = st["T"]
    static_q = st["q"].clone()
    static_k = st["k"].clone()
    static_v = st["v"].clone()
    static_loc = torch.from_numpy(st["loc"]).to(dev)
    cap = sb.Batch(True, [sb.Req(r.table_idx, r.cached_len, r.device_len())
                          for r in b.padded_reqs], b.positions, static_loc)
    be.prepare_for_capture(cap)
    assert cap.uses_capture_buffers() and cap.fused_mixed_cus() == b.fused_mixed_cus()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        be.forward(static_q, static_k, static_v, 0, cap)  # warm-up (same values re-stored)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_o = be.forward(static_q, static_k, static_v, 0, cap)
    torch.cuda.synchronize()

    longest = np.full(N_DEC, 1024)
    longest[[5, 40]] = L
    sets = [
        ("replay 1: new decode lengths, same chunk", rng.integers(1024, L + 1, N_DEC), 4096, 6144),
        ("replay 2: 1500-token chunk on a 2000 prefix, two 32K rows", longest, 2000, 3500),
        ("replay 3: 2048-token chunk on a 30720 prefix, short rows",
         rng.integers(1, 300, N_DEC), L - CHUNK, L),
    ]
    for what, lens, cached, dev_len in sets:
        note(what)
        st = c.step(lens, cached, dev_len)
        rb = st["batch"]
        be.prepare_metadata(rb)
        be.prepare_for_replay(rb)
        T = st["T"]
        assert T <= T_cap
        static_q.zero_()
        static_q[:T].copy_(st["q"])
        static_k[:T].copy_(st["k"])
        static_v[:T].copy_(st["v"])
        static_loc.fill_(c.dummy_slot)  # padding rows store into the spare page
        static_loc[:T].copy_(torch.from_numpy(st["loc"]).to(dev))
        graph.replay()
        torch.cuda.synchronize()
        c.apply_store(st)
        dec_sample = np.unique(np.concatenate([[int(np.argmax(lens))],
                                               rng.choice(N_DEC, 23, replace=False)]))
        c.check(oracle, st, static_o[:T], dec_sample, chunk_rows(rng, dev_len - cached, 128),
                what)
        assert torch.isfinite(static_o[:T].float()).all()
    # capacity checks on the host: a chunk longer than captured is refused
    st = c.step(np.full(N_DEC, 100), 0, CHUNK + 16)
    be.prepare_metadata(st["batch"])
    with pytest.raises(RuntimeError, match="max_prefill_qo"):
        be.prepare_for_replay(st["batch"])
