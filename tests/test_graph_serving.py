"""Serving-loop contracts around the backend, against the oracle:

* the scheduler's stream overlap: step n + 1's metadata is prepared on a
  scheduler stream while step n's forward runs on the engine stream, which
  waits on the prepare's event, and the metadata tensors are marked used on
  the engine stream (src/scheduler/scheduler.cc:152-180,276,391-396; the
  reference backend's pinned ring, src/attention/flashinfer_backend.cu:
  103-128), eagerly and through a replayed decode graph;
* GraphRunner::pad_batch (src/engine/engine.cc:628-645) for mixed steps: a
  step with fewer decode rows than a captured mixed graph is padded with the
  dummy request (the page table's spare row) and replayed through it; the
  padding rows read and write only the spare slot.
"""
import math
import sys

import numpy as np
import pytest
import torch

from conftest import pkg, wl
from helpers import assert_attn_close, u16

pytestmark = pytest.mark.gpu

D, P = 128, 16
SCALE = 1 / math.sqrt(D)


def note(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _pool(sb, dev, num_pages, hkv, seed):
    cache = sb.MHAKVCache(hkv, 1, D, num_pages + 1, P, 0)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    buf = cache.buffer()
    buf.copy_(torch.randn(tuple(buf.shape), device=dev, generator=g).to(torch.bfloat16))
    return cache, g


def _record(batch, stream):
    batch.record_metadata_stream(stream.stream_id, stream.device_index)
    batch.positions.record_stream(stream)
    batch.out_loc.record_stream(stream)


# ------------------------------------------------------------------ stream overlap

HQ_O, HKV_O, B_O, STEPS = 32, 8, 48, 6


class Overlap:
    """Decode steps of B_O requests growing one token per step over a page
    table holding every slot they will need (pages allocated up front)."""

    def __init__(self, sb, dev):
        rng = np.random.default_rng(120)
        self.lens0 = rng.integers(256, 3000, B_O)
        last = self.lens0 + 2 * STEPS
        self.full = wl.make_paged_batch(rng, last - 1, last, page_size=P, decode=True)
        self.pt = self.full.page_table
        self.cache, self.g = _pool(sb, dev, self.full.num_pages, HKV_O, 121)
        self.backend = sb.HipAttnBackend(self.cache, HQ_O, HKV_O, D)
        self.backend.set_page_table(torch.from_numpy(self.pt).to(dev))
        self.sb, self.dev = sb, dev
        torch.cuda.synchronize()
        self.kc = u16(self.cache.k_cache(0))
        self.vc = u16(self.cache.v_cache(0))
        n = 2 * STEPS
        self.q = [torch.randn((B_O, HQ_O * D), device=dev, generator=self.g).to(torch.bfloat16)
                  for _ in range(n)]
        self.k = [torch.randn((B_O, HKV_O * D), device=dev, generator=self.g).to(torch.bfloat16)
                  for _ in range(n)]
        self.v = [torch.randn((B_O, HKV_O * D), device=dev, generator=self.g).to(torch.bfloat16)
                  for _ in range(n)]
        torch.cuda.synchronize()

    def lens(self, n):
        return self.lens0 + n + 1

    def batch(self, n):
        """Step n's batch, its positions and slots sent from the current stream."""
        lens = self.lens(n)
        reqs = [self.sb.Req(i, int(x) - 1, int(x)) for i, x in enumerate(lens)]
        pos = (lens - 1).astype(np.int32)
        loc = self.pt[np.arange(B_O), pos].astype(np.int32)
        return self.sb.Batch(False, reqs, torch.from_numpy(pos).to(self.dev, non_blocking=True),
                             torch.from_numpy(loc).to(self.dev, non_blocking=True)), loc

    def expect(self, n, loc):
        self.kc[loc] = u16(self.k[n]).reshape(B_O, HKV_O, D)
        self.vc[loc] = u16(self.v[n]).reshape(B_O, HKV_O, D)
        lens = self.lens(n)
        ip = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        idx = np.concatenate([self.pt[r, :lens[r]] for r in range(B_O)]).astype(np.int32)
        q = u16(self.q[n]).reshape(B_O, HQ_O, D).copy()
        from oracle import oracle
        return oracle.decode(q, self.kc, self.vc, idx, ip, SCALE).reshape(B_O, -1)


def _busy(x):
    """Engine-stream work ahead of each forward, so the scheduler stream's
    prepare of the next step runs while the engine is still on this one."""
    for _ in range(3):
        x = x @ x
        x = x * (1.0 / x.abs().max().clamp(min=1.0))
    return x


def test_prepare_on_scheduler_stream_overlaps_forward(oracle, dev):
    sb = pkg.backend.load()
    ov = Overlap(sb, dev)
    engine = torch.cuda.current_stream()
    sched = torch.cuda.Stream()
    busy = torch.randn((2048, 2048), device=dev, generator=ov.g).to(torch.bfloat16)
    results = []

    def prepare(n):
        with torch.cuda.stream(sched):
            b, loc = ov.batch(n)
            ov.backend.prepare_metadata(b)
            ev = torch.cuda.Event()
            ev.record(sched)
        return b, loc, ev

    # eager steps: forward n on the engine stream, prepare n + 1 on the
    # scheduler stream meanwhile; each batch dropped on the host as soon as
    # its forward is queued (its tensors freed while the engine may still
    # read them: record_stream keeps them from being reused too early)
    note("overlap: eager steps")
    nxt = prepare(0)
    for n in range(STEPS):
        b, loc, ev = nxt
        nxt = None
        engine.wait_event(ev)
        _record(b, engine)
        busy = _busy(busy)
        o = ov.backend.forward(ov.q[n], ov.k[n], ov.v[n], 0, b)
        results.append((n, loc, o))
        del b
        if n + 1 < STEPS:
            nxt = prepare(n + 1)
    torch.cuda.synchronize()

    # replayed steps: one captured decode graph; prepare_for_replay runs on
    # the engine stream after the wait, as GraphRunner::replay does
    note("overlap: replayed steps")
    be = ov.backend
    be.init_capture_graph(int(ov.pt.shape[1]), [B_O])
    sq = torch.zeros((B_O, HQ_O * D), device=dev, dtype=torch.bfloat16)
    sk = torch.zeros((B_O, HKV_O * D), device=dev, dtype=torch.bfloat16)
    sv = torch.zeros_like(sk)
    spare = int(ov.pt[B_O, 0])
    sloc = torch.full((B_O,), spare, dtype=torch.int32, device=dev)
    cap = sb.Batch(False, [sb.Req(B_O, 0, 1) for _ in range(B_O)],
                   torch.zeros(B_O, dtype=torch.int32, device=dev), sloc)
    be.prepare_for_capture(cap)
    side = torch.cuda.Stream()
    side.wait_stream(engine)
    with torch.cuda.stream(side):
        be.forward(sq, sk, sv, 0, cap)
    engine.wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        so = be.forward(sq, sk, sv, 0, cap)
    torch.cuda.synchronize()
    outs = [torch.empty_like(so) for _ in range(STEPS)]
    nxt = prepare(STEPS)
    for i in range(STEPS):
        n = STEPS + i
        b, loc, ev = nxt
        nxt = None
        engine.wait_event(ev)
        _record(b, engine)
        busy = _busy(busy)
        be.prepare_for_replay(b)
        sq.copy_(ov.q[n])
        sk.copy_(ov.k[n])
        sv.copy_(ov.v[n])
        sloc.copy_(b.out_loc)
        graph.replay()
        outs[i].copy_(so)
        results.append((n, loc, outs[i]))
        del b
        if i + 1 < STEPS:
            nxt = prepare(n + 1)
    torch.cuda.synchronize()
    for n, loc, o in results:
        assert_attn_close(o.float().cpu().numpy(), ov.expect(n, loc),
                          what=f"overlapped step {n}")
    del graph


# ------------------------------------------------------------------ mixed padding

HQ_M, HKV_M, N_DEC, QO, PREFIX, LMAX = 32, 4, 64, 256, 512, 2048


def test_mixed_step_padded_into_captured_graph(oracle, dev):
    """A 60-decode-row step replayed through a graph captured with 64: four
    dummy requests pad it; every real row matches the oracle; the pool
    changes only at the real tokens' slots and the spare slot."""
    sb = pkg.backend.load()
    rng = np.random.default_rng(130)
    full = wl.make_paged_batch(rng, [LMAX - 1] * (N_DEC + 1), [LMAX] * (N_DEC + 1), page_size=P)
    pt = full.page_table
    spare_row = N_DEC + 1
    spare = int(pt[spare_row, 0])
    cache, g = _pool(sb, dev, full.num_pages, HKV_M, 131)
    be = sb.HipAttnBackend(cache, HQ_M, HKV_M, D)
    be.set_page_table(torch.from_numpy(pt).to(dev))
    be.init_mixed_capture_graph(LMAX, N_DEC, 1, QO)
    dummy = sb.Req(spare_row, 0, 1)

    def make(dec_rows, dec_lens):
        reqs = [sb.Req(int(r), int(n) - 1, int(n)) for r, n in zip(dec_rows, dec_lens)]
        reqs.append(sb.Req(N_DEC, PREFIX, PREFIX + QO))
        return sb.Batch(True, reqs, torch.zeros(1, dtype=torch.int32, device=dev),
                        torch.zeros(1, dtype=torch.int32, device=dev))

    def tokens(batch):
        pos, loc, rows = [], [], []
        for r in batch.padded_reqs:
            p = np.arange(r.cached_len, r.device_len())
            pos.append(p)
            loc.append(pt[r.table_idx, p])
        pos = np.concatenate(pos).astype(np.int32)
        loc = np.concatenate(loc).astype(np.int32)
        batch.positions = torch.from_numpy(pos).to(dev)
        batch.out_loc = torch.from_numpy(loc).to(dev)
        return loc

    # no captured step yet: nothing to pad to
    b0 = make(np.arange(N_DEC), rng.integers(1, LMAX + 1, N_DEC))
    assert not be.pad_mixed_batch(b0, dummy)
    note("mixed padding: capture 64 decode rows + one 256-token chunk")
    cap = make(np.arange(N_DEC), np.full(N_DEC, LMAX))
    loc_cap = tokens(cap)
    T_cap = len(loc_cap)
    sq = torch.zeros((T_cap, HQ_M * D), device=dev, dtype=torch.bfloat16)
    sk = torch.zeros((T_cap, HKV_M * D), device=dev, dtype=torch.bfloat16)
    sv = torch.zeros_like(sk)
    sloc = torch.full((T_cap,), spare, dtype=torch.int32, device=dev)
    cap.out_loc = sloc  # the capture step stores into the spare slot only
    be.prepare_for_capture(cap)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        be.forward(sq, sk, sv, 0, cap)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        so = be.forward(sq, sk, sv, 0, cap)
    torch.cuda.synchronize()

    note("mixed padding: a 60-row step through the 64-row graph")
    rows = rng.choice(N_DEC, 60, replace=False)
    lens = rng.integers(1, LMAX + 1, 60)
    lens[0] = LMAX
    b = make(rows, lens)
    assert be.pad_mixed_batch(b, dummy)
    assert b.padded_size() == N_DEC + 1
    assert all(r.table_idx == spare_row for r in b.padded_reqs[61:])
    loc = tokens(b)
    T = len(loc)
    assert T == T_cap
    # more decode rows than any captured step, or another prefill count: no fit
    too_many = make(np.arange(N_DEC), np.full(N_DEC, 5))
    too_many.padded_reqs = too_many.padded_reqs + [sb.Req(0, 3, 4)]
    assert not be.pad_mixed_batch(too_many, dummy)
    two_pre = make(rows[:10], lens[:10])
    two_pre.padded_reqs = two_pre.padded_reqs + [sb.Req(int(rows[11]), 100, 300)]
    assert not be.pad_mixed_batch(two_pre, dummy)

    be.prepare_metadata(b)
    assert b.num_decode_rows() == N_DEC and b.num_prefill_rows() == 1
    be.prepare_for_replay(b)
    before_k = u16(cache.k_cache(0)).copy()
    before_v = u16(cache.v_cache(0)).copy()
    q = torch.randn((T, HQ_M * D), device=dev, generator=g).to(torch.bfloat16)
    k = torch.randn((T, HKV_M * D), device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn((T, HKV_M * D), device=dev, generator=g).to(torch.bfloat16)
    sq.copy_(q)
    sk.copy_(k)
    sv.copy_(v)
    sloc.copy_(b.out_loc)
    graph.replay()
    torch.cuda.synchronize()

    # pool: the real tokens' slots hold their k/v; besides them only the
    # spare slot changed
    real = T - 4
    after_k, after_v = u16(cache.k_cache(0)), u16(cache.v_cache(0))
    kc, vc = before_k.copy(), before_v.copy()
    kc[loc[:real]] = u16(k[:real]).reshape(real, HKV_M, D)
    vc[loc[:real]] = u16(v[:real]).reshape(real, HKV_M, D)
    changed = np.nonzero((after_k != kc).any(axis=(1, 2)) | (after_v != vc).any(axis=(1, 2)))[0]
    assert set(changed.tolist()) <= {spare}, changed[:8]
    assert spare not in set(loc[:real].tolist())

    # every real row against the oracle (the padded batch's own layout)
    qo = np.array([r.device_len() - r.cached_len for r in b.padded_reqs])
    kv = np.array([r.device_len() for r in b.padded_reqs])
    qo_ip = np.concatenate([[0], np.cumsum(qo)]).astype(np.int32)
    kv_ip = np.concatenate([[0], np.cumsum(kv)]).astype(np.int32)
    idx = np.concatenate([pt[r.table_idx, :r.device_len()] for r in b.padded_reqs])
    kc[spare] = after_k[spare]  # whichever dummy's store landed last
    vc[spare] = after_v[spare]
    ref = oracle.prefill(u16(q).reshape(T, HQ_M, D).copy(), kc, vc, idx.astype(np.int32),
                         qo_ip, kv_ip, SCALE).reshape(T, -1)
    assert_attn_close(so[:real].float().cpu().numpy(), ref[:real], what="padded mixed step")
    del graph
