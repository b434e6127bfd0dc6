"""A scheduler-shaped serving loop over 16-token pages, every step against the
oracle: the reference's CacheManager::allocate_paged
(src/scheduler/prefill.cc:189-206) hands out pages and writes them into the
page table on the device (write_page_table), the new tokens' slots come from
the device gather of the table (gather_int32_2d, scheduler.cc:332), then
HipAttnBackend runs a prefill step and decode steps -- eagerly, and the
decode steps again through one captured graph replayed with the growing
lengths (GraphRunner, engine.cc:670-743). This is the page_size > 1 path the
reference's Engine refuses (engine.cc:421-422), end to end."""
import math
import sys

import numpy as np
import pytest
import torch

from conftest import capi, pkg
from helpers import assert_attn_close, u16

pytestmark = pytest.mark.gpu

D, P = 128, 16
HQ, HKV = 32, 8
MAX_REQ, MAX_SEQ = 4, 512
SCALE = 1 / math.sqrt(D)


def note(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


class Loop:
    def __init__(self, sb, dev, seed):
        self.sb, self.dev = sb, dev
        self.rng = np.random.default_rng(seed)
        self.num_pages = MAX_REQ * MAX_SEQ // P + 8
        self.cache = sb.MHAKVCache(HKV, 1, D, self.num_pages + 1, P, 0)
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        self.g = g
        self.cache.buffer().copy_(torch.randn(tuple(self.cache.buffer().shape), device=dev,
                                              generator=g).to(torch.bfloat16))
        self.pt = torch.zeros((MAX_REQ + 1, MAX_SEQ), dtype=torch.int32, device=dev)
        self.pt[MAX_REQ].fill_(self.num_pages * P)  # graph dummy row (engine.cc:472)
        self.free = [int(x) * P for x in self.rng.permutation(self.num_pages)]
        self.backend = sb.HipAttnBackend(self.cache, HQ, HKV, D)
        self.backend.set_page_table(self.pt)
        self.kc = u16(self.cache.k_cache(0))  # host mirror of the pool
        self.vc = u16(self.cache.v_cache(0))
        self.pt_host = self.pt.cpu().numpy().copy()

    def allocate(self, cached, device):
        """CacheManager::allocate_paged + write_page_table for requests 0..n-1."""
        info, pages = [], []
        for r, (c, d) in enumerate(zip(cached, device)):
            first, last = -(-c // P), -(-d // P)
            if last > first:
                info.append((r, first, last))
                pages += [self.free.pop(0) for _ in range(last - first)]
        if pages:
            self.sb.write_page_table(self.pt, pages, info, P)
            i = 0
            for r, first, last in info:  # the host mirror, expanded the reference's way
                for page in range(first, last):
                    self.pt_host[r, page * P:(page + 1) * P] = pages[i] + np.arange(P)
                    i += 1

    def step(self, cached, device, is_prefill):
        n = len(cached)
        self.allocate(cached, device)
        req = np.concatenate([np.full(d - c, r) for r, (c, d) in enumerate(zip(cached, device))])
        pos = np.concatenate([np.arange(c, d) for c, d in zip(cached, device)])
        out_loc = capi.gather_int32_2d(self.pt, torch.from_numpy(req.astype(np.int32)).to(self.dev),
                                       torch.from_numpy(pos.astype(np.int32)).to(self.dev))
        T = len(pos)
        q = torch.randn((T, HQ * D), device=self.dev, generator=self.g).to(torch.bfloat16)
        k = torch.randn((T, HKV * D), device=self.dev, generator=self.g).to(torch.bfloat16)
        v = torch.randn((T, HKV * D), device=self.dev, generator=self.g).to(torch.bfloat16)
        reqs = [self.sb.Req(r, int(c), int(d)) for r, (c, d) in enumerate(zip(cached, device))]
        batch = self.sb.Batch(is_prefill, reqs, torch.from_numpy(pos.astype(np.int32)).to(self.dev),
                              out_loc)
        return dict(batch=batch, q=q, k=k, v=v, T=T, loc=self.pt_host[req, pos],
                    cached=list(cached), device=list(device), out_loc=out_loc)

    def expect(self, st):
        """Store the step's k/v in the host mirror, then the oracle's attention."""
        from oracle import oracle
        T = st["T"]
        self.kc[st["loc"]] = u16(st["k"]).reshape(T, HKV, D)
        self.vc[st["loc"]] = u16(st["v"]).reshape(T, HKV, D)
        dev_lens = np.array(st["device"])
        qo = dev_lens - np.array(st["cached"])
        qo_ip = np.concatenate([[0], np.cumsum(qo)]).astype(np.int32)
        kv_ip = np.concatenate([[0], np.cumsum(dev_lens)]).astype(np.int32)
        idx = np.concatenate([self.pt_host[r, :d] for r, d in enumerate(dev_lens)]).astype(np.int32)
        q = u16(st["q"]).reshape(T, HQ, D).copy()
        return oracle.prefill(q, self.kc, self.vc, idx, qo_ip, kv_ip, SCALE).reshape(T, -1)


def test_serving_loop_pages_prefill_decode_and_replay(oracle, dev):
    sb = pkg.backend.load()
    note("serving loop: prefill, then decode steps eager and replayed, 16-token pages")
    lp = Loop(sb, dev, 100)
    prompts = [37, 100, 16, 250]
    st = lp.step([0] * 4, prompts, True)
    np.testing.assert_array_equal(st["out_loc"].cpu().numpy(), st["loc"])  # device gather
    lp.backend.prepare_metadata(st["batch"])
    o = lp.backend.forward(st["q"], st["k"], st["v"], 0, st["batch"])
    torch.cuda.synchronize()
    assert_attn_close(o.float().cpu().numpy(), lp.expect(st), what="prefill step")
    np.testing.assert_array_equal(lp.pt.cpu().numpy(), lp.pt_host)  # device page table

    lens = list(prompts)
    # eager decode steps (pages are allocated as a request crosses a page boundary)
    for i in range(10):
        st = lp.step(lens, [x + 1 for x in lens], False)
        lp.backend.prepare_metadata(st["batch"])
        o = lp.backend.forward(st["q"], st["k"], st["v"], 0, st["batch"])
        torch.cuda.synchronize()
        assert_attn_close(o.float().cpu().numpy(), lp.expect(st), what=f"eager decode {i}")
        lens = [x + 1 for x in lens]
    np.testing.assert_array_equal(lp.pt.cpu().numpy(), lp.pt_host)

    # the same loop through one captured decode graph
    lp.backend.init_capture_graph(MAX_SEQ, [4])
    sq = torch.zeros((4, HQ * D), device=dev, dtype=torch.bfloat16)
    sk = torch.zeros((4, HKV * D), device=dev, dtype=torch.bfloat16)
    sv = torch.zeros_like(sk)
    dummy = lp.num_pages * P
    sloc = torch.full((4,), dummy, dtype=torch.int32, device=dev)
    cap = sb.Batch(False, [sb.Req(r, MAX_SEQ - 1, MAX_SEQ) for r in range(4)],
                   torch.zeros(4, dtype=torch.int32, device=dev), sloc)
    lp.backend.prepare_for_capture(cap)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        lp.backend.forward(sq, sk, sv, 0, cap)  # warm-up: stores zeros at the dummy slot
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        so = lp.backend.forward(sq, sk, sv, 0, cap)
    for i in range(10):
        st = lp.step(lens, [x + 1 for x in lens], False)
        lp.backend.prepare_metadata(st["batch"])
        lp.backend.prepare_for_replay(st["batch"])
        sq.copy_(st["q"])
        sk.copy_(st["k"])
        sv.copy_(st["v"])
        sloc.copy_(st["out_loc"])
        graph.replay()
        torch.cuda.synchronize()
        assert_attn_close(so.float().cpu().numpy(), lp.expect(st), what=f"replayed decode {i}")
        lens = [x + 1 for x in lens]
    # every page handed out is in the table, once
    used = lp.pt_host[:4][np.arange(MAX_SEQ)[None, :] < np.array(lens)[:, None]]
    assert len(np.unique(used)) == sum(lens)
