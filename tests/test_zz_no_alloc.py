"""sgl_paged_decode_noalloc (no workspace argument, the library's own device
scratch) against sgl_paged_decode with a caller workspace: captured in a
HIP graph as the file's first no-alloc call (so, run alone, the process's
first no-alloc call is inside the capture) and replayed with new lengths;
two eager calls in a row, the second with a smaller batch; the status word
read back from the scratch. Each result is bitwise equal to the workspace
entry point with the same plan and within the attention tolerance of the
oracle. Runs last (its file name sorts last) and also alone in a fresh
process."""
import math
import sys

import numpy as np
import pytest
import torch

from conftest import capi, wl
from helpers import assert_attn_close, u16

pytestmark = pytest.mark.gpu


def note(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _case(oracle, dev, lens, hq, hkv, seed):
    rng = np.random.default_rng(seed)
    b = wl.make_paged_batch(rng, [x - 1 for x in lens], lens, page_size=16, decode=True)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    kc = torch.randn((b.num_slots, hkv, 128), device=dev, generator=g).to(torch.bfloat16)
    vc = torch.randn((b.num_slots, hkv, 128), device=dev, generator=g).to(torch.bfloat16)
    qkv = torch.randn((len(lens), (hq + 2 * hkv) * 128), device=dev, generator=g)
    q = qkv.to(torch.bfloat16)[:, :hq * 128].view(len(lens), hq, 128)
    idx = torch.from_numpy(b.indices).to(dev)
    kvp = torch.from_numpy(b.kv_indptr).to(dev)
    plan = capi.decode_plan(b.kv_indptr, hq, hkv, 128)
    assert plan.workspace_bytes <= capi.DECODE_SCRATCH_BYTES
    o_ws = torch.full((len(lens), hq, 128), float("nan"), device=dev, dtype=torch.bfloat16)
    o_na = torch.full_like(o_ws, float("nan"))
    capi.paged_decode(plan, q, kc, vc, idx, kvp, o_ws, capi.decode_workspace(plan, dev))
    capi.paged_decode_noalloc(plan, q, kc, vc, idx, kvp, o_na)
    torch.cuda.synchronize()
    assert torch.equal(o_ws.view(torch.int16), o_na.view(torch.int16))
    ref = oracle.decode(u16(q).copy(), u16(kc), u16(vc), b.indices, b.kv_indptr,
                        1 / math.sqrt(128))
    assert_attn_close(o_na.float().cpu().numpy(), ref, what=f"noalloc decode {lens[:4]}")
    return plan


def test_noalloc_decode_captured_in_a_graph(oracle, dev):
    """The first no-alloc call of this file happens inside a stream capture
    (the plan, made before it, resolved the scratch address); each replay
    after new lengths and slots are written in place equals the workspace
    entry point on the same plan, bit for bit."""
    note("noalloc decode: first call inside a graph capture, 4 replays")
    B, hq, hkv, D = 24, 32, 8, 128
    cap_len = 3000
    plan = capi.decode_plan(np.arange(B + 1, dtype=np.int32) * cap_len, hq, hkv, D)
    assert plan.workspace_bytes <= capi.DECODE_SCRATCH_BYTES
    slots = B * cap_len + 16
    g = torch.Generator(device=dev)
    g.manual_seed(90)
    kc = torch.randn((slots, hkv, D), device=dev, generator=g).to(torch.bfloat16)
    vc = torch.randn((slots, hkv, D), device=dev, generator=g).to(torch.bfloat16)
    q = torch.empty((B, hq, D), device=dev, dtype=torch.bfloat16)
    idx = torch.zeros(B * cap_len, dtype=torch.int32, device=dev)
    kvp = torch.zeros(B + 1, dtype=torch.int32, device=dev)
    o_g = torch.empty((B, hq, D), device=dev, dtype=torch.bfloat16)
    rng = np.random.default_rng(91)

    def fill(i):
        lens = rng.integers(1, cap_len + 1, B)
        if i == 1:
            lens[:] = 1  # all requests at one token
        if i == 2:
            lens[3] = 0  # an empty request
        ind = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        perm = rng.permutation(slots - 16)[:int(ind[-1])].astype(np.int32)
        kvp.copy_(torch.from_numpy(ind))
        idx[:ind[-1]].copy_(torch.from_numpy(perm))
        q.copy_(torch.randn((B, hq, D), device=dev, generator=g).to(torch.bfloat16))
        return ind, perm

    fill(0)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        capi.paged_decode_noalloc(plan, q, kc, vc, idx, kvp, o_g)
    ws = capi.decode_workspace(plan, dev)
    o_e = torch.empty_like(o_g)
    for i in range(4):
        note(f"noalloc graph replay {i}")
        ind, perm = fill(i)
        o_g.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert capi.decode_status(None) == 0
        capi.paged_decode(plan, q, kc, vc, idx, kvp, o_e, ws)
        torch.cuda.synchronize()
        assert torch.equal(o_g.view(torch.int16), o_e.view(torch.int16)), f"replay {i}"
        ref = oracle.decode(u16(q).copy(), u16(kc), u16(vc), perm, ind, 1 / math.sqrt(D))
        got = o_g.float().cpu().numpy()
        if i == 2:
            assert (got[3] == 0).all()
        assert_attn_close(got, ref, what=f"noalloc graph replay {i}")
    del graph


def test_noalloc_decode_matches_workspace_entry_point(oracle, dev):
    note("noalloc decode: large batch, then a smaller one")
    rng = np.random.default_rng(80)
    big = [int(x) for x in rng.integers(128, 4097, 96)] + [32768]
    p1 = _case(oracle, dev, big, 32, 8, 81)
    assert p1.split_kv
    p2 = _case(oracle, dev, [700, 3, 1500], 16, 8, 82)
    assert p2.num_units < p1.num_units


def test_noalloc_decode_rejects_oversized_plan(dev):
    note("noalloc decode: plan above the scratch size")
    # 16q/1kv: eight units per CU; 4M tokens need more partial slots than fit
    plan = capi.decode_plan([0, 1 << 22], 16, 1, 128)
    assert plan.workspace_bytes > capi.DECODE_SCRATCH_BYTES
    q = torch.zeros((1, 16, 128), device=dev, dtype=torch.bfloat16)
    kc = torch.zeros((16, 1, 128), device=dev, dtype=torch.bfloat16)
    idx = torch.zeros(16, dtype=torch.int32, device=dev)
    kvp = torch.tensor([0, 16], dtype=torch.int32, device=dev)
    with pytest.raises(capi.SglError) as e:
        capi.paged_decode_noalloc(plan, q, kc, kc, idx, kvp, q.clone())
    assert e.value.status == -3


def test_noalloc_decode_status_word(oracle, dev):
    """A batch past the plan's capacity: NaN rows past it and the CAPACITY
    word in the scratch, read with decode_status(None); the next fitting
    call clears it."""
    note("noalloc decode: capacity status read from the scratch")
    rng = np.random.default_rng(22)
    lens = [100, 40, 500, 30]
    b = wl.make_paged_batch(rng, [x - 1 for x in lens], lens, page_size=16, decode=True)
    plan = capi.decode_plan(np.array([0, 100, 200, 300, 400], np.int32), 16, 8, 128)
    cap = plan.max_total_tokens
    assert b.kv_indptr[2] <= cap < b.kv_indptr[3]
    g = torch.Generator(device=dev)
    g.manual_seed(23)
    kc = torch.randn((b.num_slots, 8, 128), device=dev, generator=g).to(torch.bfloat16)
    vc = torch.randn((b.num_slots, 8, 128), device=dev, generator=g).to(torch.bfloat16)
    q = torch.randn((4, 16, 128), device=dev, generator=g).to(torch.bfloat16)
    o = torch.zeros((4, 16, 128), device=dev, dtype=torch.bfloat16)
    idx = torch.from_numpy(b.indices).to(dev)
    capi.paged_decode_noalloc(plan, q, kc, vc, idx, torch.from_numpy(b.kv_indptr).to(dev), o)
    assert capi.decode_status(None) == -3
    got = o.float().cpu().numpy()
    for r in range(4):
        assert np.isnan(got[r]).all() == bool(b.kv_indptr[r + 1] > cap), f"request {r}"
    fit = np.array([0, 100, 200, 300, 400], np.int32)
    capi.paged_decode_noalloc(plan, q, kc, vc, idx, torch.from_numpy(fit).to(dev), o)
    assert capi.decode_status(None) == 0
    ref = oracle.decode(u16(q).copy(), u16(kc), u16(vc), b.indices, fit, 1 / math.sqrt(128))
    assert_attn_close(o.float().cpu().numpy(), ref, what="fitting batch after overflow")
