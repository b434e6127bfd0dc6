"""sgl_paged_decode_noalloc (no workspace argument, the library's own device
scratch) against sgl_paged_decode with a caller workspace: two calls in a
row, the second with a smaller batch, each bitwise equal to the workspace
entry point and within the attention tolerance of the oracle. Runs last (its
file name sorts last) and also alone in a fresh process."""
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
    # 32q/1kv: eight units per CU; 4M tokens need more partial slots than fit
    plan = capi.decode_plan([0, 1 << 22], 16, 1, 128)
    assert plan.workspace_bytes > capi.DECODE_SCRATCH_BYTES
    q = torch.zeros((1, 16, 128), device=dev, dtype=torch.bfloat16)
    kc = torch.zeros((16, 1, 128), device=dev, dtype=torch.bfloat16)
    idx = torch.zeros(16, dtype=torch.int32, device=dev)
    kvp = torch.tensor([0, 16], dtype=torch.int32, device=dev)
    with pytest.raises(capi.SglError) as e:
        capi.paged_decode_noalloc(plan, q, kc, kc, idx, kvp, q.clone())
    assert e.value.status == -3
