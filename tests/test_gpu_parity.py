"""GPU parity of the HIP hot path against the CPU oracle (marked gpu).

Every call goes through the C ABI (libsgl_attn.so via capi). Bars:
bit-exact for KV placement, page indexing and token-pool plumbing;
<= 1 bf16 ulp for RMSNorm / RoPE (fp32 math with one rounding per
reference rounding point, reduction order differs); attention outputs
within 2e-2 abs + 1e-2 rel of the fp32-softmax oracle.
"""
import math
import sys

import numpy as np
import pytest
import torch

from conftest import capi, wl
from helpers import (assert_attn_close, assert_bf16_close, bf16_f32, bf16_ulp_dist,
                     forced_plan, from_u16, u16)

pytestmark = pytest.mark.gpu


def note(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def randn_bf16(shape, dev, gen, scale=1.0):
    return (torch.randn(shape, device=dev, generator=gen) * scale).to(torch.bfloat16)


def gen(dev, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return g


# ------------------------------------------------------------------ KV store

@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("T,hq,hkv,d", [(1, 16, 8, 128), (257, 16, 8, 128), (64, 32, 4, 128),
                                        (33, 2, 1, 12), (0, 16, 8, 128)])
def test_store_kv_bit_exact(oracle, dev, idx_dtype, T, hq, hkv, d):
    note(f"store_kv T={T} hq={hq} hkv={hkv} d={d} idx={idx_dtype}")
    g = gen(dev, 1)
    slots = max(2 * T, 8)
    qkv = randn_bf16((T, (hq + 2 * hkv) * d), dev, g)
    k = qkv[:, hq * d:(hq + hkv) * d]
    v = qkv[:, (hq + hkv) * d:]
    kc = randn_bf16((slots, hkv, d), dev, g)
    vc = randn_bf16((slots, hkv, d), dev, g)
    loc = torch.randperm(slots, device=dev, generator=g)[:T].to(idx_dtype)
    kc_ref, vc_ref = u16(kc).reshape(slots, -1), u16(vc).reshape(slots, -1)
    qkv_h = u16(qkv)
    oracle.store_kv(kc_ref, vc_ref, qkv_h[:, hq * d:], qkv_h[:, (hq + hkv) * d:],
                    loc.cpu().numpy())
    capi.store_kv(kc, vc, k, v, loc)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(u16(kc).reshape(slots, -1), kc_ref)
    np.testing.assert_array_equal(u16(vc).reshape(slots, -1), vc_ref)


# ------------------------------------------------------------------ metadata

def test_build_indices_bit_exact(oracle, dev):
    note("build_decode_indices / build_prefill_indices")
    rng = np.random.default_rng(2)
    rows, cols = 40, 600
    pt = rng.integers(0, 1 << 20, (rows, cols)).astype(np.int32)
    B = 37
    ti = rng.integers(-1, rows + 1, B).astype(np.int32)
    lens = rng.integers(0, 700, B)
    ip = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    want = oracle.build_indices(pt, ti, ip)
    for fn in (capi.build_decode_indices, capi.build_prefill_indices):
        out = torch.zeros(int(ip[-1]), dtype=torch.int32, device=dev)
        fn(torch.from_numpy(pt).to(dev), torch.from_numpy(ti).to(dev),
           torch.from_numpy(ip).to(dev), out)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy(), want)


def test_workload_indices_on_gpu_match_generator(dev):
    note("cfg4 decode indices from the page table")
    w = wl.cfg4_decode_large(seed=3)
    b = w.batch
    out = torch.zeros(len(b.indices), dtype=torch.int32, device=dev)
    capi.build_decode_indices(torch.from_numpy(b.page_table).to(dev),
                              torch.from_numpy(b.table_idx).to(dev),
                              torch.from_numpy(b.kv_indptr).to(dev), out)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), b.indices)


def test_token_pool_bit_exact(oracle, dev):
    note("write_token_pool / gather_int32_2d")
    rng = np.random.default_rng(4)
    rows, cols, n = 17, 300, 5000
    pool = rng.integers(0, 99, (rows, cols)).astype(np.int32)
    req = rng.integers(-1, rows + 1, n).astype(np.int32)
    pos = rng.integers(-2, cols + 2, n).astype(np.int32)
    # unique (req, pos) targets so the scatter order cannot matter
    key = req.astype(np.int64) * 1000 + pos
    _, first = np.unique(key, return_index=True)
    req, pos = req[first], pos[first]
    tok = rng.integers(0, 1 << 30, len(req)).astype(np.int32)
    want = pool.copy()
    oracle.write_token_pool(want, req, pos, tok)
    d_pool = torch.from_numpy(pool).to(dev)
    capi.write_token_pool(d_pool, torch.from_numpy(req).to(dev), torch.from_numpy(pos).to(dev),
                          torch.from_numpy(tok).to(dev))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(d_pool.cpu().numpy(), want)
    got = capi.gather_int32_2d(d_pool, torch.from_numpy(req).to(dev),
                               torch.from_numpy(pos).to(dev))
    np.testing.assert_array_equal(got.cpu().numpy(), oracle.gather_int32_2d(want, req, pos))


@pytest.mark.parametrize("P", [1, 16])
def test_write_page_table_bit_exact(oracle, dev, P):
    """Device page-table write vs the oracle: a scheduler step's worth of
    allocations (prefix-hit requests taking their new pages, a 2048-page
    chunk, decode requests crossing into a new page) plus allocations on
    rows or columns outside the table, which write nothing."""
    note(f"write_page_table P={P}")
    rng = np.random.default_rng(6 + P)
    rows, cols = 40, 2100 * P
    alloc = [[0, 0, 2048], [5, 3, 4], [7, 0, 1], [rows + 2, 0, 3], [9, 2099, 2103], [-1, 0, 2]]
    for r in range(10, 38):
        first = int(rng.integers(0, 100))
        alloc.append([r, first, first + int(rng.integers(0, 40))])
    n = sum(b - a for _, a, b in alloc)
    pages = (rng.permutation(200000)[:n] * P).astype(np.int32)
    table = rng.integers(0, 1 << 20, (rows, cols)).astype(np.int32)
    want = table.copy()
    assert oracle.write_page_table(want, pages, alloc, P) == n
    d = torch.from_numpy(table).to(dev)
    capi.write_page_table(d, torch.from_numpy(pages).to(dev),
                          torch.tensor(alloc, dtype=torch.int32, device=dev), P)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(d.cpu().numpy(), want)


def test_write_page_table_then_decode_indices(dev):
    """Pages written on the device give the same decode indices as the
    workload generator's host-expanded page table (the scheduler's path)."""
    note("write_page_table -> build_decode_indices")
    rng = np.random.default_rng(9)
    lens = [1, 16, 17, 500, 4096]
    b = wl.make_paged_batch(rng, [x - 1 for x in lens], lens, page_size=16, decode=True)
    pt = b.page_table
    alloc, pages = [], []
    for r, n in enumerate(lens):
        npg = -(-n // 16)
        alloc.append([r, 0, npg])
        pages += [int(pt[r, 16 * i]) for i in range(npg)]
    d = torch.zeros(pt.shape, dtype=torch.int32, device=dev)
    capi.write_page_table(d, torch.tensor(pages, dtype=torch.int32, device=dev),
                          torch.tensor(alloc, dtype=torch.int32, device=dev), 16)
    out = torch.empty(int(b.kv_indptr[-1]), dtype=torch.int32, device=dev)
    capi.build_decode_indices(d, torch.from_numpy(b.table_idx).to(dev),
                              torch.from_numpy(b.kv_indptr).to(dev), out)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), b.indices)


def test_copy_i32_batched(dev):
    """sgl_copy_i32: several int32 copies of mixed lengths and alignments in
    one launch, bit-exact; elements past each count untouched."""
    note("copy_i32")
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    lens = [1, 5, 0, 4096 + 3, 700_001, 64, 17, 2]
    src = [torch.randint(-2**31, 2**31 - 1, (n + 8,), device=dev, generator=g,
                         dtype=torch.int32) for n in lens]
    dst = [torch.full((n + 8,), -7, device=dev, dtype=torch.int32) for n in lens]
    # an unaligned source and destination (offset by one element)
    pairs = [(s[1:] if i == 3 else s, d[1:] if i == 4 else d, n)
             for i, (s, d, n) in enumerate(zip(src, dst, lens))]
    capi.copy_i32(pairs)
    torch.cuda.synchronize()
    for i, (s_, d_, n) in enumerate(pairs):
        assert torch.equal(d_[:n], s_[:n]), i
        assert (d_[n:] == -7).all(), i


# ------------------------------------------------------------------ RoPE / norm

def test_cos_sin_cache(oracle, dev):
    note("rope cos/sin cache 40960 x 64")
    cos, sin = capi.rope_cos_sin_cache(40960, 128, 1e6, dev)
    rc, rs = oracle.cos_sin_cache(40960, 128, 1e6)
    torch.cuda.synchronize()
    assert np.abs(cos.cpu().numpy() - rc).max() <= 2e-6
    assert np.abs(sin.cpu().numpy() - rs).max() <= 2e-6


TORCH_DT = {"bf16": torch.bfloat16, "fp16": torch.float16}


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("d", [64, 128, 256, 96])
def test_qk_rmsnorm(oracle, dev, d, dtype):
    note(f"qk_rmsnorm d={d} {dtype}")
    g = gen(dev, 5)
    T, hq, hkv = 37, 16, 8
    dt = TORCH_DT[dtype]
    qkv = (torch.randn((T, (hq + 2 * hkv) * d), device=dev, generator=g) * 2.0).to(dt)
    q = qkv[:, :hq * d].view(T, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].view(T, hkv, d)
    qw = (torch.rand(d, device=dev, generator=g) + 0.5).to(dt)
    kw = torch.randn(d, device=dev, generator=g).to(dt)
    qh, kh = u16(q).copy(), u16(k).copy()
    oracle.qk_rmsnorm(qh, kh, u16(qw), u16(kw), 1e-6, dtype=dtype)
    capi.qk_rmsnorm(q, k, qw, kw, 1e-6)
    torch.cuda.synchronize()
    assert bf16_ulp_dist(u16(q), qh).max() <= 1
    assert bf16_ulp_dist(u16(k), kh).max() <= 1


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_qk_rmsnorm_fused_equals_separate(dev, dtype):
    # tests/layers/test_normalization.cpp:21-53 (fp16, T 7, 16q/8kv, d 128,
    # eps 1e-6, randn weights, allclose 1e-3), here bitwise and in both dtypes.
    note(f"qk_rmsnorm fused vs separate {dtype}")
    g = gen(dev, 6)
    dt = TORCH_DT[dtype]
    q = torch.randn((7, 16, 128), device=dev, generator=g).to(dt)
    k = torch.randn((7, 8, 128), device=dev, generator=g).to(dt)
    qw = torch.randn(128, device=dev, generator=g).to(dt)
    kw = torch.randn(128, device=dev, generator=g).to(dt)
    qa, ka, qb, kb = q.clone(), k.clone(), q.clone(), k.clone()
    capi.qk_rmsnorm(qa, ka, qw, kw, 1e-6)
    capi.qk_rmsnorm(qb, None, qw, None, 1e-6)
    capi.qk_rmsnorm(kb, None, kw, None, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(qa.view(torch.int16), qb.view(torch.int16))
    assert torch.equal(ka.view(torch.int16), kb.view(torch.int16))


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("d,rd,full", [(128, 128, False), (64, 64, False), (128, 64, False),
                                       (80, 80, True), (128, 128, True)])
def test_rope(oracle, dev, d, rd, full, dtype):
    note(f"rope d={d} rotary={rd} full_width_cache={full} {dtype}")
    g = gen(dev, 7)
    T, hq, hkv = 45, 8, 2
    qkv = torch.randn((T, (hq + 2 * hkv) * d), device=dev, generator=g).to(TORCH_DT[dtype])
    q = qkv[:, :hq * d].view(T, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].view(T, hkv, d)
    pos = torch.randint(0, 4096, (T,), device=dev, generator=g, dtype=torch.int32)
    cos, sin = capi.rope_cos_sin_cache(4096, rd, 1e4, dev)
    if full:
        cos, sin = torch.cat([cos, cos], 1).contiguous(), torch.cat([sin, sin], 1).contiguous()
    qh, kh = u16(q).copy(), u16(k).copy()
    oracle.rope(qh, kh, cos.cpu().numpy(), sin.cpu().numpy(), pos.cpu().numpy(), rd, dtype=dtype)
    capi.rope(pos, q, k, cos, sin, rd)
    torch.cuda.synchronize()
    assert_bf16_close(u16(q), qh, what="rope q", dtype=dtype)
    assert_bf16_close(u16(k), kh, what="rope k", dtype=dtype)


def _fused_inputs(dev, T, hq, hkv, d, seed, slots=None):
    g = gen(dev, seed)
    slots = slots or T
    qkv = randn_bf16((T, (hq + 2 * hkv) * d), dev, g)
    kc = randn_bf16((slots, hkv, d), dev, g)
    vc = randn_bf16((slots, hkv, d), dev, g)
    qw = (torch.rand(d, device=dev, generator=g) + 0.5).to(torch.bfloat16)
    kw = (torch.rand(d, device=dev, generator=g) + 0.5).to(torch.bfloat16)
    pos = torch.randint(0, 8192, (T,), device=dev, generator=g, dtype=torch.int32)
    loc = torch.randperm(slots, device=dev, generator=g)[:T].to(torch.int32)
    cos, sin = capi.rope_cos_sin_cache(8192, d, 1e6, dev)
    return qkv, kc, vc, qw, kw, pos, loc, cos, sin


@pytest.mark.parametrize("k_back", [True, False])
@pytest.mark.parametrize("T,hq,hkv,d", [(8192, 16, 8, 128), (100, 32, 4, 128), (77, 8, 2, 64),
                                      (1, 16, 8, 128), (2, 64, 4, 128)])
def test_fused_qknorm_rope_store(oracle, dev, T, hq, hkv, d, k_back):
    note(f"fused qknorm+rope+store T={T} hq={hq} hkv={hkv} d={d} k_back={k_back}")
    qkv, kc, vc, qw, kw, pos, loc, cos, sin = _fused_inputs(dev, T, hq, hkv, d, 8)
    # separate GPU kernels in the reference order: norm -> rope -> store
    qkv2, kc2, vc2 = qkv.clone(), kc.clone(), vc.clone()
    q2 = qkv2[:, :hq * d].view(T, hq, d)
    k2 = qkv2[:, hq * d:(hq + hkv) * d].view(T, hkv, d)
    v2 = qkv2[:, (hq + hkv) * d:].view(T, hkv, d)
    capi.qk_rmsnorm(q2, k2, qw, kw, 1e-6)
    capi.rope(pos, q2, k2, cos, sin)
    capi.store_kv(kc2, vc2, k2, v2, loc)
    # oracle on host copies
    h = u16(qkv).copy()
    qh = h[:, :hq * d].reshape(T, hq, d).copy()
    kh = h[:, hq * d:(hq + hkv) * d].reshape(T, hkv, d).copy()
    vh = h[:, (hq + hkv) * d:].reshape(T, hkv * d).copy()
    oracle.qk_rmsnorm(qh, kh, u16(qw), u16(kw), 1e-6)
    # The norm's bf16 output may sit one ulp from the oracle's; RoPE then
    # carries that input difference into x cos - y sin with |cos|, |sin| <= 1,
    # i.e. up to ulp(x) + ulp(y) <= 2^-7 (|x| + |y|) absolute, which under
    # cancellation spans several ulps of the (small) output.
    def carried(xh):
        x = np.abs(bf16_f32(xh).astype(np.float64))
        return 2.0 ** -7 * (x + np.roll(x, d // 2, axis=-1)) + 1e-6
    q_tol, k_tol = carried(qh), carried(kh).reshape(T, -1)
    oracle.rope(qh, kh, cos.cpu().numpy(), sin.cpu().numpy(), pos.cpu().numpy())
    kc_ref, vc_ref = u16(kc).reshape(T, -1).copy(), u16(vc).reshape(T, -1).copy()
    oracle.store_kv(kc_ref, vc_ref, kh.reshape(T, -1), vh, loc.cpu().numpy())
    # fused
    qkv_in = qkv.clone()
    capi.fused_qknorm_rope_store(qkv, kc, vc, qw, kw, cos, sin, pos, loc, hq, hkv, d, 1e-6,
                                 write_k_back=k_back)
    torch.cuda.synchronize()
    # fused == separate GPU kernels, bit for bit
    if k_back:
        assert torch.equal(qkv.view(torch.int16), qkv2.view(torch.int16))
    else:  # q like the separate kernels, k and v parts of qkv untouched
        assert torch.equal(qkv[:, :hq * d].view(torch.int16), qkv2[:, :hq * d].view(torch.int16))
        assert torch.equal(qkv[:, hq * d:].view(torch.int16), qkv_in[:, hq * d:].view(torch.int16))
    assert torch.equal(kc.view(torch.int16), kc2.view(torch.int16))
    assert torch.equal(vc.view(torch.int16), vc2.view(torch.int16))
    # vs oracle: within 2 ulps (two chained roundings, norm then RoPE), or
    # within the norm's rounding carried through the rotation (above);
    # exact placement (V is a pure copy)
    assert_bf16_close(u16(qkv)[:, :hq * d].reshape(T, hq, d), qh, what="fused q", max_ulp=2,
                      atol=q_tol)
    kc_tol = np.full(kc_ref.shape, 1e-6)
    kc_tol[loc.cpu().numpy()] = k_tol
    assert_bf16_close(u16(kc).reshape(T, -1), kc_ref, what="fused k cache", max_ulp=2,
                      atol=kc_tol)
    np.testing.assert_array_equal(u16(vc).reshape(T, -1), vc_ref)


# ------------------------------------------------------------------ decode

def _pool(dev, slots, hkv, d, seed):
    g = gen(dev, seed)
    return randn_bf16((slots, hkv, d), dev, g), randn_bf16((slots, hkv, d), dev, g)


def run_decode(dev, batch, hq, hkv, d, seed, q_indptr=None, rows=None, plan=None):
    kc, vc = _pool(dev, batch.num_slots, hkv, d, seed)
    g = gen(dev, seed + 100)
    B = batch.batch_size
    rows = B if rows is None else rows
    # q as a strided view of a qkv activation, like AttentionLayer hands it over
    qkv = randn_bf16((rows, (hq + 2 * hkv) * d), dev, g)
    q = qkv[:, :hq * d].view(rows, hq, d)
    o = torch.full((rows, hq, d), float("nan"), device=dev, dtype=torch.bfloat16)
    plan = plan or capi.decode_plan(batch.kv_indptr, hq, hkv, d)
    ws = capi.decode_workspace(plan, dev)
    idx = torch.from_numpy(batch.indices).to(dev)
    kvp = torch.from_numpy(batch.kv_indptr).to(dev)
    qip = None if q_indptr is None else torch.from_numpy(q_indptr).to(dev)
    scale = 1 / math.sqrt(d)
    capi.paged_decode(plan, q, kc, vc, idx, kvp, o, ws, scale, qip)
    torch.cuda.synchronize()
    return q, kc, vc, o, scale, plan


@pytest.mark.parametrize("hq,hkv", [(16, 8), (32, 8), (32, 4), (8, 8), (64, 4),
                                     (40, 8), (16, 16), (8, 1), (14, 2)])
@pytest.mark.parametrize("lens", [[512] * 4, [1, 2, 31, 32, 33, 127, 128, 129],
                                  [4096, 1, 700, 3000, 257]])
def test_decode_parity(oracle, dev, hq, hkv, lens):
    note(f"decode hq={hq} hkv={hkv} lens={lens}")
    rng = np.random.default_rng(9)
    b = wl.make_paged_batch(rng, [x - 1 for x in lens], lens, page_size=16, decode=True)
    q, kc, vc, o, scale, plan = run_decode(dev, b, hq, hkv, 128, 10)
    ref = oracle.decode(u16(q).copy(), u16(kc), u16(vc), b.indices, b.kv_indptr, scale)
    assert_attn_close(o.float().cpu().numpy(), ref, what=f"decode split={plan.split_kv}")


def test_decode_cfg1(oracle, dev):
    w = wl.cfg1_decode_small()
    note(w.name)
    s = w.shape
    q, kc, vc, o, scale, _ = run_decode(dev, w.batch, s.num_qo_heads, s.num_kv_heads,
                                        s.head_dim, 11)
    ref = oracle.decode(u16(q).copy(), u16(kc), u16(vc), w.batch.indices, w.batch.kv_indptr,
                        scale)
    assert_attn_close(o.float().cpu().numpy(), ref, what=w.name)
    assert_attn_close(o.float().cpu().numpy(), ref, what=w.name)


def test_decode_forced_split_and_q_indptr(oracle, dev):
    note("decode with small forced chunk and q rows via q_indptr")
    rng = np.random.default_rng(12)
    lens = [1000, 64, 1]
    b = wl.make_paged_batch(rng, [x - 1 for x in lens], lens, page_size=1, decode=True)
    # 128-token units: ceil(1065 / 128) = 9 units; the 1000-token request
    # spans 9 of them.
    plan = forced_plan(capi, b.kv_indptr, 16, 8, 128)
    assert plan.num_units == 9
    qip = np.array([4, 0, 2], np.int32)
    q, kc, vc, o, scale, _ = run_decode(dev, b, 16, 8, 128, 13, q_indptr=qip, rows=5, plan=plan)
    ref = oracle.decode(u16(q).copy(), u16(kc), u16(vc), b.indices, b.kv_indptr, scale,
                        q_indptr=qip)
    got = o.float().cpu().numpy()
    assert_attn_close(got[qip], ref[qip], what="split decode")
    # rows not addressed by q_indptr stay untouched
    assert torch.isnan(o[[1, 3]].float()).all()


def test_decode_cfg4_full_size(oracle, dev):
    """Full config 4 (B=256, kv up to 4096): every request against the oracle."""
    w = wl.cfg4_decode_large(seed=0)
    note(w.name)
    s = w.shape
    b = w.batch
    q, kc, vc, o, scale, plan = run_decode(dev, b, s.num_qo_heads, s.num_kv_heads, s.head_dim,
                                           14)
    assert plan.split_kv
    ref = oracle.decode(u16(q).copy(), u16(kc), u16(vc), b.indices, b.kv_indptr, scale)
    assert_attn_close(o.float().cpu().numpy(), ref, what=w.name)


@pytest.mark.parametrize("hq,hkv", [(32, 4), (32, 8)])
def test_decode_long_context(oracle, dev, hq, hkv):
    """Config 5's decode lengths: requests of 8K, 16K and 32K tokens beside
    short ones, so a 32K request spans dozens of units and the merge folds
    that many pieces."""
    note(f"decode long context hq={hq} hkv={hkv}")
    rng = np.random.default_rng(18)
    lens = [32768, 16384, 8192, 1, 1024, 32768, 77, 20000]
    b = wl.make_paged_batch(rng, [x - 1 for x in lens], lens, page_size=16, decode=True)
    q, kc, vc, o, scale, plan = run_decode(dev, b, hq, hkv, 128, 19)
    assert plan.split_kv
    W = plan.kv_chunk_size
    assert -(-32768 // W) >= 16, "a 32K request must span many units"
    ref = oracle.decode(u16(q).copy(), u16(kc), u16(vc), b.indices, b.kv_indptr, scale)
    assert_attn_close(o.float().cpu().numpy(), ref, what=f"long decode W={W}")


def test_decode_large_batch(oracle, dev):
    """700 requests (past the 512 kv_indptr entries a wave keeps in registers:
    the unit's first request comes from a binary search over memory)."""
    note("decode batch 700")
    rng = np.random.default_rng(25)
    lens = [int(x) for x in rng.integers(0, 300, 700)]
    b = wl.make_paged_batch(rng, [max(x - 1, 0) for x in lens], lens, page_size=16,
                            decode=True)
    q, kc, vc, o, scale, plan = run_decode(dev, b, 32, 8, 128, 26)
    ref = oracle.decode(u16(q).copy(), u16(kc), u16(vc), b.indices, b.kv_indptr, scale)
    assert_attn_close(o.float().cpu().numpy(), ref, what="decode batch 700")


def test_decode_many_pieces(oracle, dev):
    """80-token units on 32K and 16K requests: 410 + 205 pieces folded by the merge."""
    note("decode 410-piece merge")
    rng = np.random.default_rng(20)
    lens = [32768, 100, 16384, 64, 65]
    b = wl.make_paged_batch(rng, [x - 1 for x in lens], lens, page_size=16, decode=True)
    plan = forced_plan(capi, b.kv_indptr, 32, 4, 80)
    q, kc, vc, o, scale, _ = run_decode(dev, b, 32, 4, 128, 21, plan=plan)
    ref = oracle.decode(u16(q).copy(), u16(kc), u16(vc), b.indices, b.kv_indptr, scale)
    assert_attn_close(o.float().cpu().numpy(), ref, what="410-piece merge")


@pytest.mark.parametrize("hq,hkv,lens", [
    (16, 8, [512] * 4),                       # config 1's shape
    (32, 4, [10000, 20, 0, 1]),               # a request past the LDS slot stage, empty, one token
    (64, 4, [7, 8, 9, 15, 16, 17, 129]),      # G = 16, pieces shorter than a step
    (8, 1, [3000, 2999]),                     # one kv head
])
def test_decode_small_batch_kernel(oracle, dev, hq, hkv, lens):
    """Small batches (units at the 64-token minimum, batch x kv heads <= CUs)
    run one workgroup per (request, kv head) whose waves fold through LDS."""
    note(f"decode small-batch kernel hq={hq} hkv={hkv} lens={lens}")
    rng = np.random.default_rng(27)
    b = wl.make_paged_batch(rng, [max(x - 1, 0) for x in lens], lens, page_size=16, decode=True)
    q, kc, vc, o, scale, plan = run_decode(dev, b, hq, hkv, 128, 28)
    assert plan.kv_chunk_size == 64 and plan.batch_size * hkv <= 256
    ref = oracle.decode(u16(q).copy(), u16(kc), u16(vc), b.indices, b.kv_indptr, scale)
    assert_attn_close(o.float().cpu().numpy(), ref, what="small-batch decode")


def test_decode_plan_exceeded_reports_capacity(oracle, dev):
    """A plan reused for a longer batch: requests reaching past the plan's
    token capacity come back as NaN rows with the CAPACITY status, the others
    are correct; the next call that fits clears the status."""
    note("decode plan exceeded")
    rng = np.random.default_rng(22)
    lens = [100, 40, 500, 30]
    b = wl.make_paged_batch(rng, [x - 1 for x in lens], lens, page_size=16, decode=True)
    plan = capi.decode_plan(np.array([0, 100, 200, 300, 400], np.int32), 16, 8, 128)
    cap = plan.max_total_tokens
    assert b.kv_indptr[2] <= cap < b.kv_indptr[3]  # requests 2 and 3 reach past it
    assert capi.decode_plan_check(plan, b.kv_indptr) == -3
    kc, vc = _pool(dev, b.num_slots, 8, 128, 23)
    g = gen(dev, 24)
    q = randn_bf16((4, 16, 128), dev, g)
    o = torch.zeros((4, 16, 128), device=dev, dtype=torch.bfloat16)
    ws = capi.decode_workspace(plan, dev)
    idx = torch.from_numpy(b.indices).to(dev)
    kvp = torch.from_numpy(b.kv_indptr).to(dev)
    capi.paged_decode(plan, q, kc, vc, idx, kvp, o, ws)
    assert capi.decode_status(ws) == -3
    scale = 1 / math.sqrt(128)
    ref = oracle.decode(u16(q).copy(), u16(kc), u16(vc), b.indices, b.kv_indptr, scale)
    got = o.float().cpu().numpy()
    for r in range(4):
        if b.kv_indptr[r + 1] > cap:
            assert np.isnan(got[r]).all(), f"request {r} past capacity must be NaN"
        else:
            assert_attn_close(got[r], ref[r], what=f"request {r} within capacity")
    # more requests than the plan serves: refused on the host
    plan3 = capi.decode_plan(np.array([0, 100, 200, 300], np.int32), 16, 8, 128)
    with pytest.raises(capi.SglError):
        capi.paged_decode(plan3, q, kc, vc, idx, kvp, o, capi.decode_workspace(plan3, dev))
    # a fitting batch on the same workspace: status cleared, results correct
    fit = np.array([0, 100, 200, 300, 400], np.int32)
    capi.paged_decode(plan, q, kc, vc, idx, torch.from_numpy(fit).to(dev), o, ws)
    assert capi.decode_status(ws) == 0
    ref = oracle.decode(u16(q).copy(), u16(kc), u16(vc), b.indices, fit, scale)
    assert_attn_close(o.float().cpu().numpy(), ref, what="fitting batch after overflow")


def test_decode_plan_exceeded_more_requests_than_units(oracle, dev):
    """The capacity contract when the batch has more requests than the plan
    has units (the merge then runs one workgroup per unit): a plan for 40
    requests of 10 tokens (7 units of 64) reused for 40 longer requests;
    requests past the capacity are NaN, split requests within it fold
    correctly, the status is CAPACITY, and the next fitting call clears it."""
    note("decode plan exceeded, 40 requests on 7 units")
    rng = np.random.default_rng(41)
    plan = capi.decode_plan(np.arange(0, 401, 10, dtype=np.int32), 16, 8, 128)
    assert plan.num_units + 1 < 40 and plan.kv_chunk_size == 64
    cap = plan.max_total_tokens
    lens = [int(x) for x in rng.integers(5, 36, 40)]
    b = wl.make_paged_batch(rng, [x - 1 for x in lens], lens, page_size=16, decode=True)
    assert b.kv_indptr[-1] > cap
    kc, vc = _pool(dev, b.num_slots, 8, 128, 42)
    g = gen(dev, 43)
    q = randn_bf16((40, 16, 128), dev, g)
    o = torch.zeros((40, 16, 128), device=dev, dtype=torch.bfloat16)
    ws = capi.decode_workspace(plan, dev)
    idx = torch.from_numpy(b.indices).to(dev)
    kvp = torch.from_numpy(b.kv_indptr).to(dev)
    capi.paged_decode(plan, q, kc, vc, idx, kvp, o, ws)
    assert capi.decode_status(ws) == -3
    scale = 1 / math.sqrt(128)
    ref = oracle.decode(u16(q).copy(), u16(kc), u16(vc), b.indices, b.kv_indptr, scale)
    got = o.float().cpu().numpy()
    split = 0
    for r in range(40):
        rb, re = int(b.kv_indptr[r]), int(b.kv_indptr[r + 1])
        if re > cap:
            assert np.isnan(got[r]).all(), f"request {r} past capacity must be NaN"
        else:
            split += (re - 1) // 64 != rb // 64
            assert_attn_close(got[r], ref[r], what=f"request {r} within capacity")
    assert split > 0
    fit = np.concatenate([[0], np.cumsum([min(x, 10) for x in lens])]).astype(np.int32)
    capi.paged_decode(plan, q, kc, vc, idx, torch.from_numpy(fit).to(dev), o, ws)
    assert capi.decode_status(ws) == 0
    ref = oracle.decode(u16(q).copy(), u16(kc), u16(vc), b.indices, fit, scale)
    assert_attn_close(o.float().cpu().numpy(), ref, what="fitting batch after overflow")


def test_decode_page_permutation_invariance(dev):
    """Moving every KV row to another slot (and the table with it) leaves o bitwise unchanged."""
    note("decode page-permutation invariance")
    rng = np.random.default_rng(16)
    lens = [2000, 37, 555]
    b = wl.make_paged_batch(rng, [x - 1 for x in lens], lens, page_size=16, decode=True)
    q, kc, vc, o, scale, plan = run_decode(dev, b, 32, 8, 128, 17)
    perm = torch.randperm(kc.shape[0], device=dev)
    kc2, vc2 = torch.empty_like(kc), torch.empty_like(vc)
    kc2[perm], vc2[perm] = kc, vc
    idx2 = perm[torch.from_numpy(b.indices).to(dev).long()].to(torch.int32)
    o2 = torch.empty_like(o)
    ws = capi.decode_workspace(plan, dev)
    capi.paged_decode(plan, q, kc2, vc2, idx2, torch.from_numpy(b.kv_indptr).to(dev), o2, ws,
                      scale)
    torch.cuda.synchronize()
    assert torch.equal(o.view(torch.int16), o2.view(torch.int16))


# ------------------------------------------------------------------ prefill

def run_prefill(dev, batch, hq, hkv, d, seed):
    kc, vc = _pool(dev, batch.num_slots, hkv, d, seed)
    g = gen(dev, seed + 100)
    rows = int(batch.qo_indptr[-1])
    qkv = randn_bf16((rows, (hq + 2 * hkv) * d), dev, g)
    q = qkv[:, :hq * d].view(rows, hq, d)
    o = torch.full((rows, hq, d), float("nan"), device=dev, dtype=torch.bfloat16)
    scale = 1 / math.sqrt(d)
    capi.paged_prefill(q, kc, vc, torch.from_numpy(batch.indices).to(dev),
                       torch.from_numpy(batch.qo_indptr).to(dev),
                       torch.from_numpy(batch.kv_indptr).to(dev), int(batch.qo_lens.max()), o,
                       scale)
    torch.cuda.synchronize()
    return q, kc, vc, o, scale


def check_prefill(oracle, dev, batch, hq, hkv, seed, what):
    q, kc, vc, o, scale = run_prefill(dev, batch, hq, hkv, 128, seed)
    ref = oracle.prefill(u16(q).copy(), u16(kc), u16(vc), batch.indices, batch.qo_indptr,
                         batch.kv_indptr, scale)
    assert_attn_close(o.float().cpu().numpy(), ref, what=what)


def test_prefill_cfg2(oracle, dev):
    w = wl.cfg2_prefill_prefix()
    note(w.name)
    check_prefill(oracle, dev, w.batch, w.shape.num_qo_heads, w.shape.num_kv_heads, 20, w.name)


@pytest.mark.parametrize("hq,hkv", [(16, 8), (32, 4), (8, 8), (32, 8), (12, 4),
                                     (40, 8), (16, 16), (8, 1), (64, 8), (32, 2), (16, 1)])
def test_prefill_ragged(oracle, dev, hq, hkv):
    note(f"prefill ragged hq={hq} hkv={hkv}")
    rng = np.random.default_rng(21)
    cached = [0, 0, 5, 100, 63, 64, 1000, 17]
    dev_lens = [1, 70, 6, 300, 64, 200, 1001, 129]
    b = wl.make_paged_batch(rng, cached, dev_lens, page_size=16)
    check_prefill(oracle, dev, b, hq, hkv, 22, f"prefill ragged {hq}/{hkv}")


@pytest.mark.parametrize("hq,hkv,qo_last", [(16, 8, 100), (32, 4, 32)])
def test_prefill_split_kv_short_shares(oracle, dev, hq, hkv, qo_last):
    """Launches that leave CUs idle (at most one 64-row item per CU) split
    each item's kv tiles between two 2-wave groups. Requests of 1, 3, 5, 6
    and 10 kv tiles give the groups 1/0, 2/1, 3/2, 3/3 tiles (every tile's
    gathers in flight at once, the third V tile staged in registers) and 5/5
    (the double-buffered ring); the last request spans several items."""
    note(f"prefill split-kv short shares hq={hq} hkv={hkv}")
    rng = np.random.default_rng(37)
    cached = [0, 100, 250, 352, 600, 40]
    dev_lens = [32, 132, 282, 384, 632, 40 + qo_last]
    b = wl.make_paged_batch(rng, cached, dev_lens, page_size=16)
    check_prefill(oracle, dev, b, hq, hkv, 38, f"split-kv short shares {hq}/{hkv}")


def test_prefill_chunked_extend_and_empty_extend(oracle, dev):
    """Chunked prefill: a second chunk on its first chunk's cache; extend 0 -> qo 1."""
    note("prefill chunked extend / zero extend")
    rng = np.random.default_rng(23)
    b = wl.make_paged_batch(rng, [512, 300, 40], [1024, 300, 41], page_size=1)
    assert list(b.qo_lens) == [512, 1, 1]
    check_prefill(oracle, dev, b, 32, 4, 24, "chunked extend")


def test_prefill_long_no_prefix_matches_textbook(oracle, dev):
    note("prefill qo == kv (no prefix), 1500 tokens")
    rng = np.random.default_rng(25)
    b = wl.make_paged_batch(rng, [0], [1500], page_size=16)
    check_prefill(oracle, dev, b, 16, 8, 26, "textbook causal")


def _run_mixed(dev, batch, hq, hkv, seed, decode_cus):
    """One sgl_paged_mixed call over a batch: requests with qo == 1 as decode
    rows, the others as prefill rows, sharing q, the pool and o."""
    kc, vc = _pool(dev, batch.num_slots, hkv, 128, seed)
    g = gen(dev, seed + 100)
    rows = int(batch.qo_indptr[-1])
    q = randn_bf16((rows, hq, 128), dev, g)
    o = torch.full((rows, hq, 128), float("nan"), device=dev, dtype=torch.bfloat16)
    qo, kv = batch.qo_lens, batch.kv_lens
    dec = [r for r in range(batch.batch_size) if qo[r] == 1]
    pre = [r for r in range(batch.batch_size) if qo[r] > 1]
    seg = lambda r: batch.indices[batch.kv_indptr[r]:batch.kv_indptr[r + 1]]  # noqa: E731
    dec_ip = np.concatenate([[0], np.cumsum(kv[dec])]).astype(np.int32)
    pre_qo = np.concatenate([[0], np.cumsum(qo[pre])]).astype(np.int32)
    pre_kv = np.concatenate([[0], np.cumsum(kv[pre])]).astype(np.int32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)  # noqa: E731
    plan = capi.decode_plan_cus(dec_ip, hq, hkv, 128, decode_cus)
    ws = capi.decode_workspace(plan, dev)
    capi.paged_mixed(plan, q, kc, vc, t(np.concatenate([seg(r) for r in dec])), t(dec_ip),
                     t(batch.qo_indptr[dec]), t(np.concatenate([seg(r) for r in pre])), t(pre_qo),
                     t(pre_kv), t(batch.qo_indptr[pre]), int(qo[pre].max()), o, ws)
    torch.cuda.synchronize()
    return q, kc, vc, o, ws


@pytest.mark.parametrize("hq,hkv,decode_cus", [(32, 4, 160), (32, 4, 8), (32, 8, 64), (16, 2, 96),
                                               (8, 1, 200), (32, 4, 256)])
def test_paged_mixed_one_launch(oracle, dev, hq, hkv, decode_cus):
    """sgl_paged_mixed (decode units and prefill items in one launch, decode
    on decode_cus CUs): decode rows with kv 1..6000 beside two prefill chunks
    (one on a cached prefix), rows interleaved by request, all against the
    oracle; the status word stays OK."""
    note(f"paged mixed hq={hq} hkv={hkv} decode_cus={decode_cus}")
    rng = np.random.default_rng(33 + hkv + decode_cus)
    kv_dec = [int(x) for x in rng.integers(1, 6000, 13)]
    cached = [x - 1 for x in kv_dec[:5]] + [300] + [x - 1 for x in kv_dec[5:]] + [0]
    dev_lens = kv_dec[:5] + [300 + 700] + kv_dec[5:] + [200]
    b = wl.make_paged_batch(rng, cached, dev_lens, page_size=16)
    q, kc, vc, o, ws = _run_mixed(dev, b, hq, hkv, 34, decode_cus)
    ref = oracle.prefill(u16(q).copy(), u16(kc), u16(vc), b.indices, b.qo_indptr, b.kv_indptr,
                         1 / math.sqrt(128))
    assert_attn_close(o.float().cpu().numpy(), ref, what=f"mixed {hq}/{hkv} cus {decode_cus}")
    assert capi.decode_status(ws) == 0


@pytest.mark.parametrize("seed", range(4))
def test_paged_mixed_random(oracle, dev, seed):
    """Seeded random mixed batches through sgl_paged_mixed: head layout,
    decode rows (some empty), one to three prefill requests with or without
    a cached prefix, interleaved in random order, and the decode CU share;
    every row against the oracle."""
    rng = np.random.default_rng(500 + seed)
    hkv = int(rng.choice([1, 2, 4, 8]))
    hq = hkv * int(rng.choice([1, 2, 4, 8]))
    n_dec, n_pre = int(rng.integers(1, 24)), int(rng.integers(1, 4))
    kv_dec = [int(x) for x in rng.integers(0, 5000, n_dec)]
    kv_dec[0] = max(kv_dec[0], 1)
    pre_prefix = [int(x) for x in rng.integers(0, 600, n_pre)]
    pre_qo = [int(x) for x in rng.integers(2, 400, n_pre)]
    reqs = [(max(k - 1, 0), k) for k in kv_dec] + [(p, p + q) for p, q in zip(pre_prefix, pre_qo)]
    order = rng.permutation(len(reqs))
    cached = [reqs[i][0] for i in order]
    dev_lens = [reqs[i][1] for i in order]
    cus = int(rng.integers(1, 32)) * 8
    note(f"paged mixed random seed={seed} hq={hq} hkv={hkv} dec={n_dec} pre={n_pre} cus={cus}")
    b = wl.make_paged_batch(rng, cached, dev_lens, page_size=16)
    q, kc, vc, o, ws = _run_mixed(dev, b, hq, hkv, 40 + seed, cus)
    ref = oracle.prefill(u16(q).copy(), u16(kc), u16(vc), b.indices, b.qo_indptr, b.kv_indptr,
                         1 / math.sqrt(128))
    assert_attn_close(o.float().cpu().numpy(), ref, what=f"mixed random seed {seed}")
    assert capi.decode_status(ws) == 0


@pytest.mark.parametrize("hq,hkv", [(8, 1), (16, 2)])
def test_paged_mixed_long_units(oracle, dev, hq, hkv):
    """Long decode rows on few CUs at 1 and 2 kv heads: 8 or 4 units share a
    fused workgroup's LDS, so the plan caps the unit length (at most 4032
    and 8064 tokens, less what the per-wave K tiles take) rather than exceed
    it; results against the oracle."""
    note(f"paged mixed long units hq={hq} hkv={hkv}")
    rng = np.random.default_rng(35 + hkv)
    kv_dec = [int(x) for x in rng.integers(30000, 45000, 7)]
    cached = [x - 1 for x in kv_dec] + [200]
    b = wl.make_paged_batch(rng, cached, kv_dec + [500], page_size=16)
    plan = capi.decode_plan_cus(np.concatenate([[0], np.cumsum(kv_dec)]).astype(np.int32),
                                hq, hkv, 128, 8)
    assert plan.kv_chunk_size <= (4032 if hkv == 1 else 8064)
    q, kc, vc, o, ws = _run_mixed(dev, b, hq, hkv, 36, 8)
    ref = oracle.prefill(u16(q).copy(), u16(kc), u16(vc), b.indices, b.qo_indptr, b.kv_indptr,
                         1 / math.sqrt(128))
    assert_attn_close(o.float().cpu().numpy(), ref, what=f"mixed long units {hq}/{hkv}")
    assert capi.decode_status(ws) == 0


def test_prefill_mixed_decode_rows(oracle, dev):
    """Config-5 shape of batch (qo 1 rows next to a 2048 chunk), scaled down."""
    note("prefill with qo=1 rows beside a long chunk")
    rng = np.random.default_rng(27)
    kv = list(rng.integers(100, 3000, 6)) + [4096 + 512]
    cached = [x - 1 for x in kv[:-1]] + [4096]
    b = wl.make_paged_batch(rng, cached, kv, page_size=16)
    check_prefill(oracle, dev, b, 32, 4, 28, "mixed prefill")


@pytest.mark.parametrize("hq,hkv,B,qo,prefix", [(64, 4, 2, 512, 256), (32, 4, 1, 2048, 128)])
def test_prefill_wide_workgroups(oracle, dev, hq, hkv, B, qo, prefix):
    """Shapes that select the 8-wave (256-row) prefill workgroups: long
    chunks (qo * G >= 8192) that still give every CU a workgroup."""
    note(f"prefill 8-wave path hq={hq} hkv={hkv} B={B} qo={qo} prefix={prefix}")
    rng = np.random.default_rng(29)
    b = wl.make_paged_batch(rng, [prefix] * B, [prefix + qo] * B, page_size=16)
    check_prefill(oracle, dev, b, hq, hkv, 30, "prefill 8-wave")


@pytest.mark.parametrize("hq,hkv,qo,prefix", [
    (32, 4, [1024, 584], [100, 333]),   # paired tiles; the short request has an odd tile count
    (64, 4, [768, 700], [64, 0]),       # 8-wave tiles, more than one workgroup per CU (unpaired)
])
def test_prefill_wide_ragged(oracle, dev, hq, hkv, qo, prefix):
    """Ragged batches on the 8-wave paths: with at most one workgroup per
    CU each workgroup takes a tile from both ends of a request's causal range
    (a shorter request has fewer pairs, and an odd count leaves the middle
    tile's second group empty); otherwise heavy-first single tiles."""
    note(f"prefill 8-wave ragged hq={hq} hkv={hkv} qo={qo} prefix={prefix}")
    rng = np.random.default_rng(31)
    b = wl.make_paged_batch(rng, prefix, [p + q for p, q in zip(prefix, qo)], page_size=16)
    check_prefill(oracle, dev, b, hq, hkv, 32, "prefill 8-wave ragged")



def check_prefill_rows(oracle, batch, q, kc, vc, o, scale, r, toks, what):
    """Sampled query tokens of request r: token i of its chunk sees the kv
    prefix [0, kv - qo + i] (the causal definition), one oracle decode
    over that prefix per token, every head."""
    qo0, kv0 = int(batch.qo_indptr[r]), int(batch.kv_indptr[r])
    qo_len = int(batch.qo_indptr[r + 1]) - qo0
    kv_len = int(batch.kv_indptr[r + 1]) - kv0
    toks = np.asarray(toks)
    vis = kv_len - qo_len + toks + 1
    ip = np.concatenate([[0], np.cumsum(vis)]).astype(np.int32)
    idx = np.concatenate([batch.indices[kv0:kv0 + n] for n in vis]).astype(np.int32)
    ref = oracle.decode(u16(q[qo0 + toks]).copy(), u16(kc), u16(vc), idx, ip, scale)
    assert_attn_close(o[qo0 + toks].float().cpu().numpy(), ref, what=what)


@pytest.mark.parametrize("qo,prefix,page", [
    (2048, 4096, 16),  # configuration 5's chunk
    (2048, 0, 1),      # no prefix: the pairs' light tiles see few kv tiles
    (1040, 300, 16),   # an odd tile count: the middle tile's second group is empty
    (1024, 30000, 16), # a long prefix: pairs of nearly equal tiles
])
def test_prefill_paired_launch_sampled(oracle, dev, qo, prefix, page):
    """The paired launch (32q/4kv, one request, at most one workgroup per
    CU) at full size: sampled tokens of every pair position (every 16-token
    tile's first and last token, every third tile, plus random ones)
    against the oracle, and no row left unwritten."""
    note(f"prefill paired launch qo={qo} prefix={prefix} page={page}")
    rng = np.random.default_rng(qo + prefix)
    b = wl.make_paged_batch(rng, [prefix], [prefix + qo], page_size=page)
    q, kc, vc, o, scale = run_prefill(dev, b, 32, 4, 128, 40)
    assert not torch.isnan(o.float()).any()
    edges = np.unique(np.concatenate([np.arange(0, qo, 16), np.arange(15, qo, 16)]))
    sample = np.unique(np.concatenate([edges[::3], rng.choice(qo, 64, replace=False)]))
    check_prefill_rows(oracle, b, q, kc, vc, o, scale, 0, sample, f"paired {qo}/{prefix}")


@pytest.mark.parametrize("seed", [0, 1, 2, 3, 4, 5])
def test_prefill_random_batches(oracle, dev, seed):
    """Seeded random ragged batches (lengths, prefixes, head groups, page
    sizes) across the 4-wave, 8-wave and paired 8-wave launches; the seed
    picks the shape, so each case names itself."""
    rng = np.random.default_rng(100 + seed)
    hq, hkv = [(32, 4), (32, 8), (32, 4), (64, 4), (64, 8), (32, 4)][seed]
    B = int(rng.integers(1, 4))
    big = seed % 2 == 0  # long chunks reach the 8-wave paths
    qo = rng.integers(256 if big else 1, (2600 if big else 700) // max(1, hq // hkv // 4), B)
    if seed == 2:  # one chunk of 2017..2048 tokens at G = 8: the paired launch
        B, qo = 1, rng.integers(2017, 2049, 1)
    prefix = rng.integers(0, 1500, B)
    page = int(rng.choice([1, 16]))
    note(f"prefill random seed={seed} hq={hq} hkv={hkv} qo={list(qo)} prefix={list(prefix)} "
         f"page={page}")
    b = wl.make_paged_batch(rng, [int(p) for p in prefix], [int(p + q) for p, q in zip(prefix, qo)],
                            page_size=page)
    check_prefill(oracle, dev, b, hq, hkv, 200 + seed, f"prefill random {seed}")


def test_prefill_empty_kv_rows_are_zero(oracle, dev):
    """A request with no visible kv token gets zero rows (as decode writes for
    an empty request); its neighbours are unaffected."""
    note("prefill empty-kv request")
    rng = np.random.default_rng(60)
    b = wl.make_paged_batch(rng, [0, 10], [300, 90], page_size=16)
    hq, hkv = 16, 8
    kc, vc = _pool(dev, b.num_slots, hkv, 128, 61)
    g = gen(dev, 62)
    # request 1 is given 5 query rows and kv_len 0
    qo = np.array([0, 300, 305], np.int32)
    kvp = np.array([0, 300, 300], np.int32)
    q = randn_bf16((305, hq, 128), dev, g)
    o = torch.full((305, hq, 128), float("nan"), device=dev, dtype=torch.bfloat16)
    capi.paged_prefill(q, kc, vc, torch.from_numpy(b.indices).to(dev),
                       torch.from_numpy(qo).to(dev), torch.from_numpy(kvp).to(dev), 300, o)
    torch.cuda.synchronize()
    got = o.float().cpu().numpy()
    assert (got[300:] == 0).all()
    ref = oracle.prefill(u16(q[:300]).copy(), u16(kc), u16(vc), b.indices[:300], qo[:2], kvp[:2],
                         1 / math.sqrt(128))
    assert_attn_close(got[:300], ref, what="neighbour of the empty request")
