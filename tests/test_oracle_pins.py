"""Pins of the CPU oracle (CPU only).

The reference ships no golden vectors for this path (its attention math is
FlashInfer's, which is not in the tree), so each oracle function is pinned
by something other than its own formula: a library routine (torch CPU,
HF transformers), a closed form, an invariant, or the hand-written
known-answer vectors in tests/golden/. Each check is chosen so that a
plausible slip (wrong sign, swapped half, off-by-one in the causal offset,
wrong head grouping) fails it.
"""
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import wl
from helpers import bf16_f32, bf16_ulp_dist

GOLDEN = Path(__file__).resolve().parent / "golden"


def to_u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def rand_bf16(rng, shape, scale=1.0):
    x = torch.from_numpy(rng.standard_normal(shape).astype(np.float32) * scale)
    return to_u16(x.to(torch.bfloat16))


# ------------------------------------------------------------------ bf16

def test_bf16_rounding_matches_torch_cast(oracle):
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * 10,
        np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40, 3.0e38, 1.0 + 2**-8,
                  1.0 + 3 * 2**-8, 1.0 + 2**-9, 65504.0], np.float32),
    ])
    # halfway cases: low 16 bits exactly 0x8000, both parities of bit 16
    halfway = (np.arange(1000, dtype=np.uint32) << 17 | 0x3F808000).view(np.float32)
    halfway2 = (np.arange(1000, dtype=np.uint32) << 17 | 0x3F818000).view(np.float32)
    x = np.concatenate([x, halfway, halfway2])
    want = to_u16(torch.from_numpy(x).to(torch.bfloat16))
    got = oracle.f32_to_bf16(x)
    np.testing.assert_array_equal(got, want)
    nan = oracle.f32_to_bf16(np.array([np.nan], np.float32))
    assert np.isnan(bf16_f32(nan))[0]


# ------------------------------------------------------------------ store / metadata

def test_store_kv_invariants(oracle):
    rng = np.random.default_rng(2)
    slots, elems, T, stride = 64, 24, 20, 40
    kc = rng.integers(0, 65535, (slots, elems), dtype=np.uint16)
    vc = rng.integers(0, 65535, (slots, elems), dtype=np.uint16)
    k = rng.integers(0, 65535, (T, stride), dtype=np.uint16)
    v = rng.integers(0, 65535, (T, stride), dtype=np.uint16)
    loc = rng.permutation(slots)[:T]
    kc0, vc0 = kc.copy(), vc.copy()
    oracle.store_kv(kc, vc, k, v, loc)
    np.testing.assert_array_equal(kc[loc], k[:, :elems])
    np.testing.assert_array_equal(vc[loc], v[:, :elems])
    rest = np.setdiff1d(np.arange(slots), loc)
    np.testing.assert_array_equal(kc[rest], kc0[rest])
    np.testing.assert_array_equal(vc[rest], vc0[rest])


def test_metadata_golden(oracle):
    g = json.loads((GOLDEN / "metadata_kat.json").read_text())
    for case in g["build_indices"]:
        got = oracle.build_indices(np.array(case["page_table"], np.int32),
                                   np.array(case["table_indices"], np.int32),
                                   np.array(case["kv_indptr"], np.int32))
        np.testing.assert_array_equal(got, np.array(case["expected"], np.int32))
    for case in g["gather_int32_2d"]:
        got = oracle.gather_int32_2d(np.array(case["table"], np.int32), case["req"], case["pos"])
        np.testing.assert_array_equal(got, np.array(case["expected"], np.int32))
    for case in g["write_token_pool"]:
        pool = np.array(case["pool"], np.int32)
        oracle.write_token_pool(pool, case["req"], case["pos"], case["tok"])
        np.testing.assert_array_equal(pool, np.array(case["expected"], np.int32))
    for case in g["pages_to_tokens"]:
        got = oracle.pages_to_tokens(case["page_starts"], case["page_size"])
        np.testing.assert_array_equal(got, np.array(case["expected"], np.int32))


def test_write_page_table_kat(oracle):
    """Hand-derived: page_size 4, allocations (row 2, pages 1..2) then (row 0,
    page 0) take the page starts 8, 20, 4 in that order; an allocation on a
    row past the table and a page past the columns write nothing."""
    table = np.zeros((3, 12), np.int32)
    used = oracle.write_page_table(table, [8, 20, 4, 40, 44],
                                   [[2, 1, 3], [0, 0, 1], [7, 0, 1], [1, 3, 4]], 4)
    want = np.zeros((3, 12), np.int32)
    want[2, 4:8] = [8, 9, 10, 11]
    want[2, 8:12] = [20, 21, 22, 23]
    want[0, 0:4] = [4, 5, 6, 7]
    assert used == 5
    np.testing.assert_array_equal(table, want)
    # fewer page starts than the allocations take: reported as -1
    assert oracle.write_page_table(np.zeros((3, 12), np.int32), [8], [[2, 1, 3]], 4) == -1


def test_write_page_table_is_pages_to_tokens_then_token_pool(oracle):
    """The page-table write equals the reference's two steps composed:
    expand the pages (pages_to_tokens, prefill.cc:103-119), then one
    write_token_pool of (table_idx, page * P + i, token) (prefill.cc:160-186)."""
    rng = np.random.default_rng(5)
    for P in (1, 4, 16):
        rows, cols = 6, 40 * P
        alloc = []
        for _ in range(9):
            first = int(rng.integers(0, 42))
            alloc.append([int(rng.integers(-1, rows + 1)), first, first + int(rng.integers(0, 5))])
        n = sum(b - a for _, a, b in alloc)
        pages = (rng.permutation(1000)[:n] * P).astype(np.int32)
        table = rng.integers(0, 99, (rows, cols)).astype(np.int32)
        want = table.copy()
        toks = oracle.pages_to_tokens(pages, P)
        req, pos = [], []
        for r, a, b in alloc:
            for page in range(a, b):
                req += [r] * P
                pos += [page * P + i for i in range(P)]
        oracle.write_token_pool(want, np.array(req, np.int32), np.array(pos, np.int32), toks)
        assert oracle.write_page_table(table, pages, alloc, P) == n
        np.testing.assert_array_equal(table, want)


def test_build_indices_brute_force(oracle):
    rng = np.random.default_rng(3)
    rows, cols = 9, 40
    pt = rng.integers(0, 1000, (rows, cols), dtype=np.int32)
    B = 12
    ti = rng.integers(-2, rows + 2, B).astype(np.int32)
    lens = rng.integers(0, 50, B)
    ip = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    got = oracle.build_indices(pt, ti, ip)
    want = np.zeros(ip[-1], np.int32)
    for r in range(B):
        if 0 <= ti[r] < rows:
            for p in range(lens[r]):
                want[ip[r] + p] = pt[ti[r], p] if p < cols else 0
    np.testing.assert_array_equal(got, want)


# ------------------------------------------------------------------ RoPE cache

def torch_reference_cos_sin(max_pos, rd, base):
    """The reference constructor's LibTorch statements (src/layers/rotary_embedding.cu:80-93)."""
    inv_freq = 1.0 / torch.pow(base, torch.arange(0, rd, 2, dtype=torch.float32) / float(rd))
    t = torch.arange(max_pos, dtype=torch.float32)
    freqs = torch.einsum("i,j->ij", t, inv_freq)
    return freqs.cos().numpy(), freqs.sin().numpy()


@pytest.mark.parametrize("rd,base,max_pos", [(128, 1e6, 40960), (64, 1e4, 4096), (128, 1e4, 8192)])
def test_cos_sin_cache_matches_torch(oracle, rd, base, max_pos):
    cos, sin = oracle.cos_sin_cache(max_pos, rd, base)
    tc, ts = torch_reference_cos_sin(max_pos, rd, base)
    # Row 0 is exactly (1, 0); elsewhere only last-ulp differences of libm vs
    # torch's vector cos/sin on identical fp32 arguments are allowed.
    assert (cos[0] == 1.0).all() and (sin[0] == 0.0).all()
    assert np.abs(cos - tc).max() <= 4e-6
    assert np.abs(sin - ts).max() <= 4e-6


# ------------------------------------------------------------------ RMSNorm

def test_rmsnorm_matches_torch_rms_norm(oracle):
    rng = np.random.default_rng(4)
    T, qh, kh, d, eps = 7, 16, 8, 128, 1e-6
    q = rand_bf16(rng, (T, qh, d), 3.0)
    k = rand_bf16(rng, (T, kh, d), 0.5)
    qw = to_u16(torch.from_numpy(rng.uniform(0.5, 1.5, d).astype(np.float32)).to(torch.bfloat16))
    kw = to_u16(torch.from_numpy(rng.standard_normal(d).astype(np.float32)).to(torch.bfloat16))
    q2, k2 = q.copy(), k.copy()
    oracle.qk_rmsnorm(q2, k2, qw, kw, eps)
    for x, y, w in ((q, q2, qw), (k, k2, kw)):
        xt = torch.from_numpy(bf16_f32(x))
        ref = torch.nn.functional.rms_norm(xt, (d,), eps=eps) * torch.from_numpy(bf16_f32(w))
        ref16 = to_u16(ref.to(torch.bfloat16))
        assert bf16_ulp_dist(y, ref16).max() <= 1


def test_rmsnorm_fused_equals_separate(oracle):
    # tests/layers/test_normalization.cpp:21-53: q+k in one call == one call each.
    rng = np.random.default_rng(5)
    q = rand_bf16(rng, (7, 16, 128))
    k = rand_bf16(rng, (7, 8, 128))
    qw, kw = rand_bf16(rng, (128,)), rand_bf16(rng, (128,))
    qa, ka, qb, kb = q.copy(), k.copy(), q.copy(), k.copy()
    oracle.qk_rmsnorm(qa, ka, qw, kw, 1e-6)
    oracle.qk_rmsnorm(qb, None, qw, None, 1e-6)
    oracle.qk_rmsnorm(kb, None, kw, None, 1e-6)
    np.testing.assert_array_equal(qa, qb)
    np.testing.assert_array_equal(ka, kb)


def test_rmsnorm_constant_row(oracle):
    # x = c everywhere: mean(x^2) = c^2, so out = bf16(c / sqrt(c^2 + eps) * w) ~ sign(c) w.
    d = 64
    q = np.full((1, 1, d), to_u16(torch.tensor([2.5], dtype=torch.bfloat16))[0], np.uint16)
    w = to_u16(torch.linspace(0.5, 1.5, d).to(torch.bfloat16))
    oracle.qk_rmsnorm(q, None, w, None, 1e-6)
    assert bf16_ulp_dist(q[0, 0], w).max() <= 1


def test_f16_encoding_matches_numpy(oracle):
    """The oracle's binary16 encode/decode against numpy's float16 casts:
    normals, subnormals, ties, overflow to infinity, signed zeros."""
    rng = np.random.default_rng(40)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-8, 5, 20000),
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e6, -1e6, 6.1e-5, 5.96e-8, 2.98e-8,
                  1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, np.inf, -np.inf], np.float32)])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(oracle.f32_to_f16_bits(x), want)
    back = oracle.f16_bits_to_f32(want)
    np.testing.assert_array_equal(back, want.view(np.float16).astype(np.float32))


def rand_f16(rng, shape, scale=1.0):
    return (rng.standard_normal(shape).astype(np.float32) * scale).astype(np.float16).view(np.uint16)


def f16_f32(b):
    return b.view(np.float16).astype(np.float32)


def test_rmsnorm_fp16_matches_torch_rms_norm(oracle):
    """fp16 rows (the reference's fp16 dispatch, normalization.cu:346-365)
    against torch's rms_norm in fp32 rounded once to fp16."""
    rng = np.random.default_rng(41)
    T, qh, kh, d, eps = 7, 16, 8, 128, 1e-6
    q = rand_f16(rng, (T, qh, d), 3.0)
    k = rand_f16(rng, (T, kh, d), 0.5)
    qw = rng.uniform(0.5, 1.5, d).astype(np.float16).view(np.uint16)
    kw = rng.standard_normal(d).astype(np.float16).view(np.uint16)
    q2, k2 = q.copy(), k.copy()
    oracle.qk_rmsnorm(q2, k2, qw, kw, eps, dtype="fp16")
    for x, y, w in ((q, q2, qw), (k, k2, kw)):
        xt = torch.from_numpy(f16_f32(x))
        ref = torch.nn.functional.rms_norm(xt, (d,), eps=eps) * torch.from_numpy(f16_f32(w))
        assert bf16_ulp_dist(y, to_u16(ref.to(torch.float16))).max() <= 1


def test_rmsnorm_fp16_fused_equals_separate(oracle):
    # tests/layers/test_normalization.cpp:21-53 at its own dtype (fp16) and
    # shape: q+k in one call == one call each, bit for bit.
    rng = np.random.default_rng(42)
    q = rand_f16(rng, (7, 16, 128))
    k = rand_f16(rng, (7, 8, 128))
    qw, kw = rand_f16(rng, (128,)), rand_f16(rng, (128,))
    qa, ka, qb, kb = q.copy(), k.copy(), q.copy(), k.copy()
    oracle.qk_rmsnorm(qa, ka, qw, kw, 1e-6, dtype="fp16")
    oracle.qk_rmsnorm(qb, None, qw, None, 1e-6, dtype="fp16")
    oracle.qk_rmsnorm(kb, None, kw, None, 1e-6, dtype="fp16")
    np.testing.assert_array_equal(qa, qb)
    np.testing.assert_array_equal(ka, kb)


# ------------------------------------------------------------------ RoPE

def test_rope_fp16_matches_transformers_neox(oracle):
    """fp16 rows (rotary_embedding.cu:124-146 dispatches fp16 too) against HF
    transformers' apply_rotary_pos_emb in fp32, rounded once to fp16."""
    from transformers.models.qwen3.modeling_qwen3 import apply_rotary_pos_emb
    rng = np.random.default_rng(43)
    T, qh, kh, d = 33, 4, 2, 128
    q = rand_f16(rng, (T, qh, d))
    k = rand_f16(rng, (T, kh, d))
    pos = rng.integers(0, 40960, T).astype(np.int32)
    cos, sin = oracle.cos_sin_cache(40960, d, 1e6)
    q2, k2 = q.copy(), k.copy()
    oracle.rope(q2, k2, cos, sin, pos, dtype="fp16")
    cf = torch.from_numpy(np.concatenate([cos[pos], cos[pos]], -1))
    sf = torch.from_numpy(np.concatenate([sin[pos], sin[pos]], -1))
    qt, kt = torch.from_numpy(f16_f32(q)), torch.from_numpy(f16_f32(k))
    qr, kr = apply_rotary_pos_emb(qt, kt, cf, sf, unsqueeze_dim=1)
    assert bf16_ulp_dist(q2, to_u16(qr.to(torch.float16))).max() <= 1
    assert bf16_ulp_dist(k2, to_u16(kr.to(torch.float16))).max() <= 1
    # position 0 is the identity
    z = q[:1].copy()
    oracle.rope(z, z.copy(), cos, sin, np.zeros(1, np.int32), dtype="fp16")
    np.testing.assert_array_equal(z, q[:1])


def test_rope_matches_transformers_neox(oracle):
    """HF transformers' Qwen3 apply_rotary_pos_emb (rotate_half, full-width
    cos/sin = cat(freqs, freqs)) on the same bf16 inputs."""
    from transformers.models.qwen3.modeling_qwen3 import apply_rotary_pos_emb
    rng = np.random.default_rng(6)
    T, qh, kh, d = 33, 4, 2, 128
    q = rand_bf16(rng, (T, qh, d))
    k = rand_bf16(rng, (T, kh, d))
    pos = rng.integers(0, 40960, T).astype(np.int32)
    cos, sin = oracle.cos_sin_cache(40960, d, 1e6)
    q2, k2 = q.copy(), k.copy()
    oracle.rope(q2, k2, cos, sin, pos)
    cf = torch.from_numpy(np.concatenate([cos[pos], cos[pos]], -1))
    sf = torch.from_numpy(np.concatenate([sin[pos], sin[pos]], -1))
    qt, kt = torch.from_numpy(bf16_f32(q)), torch.from_numpy(bf16_f32(k))
    qr, kr = apply_rotary_pos_emb(qt, kt, cf, sf, unsqueeze_dim=1)
    assert bf16_ulp_dist(q2, to_u16(qr.to(torch.bfloat16))).max() <= 1
    assert bf16_ulp_dist(k2, to_u16(kr.to(torch.bfloat16))).max() <= 1


def test_rope_float64_rotation_and_identities(oracle):
    rng = np.random.default_rng(7)
    T, d, base = 50, 128, 1e6
    x = rand_bf16(rng, (T, 1, d))
    pos = np.concatenate([[0], rng.integers(1, 8192, T - 1)]).astype(np.int32)
    cos, sin = oracle.cos_sin_cache(8192, d, base)
    y, kdummy = x.copy(), x.copy()
    oracle.rope(y, kdummy, cos, sin, pos)
    # position 0 is the identity, bit for bit
    np.testing.assert_array_equal(y[0], x[0])
    # float64 rotation of each (i, i + d/2) pair by pos * base^(-2i/d)
    xf = bf16_f32(x)[:, 0].astype(np.float64)
    h = d // 2
    theta = pos[:, None].astype(np.float64) * base ** (-np.arange(h) * 2.0 / d)[None, :]
    a, b = xf[:, :h], xf[:, h:]
    ref = np.concatenate([a * np.cos(theta) - b * np.sin(theta),
                          b * np.cos(theta) + a * np.sin(theta)], 1)
    got = bf16_f32(y)[:, 0].astype(np.float64)
    # bf16 output rounding plus fp32 phase error at positions up to 8192
    assert np.abs(got - ref).max() <= 2e-2 * np.abs(xf).max()
    # each rotated pair keeps its length
    r0 = np.hypot(a, b)
    r1 = np.hypot(got[:, :h], got[:, h:])
    assert np.abs(r1 - r0).max() <= 1e-2 * (1 + r0.max())


def test_rope_relative_position_invariance(oracle):
    # <R(m) q, R(n) k> depends only on m - n.
    rng = np.random.default_rng(8)
    d = 128
    cos, sin = oracle.cos_sin_cache(4096, d, 1e4)
    q = rand_bf16(rng, (2, 1, d))
    q[1] = q[0]
    k = rand_bf16(rng, (2, 1, d))
    k[1] = k[0]
    oracle.rope(q, k, cos, sin, np.array([100, 1100], np.int32))
    qf, kf = bf16_f32(q)[:, 0], bf16_f32(k)[:, 0]
    # q at 100 vs k at 100 and q at 1100 vs k at 1100: same relative offset 0
    dot0 = float(qf[0] @ kf[0])
    dot1 = float(qf[1] @ kf[1])
    assert abs(dot0 - dot1) <= 0.05 * (1 + abs(dot0))


def test_rope_half_and_full_width_cache_agree(oracle):
    rng = np.random.default_rng(10)
    d = 64
    cos, sin = oracle.cos_sin_cache(512, d, 1e4)
    cos_full = np.concatenate([cos, cos], 1)
    sin_full = np.concatenate([sin, sin], 1)
    x = rand_bf16(rng, (9, 2, d))
    kx = rand_bf16(rng, (9, 1, d))
    pos = rng.integers(0, 512, 9).astype(np.int32)
    a, ka = x.copy(), kx.copy()
    b, kb = x.copy(), kx.copy()
    oracle.rope(a, ka, cos, sin, pos)
    oracle.rope(b, kb, np.ascontiguousarray(cos_full), np.ascontiguousarray(sin_full), pos)
    np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(ka, kb)


# ------------------------------------------------------------------ attention

def sdpa_reference(qf, kf, vf, mask, scale):
    """torch SDPA in fp32; qf [Hq, Lq, D], kf/vf [Hq, Lk, D] (already head-expanded)."""
    return torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(qf)[None], torch.from_numpy(kf)[None], torch.from_numpy(vf)[None],
        attn_mask=None if mask is None else torch.from_numpy(mask)[None, None],
        scale=scale)[0].numpy()


def make_pool(rng, slots, hkv, d):
    return rand_bf16(rng, (slots, hkv, d)), rand_bf16(rng, (slots, hkv, d))


@pytest.mark.parametrize("hq,hkv", [(16, 8), (32, 4), (8, 8), (32, 8)])
def test_decode_matches_torch_sdpa(oracle, hq, hkv):
    rng = np.random.default_rng(11)
    d, slots = 128, 700
    kc, vc = make_pool(rng, slots, hkv, d)
    lens = [1, 37, 300, 129]
    ip = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    idx = rng.permutation(slots)[:ip[-1]].astype(np.int32)
    q = rand_bf16(rng, (len(lens), hq, d))
    scale = 1 / math.sqrt(d)
    out = oracle.decode(q, kc, vc, idx, ip, scale)
    G = hq // hkv
    for r, n in enumerate(lens):
        sl = idx[ip[r]:ip[r + 1]]
        kf = np.repeat(bf16_f32(kc[sl]).transpose(1, 0, 2), G, 0)
        vf = np.repeat(bf16_f32(vc[sl]).transpose(1, 0, 2), G, 0)
        qf = bf16_f32(q[r])[:, None, :]
        ref = sdpa_reference(qf, kf, vf, None, scale)[:, 0]
        np.testing.assert_allclose(out[r], ref, atol=2e-5, rtol=1e-4)


def test_decode_special_cases(oracle):
    rng = np.random.default_rng(12)
    d, hkv, hq = 128, 2, 4
    kc, vc = make_pool(rng, 64, hkv, d)
    q = rand_bf16(rng, (2, hq, d))
    # kv_len 1: output is that token's V exactly
    out = oracle.decode(q, kc, vc, np.array([5, 9], np.int32), np.array([0, 1, 2], np.int32), 0.1)
    for r, s in enumerate([5, 9]):
        for h in range(hq):
            np.testing.assert_allclose(out[r, h], bf16_f32(vc[s, h // 2]), rtol=1e-6, atol=1e-7)
    # identical K rows: softmax is uniform, output is the mean of V
    kc2 = kc.copy()
    kc2[10:30] = kc2[10]
    out = oracle.decode(q[:1], kc2, vc, np.arange(10, 30, dtype=np.int32),
                        np.array([0, 20], np.int32), 0.2)
    mean_v = bf16_f32(vc[10:30]).mean(0)
    for h in range(hq):
        np.testing.assert_allclose(out[0, h], mean_v[h // 2], atol=1e-5)


def bottom_right_mask(qo, kv):
    i = np.arange(qo)[:, None]
    j = np.arange(kv)[None, :]
    return j <= i + (kv - qo)


@pytest.mark.parametrize("hq,hkv", [(16, 8), (32, 4)])
def test_prefill_matches_torch_sdpa(oracle, hq, hkv):
    rng = np.random.default_rng(13)
    d, slots = 128, 1200
    kc, vc = make_pool(rng, slots, hkv, d)
    qo = [1, 17, 64, 100]
    kv = [1, 50, 64, 300]  # prefix 0, 33, 0, 200
    qip = np.concatenate([[0], np.cumsum(qo)]).astype(np.int32)
    kip = np.concatenate([[0], np.cumsum(kv)]).astype(np.int32)
    idx = rng.permutation(slots)[:kip[-1]].astype(np.int32)
    q = rand_bf16(rng, (qip[-1], hq, d))
    scale = 1 / math.sqrt(d)
    out = oracle.prefill(q, kc, vc, idx, qip, kip, scale)
    G = hq // hkv
    for r in range(len(qo)):
        sl = idx[kip[r]:kip[r + 1]]
        kf = np.repeat(bf16_f32(kc[sl]).transpose(1, 0, 2), G, 0)
        vf = np.repeat(bf16_f32(vc[sl]).transpose(1, 0, 2), G, 0)
        qf = bf16_f32(q[qip[r]:qip[r + 1]]).transpose(1, 0, 2)
        ref = sdpa_reference(qf, kf, vf, bottom_right_mask(qo[r], kv[r]), scale)
        np.testing.assert_allclose(out[qip[r]:qip[r + 1]], ref.transpose(1, 0, 2), atol=2e-5,
                                   rtol=1e-4)
        if qo[r] == kv[r]:  # no prefix: textbook causal attention
            ref2 = torch.nn.functional.scaled_dot_product_attention(
                torch.from_numpy(qf)[None], torch.from_numpy(kf)[None],
                torch.from_numpy(vf)[None], is_causal=True, scale=scale)[0].numpy()
            np.testing.assert_allclose(out[qip[r]:qip[r + 1]], ref2.transpose(1, 0, 2),
                                       atol=2e-5, rtol=1e-4)


def test_prefill_attention_golden(oracle):
    """Hand-computed 1-head case: pins the bottom-right causal alignment."""
    g = json.loads((GOLDEN / "attention_kat.json").read_text())
    for case in g["cases"]:
        d = case["head_dim"]
        kc = oracle.f32_to_bf16(np.array(case["k"], np.float32).reshape(-1, 1, d))
        vc = oracle.f32_to_bf16(np.array(case["v"], np.float32).reshape(-1, 1, d))
        q = oracle.f32_to_bf16(np.array(case["q"], np.float32).reshape(-1, 1, d))
        out = oracle.prefill(q, kc, vc, np.array(case["indices"], np.int32),
                             np.array(case["qo_indptr"], np.int32),
                             np.array(case["kv_indptr"], np.int32), case["sm_scale"])
        np.testing.assert_allclose(out.reshape(-1, d), np.array(case["expected"], np.float32),
                                   atol=1e-6, rtol=1e-6)


def test_attention_page_permutation_invariance(oracle):
    rng = np.random.default_rng(14)
    d, hkv, hq, slots = 128, 2, 4, 256
    kc, vc = make_pool(rng, slots, hkv, d)
    idx = rng.permutation(slots)[:150].astype(np.int32)
    q = rand_bf16(rng, (1, hq, d))
    ip = np.array([0, 150], np.int32)
    a = oracle.decode(q, kc, vc, idx, ip, 0.09)
    perm = rng.permutation(slots)
    kc2, vc2 = np.empty_like(kc), np.empty_like(vc)
    kc2[perm], vc2[perm] = kc, vc
    b = oracle.decode(q, kc2, vc2, perm[idx].astype(np.int32), ip, 0.09)
    np.testing.assert_array_equal(a, b)


# ------------------------------------------------------------------ residual path
# RMSNorm over hidden rows, fused add + RMSNorm, SiLU/GELU-and-mul
# (src/layers/normalization.cu:236-269,386-416; src/layers/activation.cu:8-77).

RES_DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16}
# One ulp of T relative to |v| is at most 2^-7 (bf16, 8-bit significand) or
# 2^-10 (fp16, 11-bit significand).
ULP = {"bf16": 2.0 ** -7, "fp16": 2.0 ** -10}


def rand_t(rng, shape, dtype, scale=1.0):
    x = torch.from_numpy(rng.standard_normal(shape).astype(np.float32) * scale)
    return x.to(RES_DTYPES[dtype]).float().numpy()


# Absolute slack: one fp16 subnormal step (fixed spacing 2^-24 below 2^-14);
# for bf16, far-tail cancellations of 1 + tanh(u) in double (~1e-15).
ATOL_T = {"bf16": 1e-12, "fp16": 2.0 ** -24}


def assert_within_ulp(got, ref, dtype, what, max_ulp=1):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    bound = max_ulp * ULP[dtype] * np.maximum(np.abs(ref), np.abs(got)) + ATOL_T[dtype]
    bad = np.abs(got - ref) > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} beyond {max_ulp} ulp; "
                           f"e.g. got {got[bad][:4]} ref {ref[bad][:4]}")


def test_round_t_matches_library_casts(oracle):
    rng = np.random.default_rng(40)
    v = (rng.standard_normal(200000) * 10.0 ** rng.uniform(-9, 5, 200000)).astype(np.float32)
    h = rng.integers(0, 0x7BFF, 20000).astype(np.uint16).view(np.float16)
    nxt = np.nextafter(h, np.float16(np.inf)).astype(np.float64)
    mid = ((h.astype(np.float64) + nxt) / 2).astype(np.float32)  # exact fp16 ties
    special = np.array([65504, 65519, 65520, 65535, 1e6, -1e6, np.inf, -np.inf, 0.0, -0.0,
                        2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 1e-30], np.float32)
    v = np.concatenate([v, mid, special])
    with np.errstate(over="ignore"):
        want16 = v.astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(oracle.round_t(v, "fp16"), want16)
    want_bf = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(oracle.round_t(v, "bf16"), want_bf)


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_hidden_rmsnorm_matches_torch_rms_norm(oracle, dtype):
    rng = np.random.default_rng(41)
    for rows, d in [(10, 128), (37, 1000), (8, 4096)]:
        x = rand_t(rng, (rows, d), dtype, 3.0)
        w = torch.from_numpy(rng.uniform(0.5, 1.5, d).astype(np.float32)).to(
            RES_DTYPES[dtype]).float().numpy()
        got = oracle.rmsnorm(x, w, 1e-6, dtype)
        ref = torch.nn.functional.rms_norm(torch.from_numpy(x).double(), (d,),
                                           torch.from_numpy(w).double(), 1e-6)
        assert_within_ulp(got, ref.numpy(), dtype, f"rmsnorm {rows}x{d}")
        # a dropped eps or a sum in place of the mean would be far outside one ulp
        assert np.mean(got == oracle.round_t(ref.float().numpy(), dtype)) > 0.98


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_hidden_rmsnorm_invariants(oracle, dtype):
    rng = np.random.default_rng(42)
    x = rand_t(rng, (16, 512), dtype)
    w = rand_t(rng, (512,), dtype)
    base = oracle.rmsnorm(x, w, 0.0, dtype)
    # with eps = 0, power-of-two scalings commute with every rounding step
    np.testing.assert_array_equal(oracle.rmsnorm(4.0 * x, w, 0.0, dtype), base)
    np.testing.assert_array_equal(oracle.rmsnorm(x, 2.0 * w, 0.0, dtype), 2.0 * base)
    # a constant row normalises to sign(c) * w
    c = np.full((3, 512), -3.0, np.float32)
    np.testing.assert_array_equal(oracle.rmsnorm(c, w, 0.0, dtype), np.broadcast_to(-w, c.shape))


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_fused_add_rmsnorm_pins(oracle, dtype):
    rng = np.random.default_rng(43)
    x = rand_t(rng, (24, 2048), dtype)
    r = rand_t(rng, (24, 2048), dtype, 4.0)
    w = rand_t(rng, (2048,), dtype)
    xo, ro = oracle.fused_add_rmsnorm(x, r, w, 1e-6, dtype)
    # residual: one rounding of the fp32 sum (torch's add then cast)
    want_r = (torch.from_numpy(x) + torch.from_numpy(r)).to(RES_DTYPES[dtype]).float().numpy()
    np.testing.assert_array_equal(ro, want_r)
    # the output normalises the unrounded sum
    s = torch.from_numpy(x).double() + torch.from_numpy(r).double()
    ref = torch.nn.functional.rms_norm(s, (2048,), torch.from_numpy(w).double(), 1e-6)
    assert_within_ulp(xo, ref.numpy(), dtype, "fused add rmsnorm")
    # zero residual reduces to the plain norm; the sum is symmetric
    z = np.zeros_like(r)
    xo0, ro0 = oracle.fused_add_rmsnorm(x, z, w, 1e-6, dtype)
    np.testing.assert_array_equal(xo0, oracle.rmsnorm(x, w, 1e-6, dtype))
    np.testing.assert_array_equal(ro0, x)
    xs, rs = oracle.fused_add_rmsnorm(r, x, w, 1e-6, dtype)
    np.testing.assert_array_equal(xs, xo)
    np.testing.assert_array_equal(rs, ro)


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_act_and_mul_matches_torch(oracle, dtype, act):
    rng = np.random.default_rng(44)
    d = 777
    inp = rand_t(rng, (33, 2 * d), dtype, 3.0)
    got = oracle.act_and_mul(inp, act, dtype)
    x = torch.from_numpy(inp[:, :d]).double()
    y = torch.from_numpy(inp[:, d:]).double()
    a = torch.nn.functional.silu(x) if act == "silu" else \
        torch.nn.functional.gelu(x, approximate="tanh")
    ref = (a * y).numpy()
    assert_within_ulp(got, ref, dtype, f"{act}_and_mul")
    assert np.mean(got == oracle.round_t(ref.astype(np.float32), dtype)) > 0.99
    # act(x) - act(-x) = x for both activations (y = 1)
    xs = np.linspace(-8, 8, 257, dtype=np.float32)
    xs = oracle.round_t(xs, dtype)
    ones = np.ones_like(xs)
    pos = oracle.act_and_mul(np.stack([np.concatenate([xs, ones])]), act, dtype)[0]
    neg = oracle.act_and_mul(np.stack([np.concatenate([-xs, ones])]), act, dtype)[0]
    slack = ULP[dtype] * (np.abs(pos) + np.abs(neg)) + 2 * ATOL_T[dtype]
    assert np.all(np.abs(pos - neg - xs) <= slack)
    assert pos[128] == 0.0  # act(0) = 0


# ------------------------------------------------------------------ sampling
# src/engine/sampling.cu:65-194: inverse-CDF draws and rejection rounds.

def dyadic_probs(rng, batch, d, zero_frac=0.2, bits=24):
    """Rows of probabilities k / 2^bits summing to exactly 1: every partial sum
    is exact in fp32, whatever the order."""
    out = np.zeros((batch, d), np.float32)
    total = 1 << bits
    for b in range(batch):
        w = rng.gamma(0.3, size=d) * (rng.random(d) > zero_frac)
        n = np.floor(w / w.sum() * total).astype(np.int64)
        n[np.argmax(n)] += total - n.sum()
        out[b] = (n / total).astype(np.float32)
    return out


def test_sampling_plain_is_inverse_cdf(oracle):
    rng = np.random.default_rng(50)
    p = dyadic_probs(rng, 16, 3001)
    u = rng.random((16,)).astype(np.float32)
    u[0], u[1] = 0.0, np.nextafter(np.float32(1), np.float32(0))
    got, _ = oracle.sample(p, u, "plain")
    for b in range(16):
        cdf = np.cumsum(p[b].astype(np.float64))
        want = int(np.searchsorted(cdf, u[b], side="right"))  # first cdf > u
        assert got[b] == want and p[b, got[b]] > 0


def _filtered_set(p, mode, k, top_p):
    """Indices a filtered draw may accept: fewer than k probabilities above
    (top-k), mass above below top_p (top-p), or both."""
    above_n = np.array([(p > x).sum() for x in p])
    above_m = np.array([p[p > x].astype(np.float64).sum() for x in p])
    ok = p > 0
    if mode in ("top_k", "top_k_top_p"):
        ok &= above_n < k
    if mode in ("top_p", "top_k_top_p"):
        ok &= above_m < top_p
    return ok


@pytest.mark.parametrize("mode", ["top_k", "top_p", "top_k_top_p"])
def test_filtered_sampling_distribution(oracle, mode):
    """Accepted draws are the renormalised filtered distribution (chi-square),
    and every accepted index lies in the filtered set."""
    rng = np.random.default_rng(51)
    d, n = 12, 40000
    base = dyadic_probs(rng, 1, d, zero_frac=0.0, bits=20)[0]
    p = np.tile(base, (n, 1))
    u = rng.random((32, n)).astype(np.float32)
    k, tp = 4, 0.7
    kw = {"top_k": dict(top_k=np.full(n, k, np.float32)), "top_p": dict(top_p_val=tp),
          "top_k_top_p": dict(top_k=np.full(n, k, np.int32), top_p_val=tp)}[mode]
    got, ok = oracle.sample(p, u, mode, **kw)
    assert ok.all()
    allowed = _filtered_set(base, mode, k, tp)
    assert allowed[got].all()
    expect = np.where(allowed, base, 0).astype(np.float64)
    expect /= expect.sum()
    counts = np.bincount(got, minlength=d)
    m = expect > 0
    chi2 = (((counts[m] - n * expect[m]) ** 2) / (n * expect[m])).sum()
    assert chi2 < 40.0, (chi2, counts, expect * n)  # dof <= 11; p(chi2 > 40) < 1e-4


def test_filtered_sampling_edge_cases(oracle):
    rng = np.random.default_rng(52)
    p = dyadic_probs(rng, 3, 257, zero_frac=0.5)
    u = rng.random((32, 3)).astype(np.float32)
    # top-k 1 and a tiny top-p both pick the (unique) largest probability
    for b in range(3):
        p[b, 7] = 0.0
        p[b, 7] = np.float32(1.0) - p[b].astype(np.float64).sum()  # keep the sum 1
    top = p.argmax(1)
    got, ok = oracle.sample(p, u, "top_k", top_k_val=1)
    assert ok.all() and (got == top).all()
    got, ok = oracle.sample(p, u, "top_p", top_p_val=1e-6)
    assert ok.all() and (got == top).all()
    # k = vocab accepts the first draw: equals the plain draw with u[0]
    got, ok = oracle.sample(p, u, "top_k", top_k_val=257)
    plain, _ = oracle.sample(p, u[0], "plain")
    assert ok.all() and (got == plain).all()


def test_torch_cpu_baseline_matches_oracle(oracle):
    """The LibTorch-CPU baseline leg (oracle/torch_cpu.py) computes what the C
    oracle computes: decode and causal prefill with prefix hits, ragged, GQA."""
    import torch
    from oracle import torch_cpu as tc
    rng = np.random.default_rng(11)
    b = wl.make_paged_batch(rng, [0, 30, 200, 5], [40, 100, 260, 5], page_size=16)
    hq, hkv, D = 8, 2, 128
    kc = oracle.f32_to_bf16(rng.standard_normal((b.num_slots, hkv, D), dtype=np.float32))
    vc = oracle.f32_to_bf16(rng.standard_normal((b.num_slots, hkv, D), dtype=np.float32))
    T = int(b.qo_indptr[-1])
    q = oracle.f32_to_bf16(rng.standard_normal((T, hq, D), dtype=np.float32))
    t = lambda a: torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)  # noqa: E731
    scale = 1 / np.sqrt(D)
    idx = torch.from_numpy(b.indices.astype(np.int64))
    got = tc.prefill(t(q), t(kc), t(vc), idx, b.qo_indptr, b.kv_indptr, scale).numpy()
    want = oracle.prefill(q, kc, vc, b.indices, b.qo_indptr, b.kv_indptr, scale)
    np.testing.assert_allclose(got, want, atol=2e-5, rtol=1e-4)
    qd = q[:4].copy()
    got = tc.decode(t(qd), t(kc), t(vc), idx, b.kv_indptr, scale).numpy()
    want = oracle.decode(qd, kc, vc, b.indices, b.kv_indptr, scale)
    np.testing.assert_allclose(got, want, atol=2e-5, rtol=1e-4)


def test_torch_cpu_fused_store_matches_oracle(oracle):
    """The LibTorch-CPU leg of the fused qk-norm + RoPE + store
    (oracle/torch_cpu.py) against the C oracle's norm -> rope -> store: V
    placement bit-exact, q and the stored k within two bf16 ulps (two chained
    roundings) or the norm's rounding carried through the rotation."""
    import torch
    from oracle import torch_cpu as tc
    rng = np.random.default_rng(12)
    T, hq, hkv, D, slots = 37, 8, 2, 128, 64
    qkv = oracle.f32_to_bf16(rng.standard_normal((T, (hq + 2 * hkv) * D), dtype=np.float32))
    qw = oracle.f32_to_bf16(rng.uniform(0.5, 1.5, D).astype(np.float32))
    kw = oracle.f32_to_bf16(rng.uniform(0.5, 1.5, D).astype(np.float32))
    cos, sin = oracle.cos_sin_cache(512, D, 1e6)
    pos = rng.integers(0, 512, T).astype(np.int32)
    loc = rng.permutation(slots)[:T].astype(np.int32)
    kc0 = oracle.f32_to_bf16(rng.standard_normal((slots, hkv * D), dtype=np.float32))
    vc0 = oracle.f32_to_bf16(rng.standard_normal((slots, hkv * D), dtype=np.float32))
    # C oracle
    qh = qkv[:, :hq * D].reshape(T, hq, D).copy()
    kh = qkv[:, hq * D:(hq + hkv) * D].reshape(T, hkv, D).copy()
    vh = qkv[:, (hq + hkv) * D:].reshape(T, hkv * D).copy()
    oracle.qk_rmsnorm(qh, kh, qw, kw, 1e-6)
    oracle.rope(qh, kh, cos, sin, pos)
    kc_ref, vc_ref = kc0.copy(), vc0.copy()
    oracle.store_kv(kc_ref, vc_ref, kh.reshape(T, -1), vh, loc)
    # LibTorch CPU
    t = lambda a: torch.from_numpy(a.copy().view(np.int16)).view(torch.bfloat16)  # noqa: E731
    qkv_t, kc_t, vc_t = t(qkv), t(kc0).view(slots, hkv, D), t(vc0).view(slots, hkv, D)
    tc.fused_qknorm_rope_store(qkv_t, kc_t, vc_t, t(qw), t(kw), torch.from_numpy(cos),
                               torch.from_numpy(sin), torch.from_numpy(pos.astype(np.int64)),
                               torch.from_numpy(loc.astype(np.int64)), hq, hkv, 1e-6)
    u = lambda x: x.contiguous().view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    np.testing.assert_array_equal(u(vc_t).reshape(slots, -1), vc_ref)
    np.testing.assert_array_equal(u(qkv_t)[:, hq * D:], qkv[:, hq * D:])  # k, v of qkv untouched
    f = lambda x: oracle.bf16_to_f32(x).astype(np.float64)  # noqa: E731

    def close(got, want, pre):
        # two chained roundings: <= 2 ulps of the output, or one ulp of the
        # normalised input pair carried through the rotation
        x = np.abs(f(pre))
        tol = np.maximum(2.0 ** -6 * np.abs(f(want)), 2.0 ** -7 * (x + np.roll(x, D // 2, -1)))
        assert np.all(np.abs(f(got) - f(want)) <= tol + 1e-6)

    qn = qkv[:, :hq * D].reshape(T, hq, D).copy()
    kn = qkv[:, hq * D:(hq + hkv) * D].reshape(T, hkv, D).copy()
    oracle.qk_rmsnorm(qn, kn, qw, kw, 1e-6)
    close(u(qkv_t)[:, :hq * D].reshape(T, hq, D), qh, qn)
    close(u(kc_t).reshape(slots, hkv, D)[loc], kc_ref.reshape(slots, hkv, D)[loc], kn)
    untouched = np.setdiff1d(np.arange(slots), loc)
    np.testing.assert_array_equal(u(kc_t).reshape(slots, -1)[untouched], kc0[untouched])


# ---------------------------------------------------------------- sampler softmax

def test_softmax_temperature_matches_torch(oracle):
    """Pins the oracle to the reference's own statements
    (engine.cc:306-308: logits.to(kFloat32) / temperatures, torch::softmax)
    run by LibTorch on the CPU: float32 there, float64 here."""
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((6, 4099)) * 4).astype(np.float32)
    t = np.array([0.3, 0.6, 1.0, 1.2, 2.0, 0.7], np.float32)
    ref = torch.softmax(torch.from_numpy(x) / torch.from_numpy(t).view(-1, 1), -1).double().numpy()
    got = oracle.softmax_temperature(x, t)
    assert np.allclose(got, ref, rtol=2e-6, atol=1e-12)


def test_softmax_temperature_brute_force_and_invariants(oracle):
    """Tiny rows against the formula term by term; rows sum to 1; a
    temperature of 1 is the plain softmax; dividing by a power of two is
    exact, so t = 2 equals t = 1 on halved logits; a dominant logit gives a
    one-hot row."""
    x = np.array([[0.5, -1.25, 3.0, 0.0], [10.0, -80.0, 10.0, 9.5]], np.float32)
    t = np.array([0.7, 1.3], np.float32)
    got = oracle.softmax_temperature(x, t)
    for r in range(2):
        y = [float(np.float32(v) / np.float32(t[r])) for v in x[r]]
        e = [math.exp(v - max(y)) for v in y]
        assert np.allclose(got[r], [v / sum(e) for v in e], rtol=1e-14, atol=0)
    rng = np.random.default_rng(3)
    z = rng.standard_normal((3, 999)).astype(np.float32)
    p1 = oracle.softmax_temperature(z, 1.0)
    assert np.allclose(p1.sum(1), 1.0, rtol=0, atol=1e-12)
    e = np.exp(z.astype(np.float64) - z.max(1, keepdims=True))
    assert np.allclose(p1, e / e.sum(1, keepdims=True), rtol=1e-14, atol=0)
    assert np.array_equal(oracle.softmax_temperature(z, 2.0), oracle.softmax_temperature(z / 2, 1.0))
    hot = oracle.softmax_temperature(np.array([[0.0, 200.0, 1.0]], np.float32), 1.0)
    assert hot[0, 1] == 1.0 and hot[0, 0] < 1e-80
