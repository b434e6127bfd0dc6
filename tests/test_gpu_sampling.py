"""GPU parity of the sampling kernels (marked gpu) against the CPU oracle,
through the C ABI: plain, top-k, top-p and top-k + top-p draws
(src/engine/sampling.cu:65-194) with the reference's call shapes
(uniform [32, batch] for the filtered draws, per-row top_k as float32 for
top-k and int32 for top-k + top-p, engine.cc:300-345).

Bars: on dyadic probabilities (k / 2^24, every partial sum exact in any
order) samples and success flags are bit-exact. On softmax probabilities
over the Qwen3 vocabulary the kernels' fp32 sums differ from the oracle's
exact CDF by their summation error, so a draw may move where u falls that
close to a boundary: every plain draw s must satisfy
cdf(s - 1) <= u + 1e-5 and cdf(s) >= u - 1e-5 on the exact CDF, and every
draw is valid (a positive probability; inside the filtered set when
accepted). A filtered draw may differ from the oracle's only on a row whose
rejection trajectory (replayed in float64) comes within SUM_TOL of a
decision boundary at some round up to its end: the target u * q within
SUM_TOL of a CDF step, or the mass above the pivot within SUM_TOL of top_p.
Every other row must give the oracle's sample and success flag exactly.
SUM_TOL = 2e-5 bounds the kernel's fp32 fixed-order sums of up to 151,936
probabilities of total mass <= 1 (block sums of 512, then a sum over
blocks: well under 1e-5), plus the same error carried into u * q.
"""
import sys

import numpy as np
import pytest
import torch

from conftest import capi
from test_oracle_pins import dyadic_probs

pytestmark = pytest.mark.gpu

QWEN3_VOCAB = 151936
SUM_TOL = 2e-5


def note(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def in_filtered_set(row, s, mode, k, top_p):
    """Whether index s may be accepted: fewer than k probabilities above it
    (top-k), their mass below top_p (top-p), or both."""
    gt = row > row[s]
    ok = row[s] > 0
    if mode in ("top_k", "top_k_top_p"):
        ok &= gt.sum() < k
    if mode in ("top_p", "top_k_top_p"):
        ok &= row[gt].astype(np.float64).sum() < top_p
    return bool(ok)


def trajectory_margin(row, u, mode, k, top_p):
    """Replays the rejection rounds (the oracle's algorithm, float64 sums) for
    one row; returns (sample, accepted, smallest distance to a decision
    boundary over the rounds taken)."""
    d = len(row)
    pivot, q = np.float32(0), np.float32(1)
    margin = np.inf
    sampled, accepted = d - 1, False
    for r in range(u.shape[0]):
        target = np.float64(np.float32(u[r] * q))
        idx = np.nonzero(row > pivot)[0]
        cdf = np.cumsum(row[idx].astype(np.float64))
        j = int(np.searchsorted(cdf, target, side="right"))
        if j < len(idx):
            sampled = int(idx[j])
            margin = min(margin, cdf[j] - target, target - (cdf[j - 1] if j > 0 else 0.0))
        else:
            sampled = d - 1
            margin = min(margin, target - (cdf[-1] if len(cdf) else 0.0))
        if row[sampled] > pivot:
            pivot = row[sampled]
        above = row > pivot
        qd = row[above].astype(np.float64).sum()
        q = np.float32(qd)
        count = int(above.sum())
        if mode in ("top_p", "top_k_top_p"):
            margin = min(margin, abs(qd - top_p))
        if mode == "top_k":
            accepted = count < k
        elif mode == "top_p":
            accepted = q < top_p
        else:
            accepted = count < k and q < top_p
        if accepted:
            break
    return sampled, accepted, margin


def run_all(oracle, dev, p, u, k, tp, exact):
    B = p.shape[0]
    pt = torch.from_numpy(p).to(dev)
    ut = torch.from_numpy(u).to(dev)
    kf = torch.from_numpy(k.astype(np.float32)).to(dev)
    ki = torch.from_numpy(k.astype(np.int32)).to(dev)
    tpt = torch.from_numpy(tp).to(dev)
    cases = {
        "plain": (capi.sampling_from_probs(pt, ut[0].contiguous()),
                  oracle.sample(p, u[0], "plain")),
        "top_k": (capi.top_k_sampling_from_probs(pt, ut, kf),
                  oracle.sample(p, u, "top_k", top_k=k.astype(np.float32))),
        "top_k scalar": (capi.top_k_sampling_from_probs(pt, ut, None, 20),
                         oracle.sample(p, u, "top_k", top_k_val=20)),
        "top_p": (capi.top_p_sampling_from_probs(pt, ut, tpt),
                  oracle.sample(p, u, "top_p", top_p=tp)),
        "top_p scalar": (capi.top_p_sampling_from_probs(pt, ut, None, 0.8),
                         oracle.sample(p, u, "top_p", top_p_val=0.8)),
        "top_k_top_p": (capi.top_k_top_p_sampling_from_probs(pt, ut, ki, 0, tpt, 0.0),
                        oracle.sample(p, u, "top_k_top_p", top_k=k.astype(np.int32), top_p=tp)),
    }
    torch.cuda.synchronize()
    for name, (g, (want, want_ok)) in cases.items():
        got = (g if isinstance(g, torch.Tensor) else g[0]).cpu().numpy()
        got_ok = None if isinstance(g, torch.Tensor) else g[1].cpu().numpy()
        assert ((got >= 0) & (got < p.shape[1])).all(), name
        assert (p[np.arange(B), got] > 0).all(), name
        if exact:
            np.testing.assert_array_equal(got, want, err_msg=name)
            if got_ok is not None:
                np.testing.assert_array_equal(got_ok, want_ok, err_msg=name)
        elif name == "plain":
            for b in range(B):
                cdf = np.cumsum(p[b].astype(np.float64))
                lo = cdf[got[b] - 1] if got[b] > 0 else 0.0
                assert lo <= u[0, b] + 1e-5 and cdf[got[b]] >= u[0, b] - 1e-5, (b, got[b], want[b])
        else:
            mode = name.split(" ")[0]
            near = 0
            for b in range(B):
                kk = 20 if name == "top_k scalar" else int(k[b])
                pp = np.float32(0.8) if name == "top_p scalar" else tp[b]
                s_ref, ok_ref, margin = trajectory_margin(p[b], u[:, b], mode, kk, pp)
                # the float64 replay is the oracle's algorithm
                assert (s_ref, ok_ref) == (int(want[b]), bool(want_ok[b])), (name, b)
                if margin > SUM_TOL:
                    assert (int(got[b]), bool(got_ok[b])) == (s_ref, ok_ref), \
                        (name, b, int(got[b]), s_ref, margin)
                else:
                    near += 1
            assert near <= B // 4, (name, near)  # the bound is not vacuous
        if got_ok is not None and name != "plain":
            mode = name.split(" ")[0]
            for b in np.nonzero(got_ok)[0][:16]:
                kk = 20 if name == "top_k scalar" else k[b]
                pp = 0.8 if name == "top_p scalar" else tp[b]
                assert in_filtered_set(p[b], got[b], mode, kk, pp), (name, b)


@pytest.mark.parametrize("batch,d", [(64, QWEN3_VOCAB), (5, 1001), (3, 4096),
                                     (4, 150001),    # odd length: bounds-checked loads
                                     (2, 1 << 21)])  # longest rows (4,096 blocks, no LDS copies)
def test_sampling_dyadic_bit_exact(oracle, dev, batch, d):
    note(f"sampling dyadic batch={batch} d={d}")
    rng = np.random.default_rng(60 + d % 97)
    p = dyadic_probs(rng, batch, d)
    u = rng.random((32, batch)).astype(np.float32)
    k = rng.integers(1, 50, batch)
    tp = rng.uniform(0.3, 0.95, batch).astype(np.float32)
    run_all(oracle, dev, p, u, k, tp, exact=True)


def test_sampling_softmax_probs(oracle, dev):
    note("sampling from softmax(logits / T), Qwen3 vocabulary")
    g = torch.Generator(device=dev)
    g.manual_seed(61)
    B = 32
    logits = torch.randn((B, QWEN3_VOCAB), device=dev, generator=g) * 4
    temp = torch.linspace(0.5, 1.5, B, device=dev).view(B, 1)
    probs = torch.softmax(logits / temp, -1).contiguous()
    u = torch.rand((32, B), device=dev, generator=g)
    rng = np.random.default_rng(62)
    k = rng.integers(1, 100, B)
    tp = rng.uniform(0.5, 0.95, B).astype(np.float32)
    run_all(oracle, dev, probs.cpu().numpy(), u.cpu().numpy(), k, tp, exact=False)


def test_sampling_rejects_bad_arguments(dev):
    note("sampling argument checks")
    p = torch.full((2, 8), 0.125, device=dev)
    with pytest.raises(ValueError):
        capi.sampling_from_probs(p.double(), torch.rand(2, device=dev))
    with pytest.raises(ValueError):
        capi.top_k_sampling_from_probs(p, torch.rand(2, device=dev), None, 3)  # needs [rounds, B]
    with pytest.raises(ValueError):
        capi.top_k_top_p_sampling_from_probs(p, torch.rand(4, 2, device=dev),
                                             torch.ones(2, device=dev), 0, None, 0.5)
    # rows longer than 2^21 probabilities are not supported
    big = torch.full((1, (1 << 21) + 1), 1.0 / ((1 << 21) + 1), device=dev)
    with pytest.raises(capi.SglError):
        capi.sampling_from_probs(big, torch.rand(1, device=dev))


def test_sampling_candidate_overflow(oracle, dev):
    """Rows whose mass exceeds 1 (k / 2^20, 40,000 entries in [2^-13, 2^-12)
    plus a tail; every partial sum still exact in fp32): the first rejection
    round expects few candidates above the pivot (q = 1 in round 0), finds
    more than LDS holds and falls back to sweeping the row; later rounds may
    switch to the candidates. Bit-exact against the oracle."""
    note("sampling: candidate overflow fallback, unnormalised dyadic rows")
    rng = np.random.default_rng(63)
    B, d = 8, QWEN3_VOCAB
    n = np.zeros((B, d), np.int64)
    for b in range(B):
        pos = rng.permutation(d)
        n[b, pos[:40000]] = rng.integers(128, 256, 40000)
        n[b, pos[40000:60000]] = rng.integers(0, 16, 20000)
    p = (n / float(1 << 20)).astype(np.float32)
    u = rng.random((32, B)).astype(np.float32)
    k = np.full(B, 3)
    tp = np.full(B, 0.5, np.float32)
    pt = torch.from_numpy(p).to(dev)
    ut = torch.from_numpy(u).to(dev)
    got, ok = capi.top_k_sampling_from_probs(pt, ut, torch.from_numpy(k.astype(np.float32)).to(dev))
    torch.cuda.synchronize()
    want, want_ok = oracle.sample(p, u, "top_k", top_k=k.astype(np.float32))
    np.testing.assert_array_equal(got.cpu().numpy(), want)
    np.testing.assert_array_equal(ok.cpu().numpy(), want_ok)


def test_sampling_low_first_pivot(oracle, dev):
    """Normalised dyadic rows with a heavy flat bulk (60,000 probabilities of
    2^-17, below the copy threshold of the first sweep) beside 2,000 larger
    ones: first draws often land in the bulk, so a round sweeps the row
    again with copies held, and later rounds return to the copies.
    Bit-exact against the oracle."""
    note("sampling: first pivot below the copy threshold")
    rng = np.random.default_rng(64)
    B, d = 16, QWEN3_VOCAB
    total = 1 << 24
    p = np.zeros((B, d), np.float32)
    for b in range(B):
        n = np.zeros(d, np.int64)
        pos = rng.permutation(d)
        n[pos[:60000]] = 128
        n[pos[60000:61000]] = 8192
        n[pos[61000:62000]] = rng.integers(600, 1200, 1000)
        n[pos[61000]] += total - n.sum()
        assert n.min() >= 0 and n.sum() == total
        p[b] = (n / total).astype(np.float32)
    u = rng.random((32, B)).astype(np.float32)
    k = rng.integers(1, 50, B)
    tp = rng.uniform(0.3, 0.95, B).astype(np.float32)
    run_all(oracle, dev, p, u, k, tp, exact=True)


# ---------------------------------------------------------------- sampler softmax
#
# sgl_softmax_temperature against the oracle's float64 softmax of
# float32(logits) / t (engine.cc:306-308). Bar (floating point): every
# probability within SOFTMAX_RTOL relative (+ SOFTMAX_ATOL absolute, for
# values below fp32's normal range) of the oracle. The kernel's scaled
# logit carries half an ulp of |y| (6e-8 |y|, logits up to ~50 here), its
# exp2 argument a few ulp of |y - max| and its fp32 row sum below 1e-5.
SOFTMAX_RTOL = 3e-5
SOFTMAX_ATOL = 1e-30


def _softmax_case(oracle, dev, logits, temps=None, temp=1.0, label=""):
    note(f"softmax_temperature {label} shape={tuple(logits.shape)} dtype={logits.dtype}")
    got = capi.softmax_temperature(logits, temps, temp)
    torch.cuda.synchronize()
    x = logits.float().cpu().numpy()
    ref = oracle.softmax_temperature(x, temps.cpu().numpy() if temps is not None else temp)
    g = got.cpu().numpy().astype(np.float64)
    err = np.abs(g - ref)
    ok = err <= SOFTMAX_RTOL * ref + SOFTMAX_ATOL
    rel = float((err / np.maximum(ref, 1e-30))[ref > 1e-30].max())
    note(f"  max relative error {rel:.3e}")
    assert ok.all(), (label, np.argwhere(~ok)[:5], rel)
    return got


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_softmax_temperature_qwen3_vocab(oracle, dev, dtype):
    """The Sampler's shape: per-row temperatures over the Qwen3 vocabulary
    (16-bit rows held in registers, fp32 rows streamed); one row with
    masked (-inf) entries. Also within the same bar of LibTorch's own
    device path, the reference's statements."""
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    B = 6
    logits = (torch.randn((B, QWEN3_VOCAB), device=dev, generator=g) * 3).to(dtype)
    logits[2, ::7] = float("-inf")
    temps = torch.tensor([0.6, 0.8, 1.0, 1.2, 0.35, 1.7], device=dev)
    got = _softmax_case(oracle, dev, logits, temps, label="qwen3")
    torch_path = torch.softmax(logits.to(torch.float32) / temps.view(B, 1), -1)
    assert torch.allclose(got, torch_path, rtol=SOFTMAX_RTOL, atol=SOFTMAX_ATOL)
    assert bool((got[2, ::7] == 0).all())


@pytest.mark.parametrize("mode", ["plain", "top_k", "top_p", "top_k_top_p"])
def test_sampling_from_logits_flat_rows(dev, mode):
    """Nearly flat rows (every probability below the copy threshold): every
    round sweeps the row again, and copies above the pivot overflow."""
    g = torch.Generator(device=dev)
    g.manual_seed(33)
    B = 6
    logits = (torch.randn((B, QWEN3_VOCAB), device=dev, generator=g) * 0.05).to(torch.bfloat16)
    logits[1, :5] = 6.0  # one row with a few dominant entries
    temps = torch.ones(B, device=dev)
    _logits_case(dev, logits, temps, mode, 34, "flat")


@pytest.mark.parametrize("vocab,offset,dtype", [
    (1003, 0, torch.bfloat16),     # partial last chunk
    (8, 0, torch.float16),         # one chunk
    (5000, 1, torch.bfloat16),     # unaligned rows: element by element
    (5001, 1, torch.float32),      # unaligned fp32 rows
    (200000, 0, torch.bfloat16),   # longer than the registers hold: streamed
    (65536, 0, torch.float16),     # register path, fewer chunks per lane
    (163840, 0, torch.bfloat16),   # exactly the 20 chunks a lane holds
    (163848, 0, torch.bfloat16),   # one chunk past them: streamed
    (32768, 0, torch.bfloat16),    # 4 chunks a lane
    (90000, 0, torch.float16),     # 11 chunks a lane, partial last chunk round
    (131080, 0, torch.bfloat16),   # 17 chunks a lane, one lane holding the 17th
])
def test_softmax_temperature_shapes(oracle, dev, vocab, offset, dtype):
    g = torch.Generator(device=dev)
    g.manual_seed(vocab + offset)
    B = 3
    base = (torch.randn((B, vocab + 8), device=dev, generator=g) * 5).to(dtype)
    logits = base[:, offset:offset + vocab]
    _softmax_case(oracle, dev, logits, None, 0.9, label=f"v{vocab}+{offset}")


def test_nonpositive_temperature_rows(dev):
    """A per-row temperature that is not positive gives that row NaN
    probabilities (the other rows are untouched), and the draws from logits
    still equal softmax then draw on every row."""
    note("softmax_temperature and draws with temperatures 0 and -1")
    g = torch.Generator(device=dev)
    g.manual_seed(71)
    B = 4
    logits = (torch.randn((B, QWEN3_VOCAB), device=dev, generator=g) * 3).to(torch.bfloat16)
    temps = torch.tensor([1.0, 0.0, -1.0, 0.7], device=dev)
    probs = capi.softmax_temperature(logits, temps)
    torch.cuda.synchronize()
    assert bool(torch.isnan(probs[1]).all()) and bool(torch.isnan(probs[2]).all())
    ref = torch.softmax(logits[[0, 3]].float() / temps[[0, 3]].view(2, 1), -1)
    assert torch.allclose(probs[[0, 3]], ref, rtol=SOFTMAX_RTOL, atol=SOFTMAX_ATOL)
    for mode in ("plain", "top_k_top_p"):
        _logits_case(dev, logits, temps, mode, 72, "nonpositive-t")


def test_softmax_temperature_rejects_bad_arguments(dev):
    x = torch.zeros((2, 16), device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        capi.softmax_temperature(x, None, 0.0)
    with pytest.raises(ValueError):
        capi.softmax_temperature(x.to(torch.int32), None, 1.0)
    probs = torch.empty((2, 16), device=dev)
    st = capi.lib().sgl_softmax_temperature(capi._p(probs), 16, capi._p(x), 16, 7, None, 1.0, 2, 16,
                                            None)
    assert st == -2  # SGL_ERR_UNSUPPORTED dtype
    st = capi.lib().sgl_softmax_temperature(capi._p(probs), 8, capi._p(x), 16, 0, None, 1.0, 2, 16,
                                            None)
    assert st == -1  # row stride below vocab


# ---------------------------------------------------------------- draws from logits
#
# sgl_sampling_from_logits computes each probability as sgl_softmax_temperature
# writes it (same operations, same row statistics), so its samples and
# success flags must equal those of softmax_temperature followed by the same
# draw from probabilities, bit for bit.

def _draw_from_probs(probs, u, mode, k, tp):
    if mode == "plain":
        return capi.sampling_from_probs(probs, u), None
    if mode == "top_k":
        return capi.top_k_sampling_from_probs(probs, u, k.float())
    if mode == "top_p":
        return capi.top_p_sampling_from_probs(probs, u, tp)
    return capi.top_k_top_p_sampling_from_probs(probs, u, k.int(), 0, tp, 0.0)


def _logits_case(dev, logits, temps, mode, seed, label):
    note(f"sampling_from_logits {label} mode={mode} shape={tuple(logits.shape)} dtype={logits.dtype}")
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    B = logits.shape[0]
    u = torch.rand((B,) if mode == "plain" else (32, B), device=dev, generator=g)
    k = torch.randint(1, 80, (B,), device=dev, generator=g)
    tp = torch.rand(B, device=dev, generator=g) * 0.5 + 0.45
    probs = capi.softmax_temperature(logits, temps)
    s_ref, ok_ref = _draw_from_probs(probs, u, mode, k, tp)
    kk = None if mode in ("plain", "top_p") else (k.float() if mode == "top_k" else k.int())
    s, ok = capi.sampling_from_logits(logits, u, mode, temps, top_k=kk,
                                      top_p=tp if mode in ("top_p", "top_k_top_p") else None)
    torch.cuda.synchronize()
    assert torch.equal(s, s_ref), (label, mode, torch.nonzero(s != s_ref)[:5])
    if ok_ref is not None:
        assert torch.equal(ok, ok_ref), (label, mode)


@pytest.mark.parametrize("mode", ["plain", "top_k", "top_p", "top_k_top_p"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_sampling_from_logits_equals_softmax_then_draw(dev, dtype, mode):
    g = torch.Generator(device=dev)
    g.manual_seed(21)
    B = 12
    logits = (torch.randn((B, QWEN3_VOCAB), device=dev, generator=g) * 3).to(dtype)
    logits[3, 1::5] = float("-inf")
    temps = torch.linspace(0.4, 1.5, B, device=dev)
    _logits_case(dev, logits, temps, mode, 7, "qwen3")


@pytest.mark.parametrize("vocab,offset,dtype", [
    (1003, 0, torch.bfloat16),    # partial last chunk, d % 4 != 0
    (5000, 1, torch.bfloat16),    # unaligned rows
    (200001, 0, torch.float16),   # rows the softmax kernel streams
    (4099, 1, torch.float32),     # unaligned fp32 rows
    (32000, 0, torch.bfloat16),   # a 32K vocabulary
    (65536, 0, torch.float16),    # 64 blocks exactly
    (QWEN3_VOCAB + 8, 0, torch.bfloat16),  # just past the Qwen3 vocabulary
    (90000, 0, torch.bfloat16),   # register-held rows, 11 chunks a lane
    (120008, 0, torch.float16),   # register-held, partial last block
    (163840, 0, torch.float16),   # the longest register-held rows (20 chunks)
    (163848, 0, torch.bfloat16),  # one chunk past them: streamed
    (40004, 0, torch.bfloat16),   # aligned, d % 8 != 0: streamed
])
def test_sampling_from_logits_shapes(dev, vocab, offset, dtype):
    g = torch.Generator(device=dev)
    g.manual_seed(vocab)
    B = 5
    base = (torch.randn((B, vocab + 13), device=dev, generator=g) * 4).to(dtype)
    logits = base[:, offset:offset + vocab]
    temps = torch.tensor([0.5, 0.8, 1.0, 1.1, 2.0], device=dev)
    for mode in ("plain", "top_k_top_p"):
        _logits_case(dev, logits, temps, mode, vocab + 1, f"v{vocab}+{offset}")


def test_sampling_from_logits_seeded_shapes(dev):
    """Seeded random shapes (vocabulary 8 to 200,000, aligned or offset
    rows, bf16 / fp16 / fp32, random temperatures and rounds): each lands on
    the register-held or the streamed path by its own length and alignment,
    and every draw equals softmax then draw."""
    rng = np.random.default_rng(2024)
    dtypes = [torch.bfloat16, torch.float16, torch.float32]
    for i in range(10):
        vocab = int(rng.choice([int(rng.integers(8, 4096)), int(rng.integers(4096, 200001))]))
        if i % 3 == 0:
            vocab = vocab // 8 * 8 or 8  # multiples of 8 reach the held path
        offset = int(rng.integers(0, 2)) if i % 2 else 0
        dtype = dtypes[i % 3]
        B = int(rng.integers(1, 6))
        g = torch.Generator(device=dev)
        g.manual_seed(100 + i)
        base = (torch.randn((B, vocab + 8), device=dev, generator=g) *
                float(rng.uniform(0.5, 6))).to(dtype)
        logits = base[:, offset:offset + vocab]
        temps = torch.from_numpy(rng.uniform(0.3, 2.0, B).astype(np.float32)).to(dev)
        mode = ["plain", "top_k", "top_p", "top_k_top_p"][i % 4]
        _logits_case(dev, logits, temps, mode, 200 + i, f"seeded{i}-v{vocab}+{offset}")


def test_sampling_from_logits_rejects_bad_arguments(dev):
    x = torch.zeros((2, 64), device=dev, dtype=torch.bfloat16)
    u = torch.rand(2, device=dev)
    out = torch.empty(2, dtype=torch.int32, device=dev)
    lib = capi.lib()
    assert lib.sgl_sampling_from_logits(capi._p(x), 64, 0, None, 1.0, capi._p(u), 4, None, None, 0,
                                        None, 0.0, capi._p(out), None, 2, 64, 1, None) == -1
    assert lib.sgl_sampling_from_logits(capi._p(x), 64, 9, None, 1.0, capi._p(u), 0, None, None, 0,
                                        None, 0.0, capi._p(out), None, 2, 64, 1, None) == -2
    assert lib.sgl_sampling_from_logits(capi._p(x), 64, 0, None, 0.0, capi._p(u), 0, None, None, 0,
                                        None, 0.0, capi._p(out), None, 2, 64, 1, None) == -1


def test_sampler_entry_points_replay_in_a_graph(dev):
    """softmax_temperature and the draw from logits captured once in a HIP
    graph; each replay, with new logits and uniforms written in place and
    eager work between replays, equals the eager calls on the same inputs."""
    g = torch.Generator(device=dev)
    g.manual_seed(99)
    B, V = 16, QWEN3_VOCAB
    logits = torch.empty((B, V), device=dev, dtype=torch.bfloat16)
    temps = torch.linspace(0.5, 1.3, B, device=dev)
    u = torch.empty((32, B), device=dev)
    k = torch.full((B,), 40, dtype=torch.int32, device=dev)
    tp = torch.full((B,), 0.85, device=dev)
    probs = torch.empty((B, V), device=dev)

    def fill(i):
        logits.copy_((torch.randn((B, V), device=dev, generator=g) * (2 + i)).to(torch.bfloat16))
        u.copy_(torch.rand((32, B), device=dev, generator=g))

    fill(0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up outside the capture
        capi.softmax_temperature(logits, temps, out=probs)
        capi.sampling_from_logits(logits, u, "top_k_top_p", temps, top_k=k, top_p=tp)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        capi.softmax_temperature(logits, temps, out=probs)
        s_g, ok_g = capi.sampling_from_logits(logits, u, "top_k_top_p", temps, top_k=k, top_p=tp)
    for i in range(4):
        note(f"graph replay {i}")
        fill(i + 1)
        graph.replay()
        torch.cuda.synchronize()
        p_eager = capi.softmax_temperature(logits, temps)
        s_e, ok_e = capi.sampling_from_logits(logits, u, "top_k_top_p", temps, top_k=k, top_p=tp)
        torch.cuda.synchronize()
        assert torch.equal(probs, p_eager)
        assert torch.equal(s_g, s_e) and torch.equal(ok_g, ok_e)
    del graph
