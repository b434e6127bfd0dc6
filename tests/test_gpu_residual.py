"""GPU parity of the residual-path kernels (marked gpu): RMSNorm over hidden
rows, fused add + RMSNorm, SiLU/GELU-and-mul, in bf16 and fp16, through the
C ABI (libsgl_attn.so via capi) against the CPU oracle.

Bars: the fused add's residual output is bit-exact (one rounding of the
fp32 sum); normalised and activated outputs are within one ulp of T of the
oracle (fp32 math with the reference's rounding points; reduction order and
the exp / reciprocal / square-root implementations differ), plus one fp16
subnormal step. Shapes: the reference tests' (10 x 128 norm, 10 x 256
activations in fp16), Qwen3 hidden sizes 1024 / 2048 / 4096 / 5120 and MLP
widths 768 / 3072 / 12288, rows longer than 8192 (second-pass path), widths
that are not a multiple of 8 (element path) and strided rows.
"""
import sys

import numpy as np
import pytest
import torch

from conftest import capi

pytestmark = pytest.mark.gpu

TORCH_DT = {"bf16": torch.bfloat16, "fp16": torch.float16}
# One ulp of T relative to |v| is at most 2^-7 (bf16, 8-bit significand) or
# 2^-10 (fp16, 11-bit significand).
ULP = {"bf16": 2.0 ** -7, "fp16": 2.0 ** -10}
ATOL_T = {"bf16": 1e-12, "fp16": 2.0 ** -24}


def note(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def rand_t(shape, dtype, dev, seed, scale=1.0):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return (torch.randn(shape, device=dev, generator=g) * scale).to(TORCH_DT[dtype])


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def assert_within_ulp(got, ref, dtype, what):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    bound = ULP[dtype] * np.maximum(np.abs(ref), np.abs(got)) + ATOL_T[dtype]
    bad = ~(np.abs(got - ref) <= bound)
    if bad.any():
        i = np.unravel_index(np.argmax(np.where(bad, np.abs(got - ref), 0)), got.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} elements beyond one ulp; "
                             f"worst at {i}: got {got[i]}, ref {ref[i]}")


NORM_CASES = [
    (10, 128, "fp16"),     # the reference test's shape
    (8192, 1024, "bf16"),  # Qwen3-0.6B hidden, a full chunk of tokens
    (257, 4096, "bf16"),   # Qwen3-8B hidden, ragged row count
    (33, 5120, "fp16"),
    (7, 12288, "bf16"),    # longer than 8192: second-pass path
    (5, 1000, "bf16"),     # not a multiple of 8: element path
    (3, 2048, "fp16"),
]


@pytest.mark.parametrize("rows,d,dtype", NORM_CASES)
def test_rmsnorm(oracle, dev, rows, d, dtype):
    note(f"rmsnorm rows={rows} d={d} {dtype}")
    x = rand_t((rows, d), dtype, dev, 1, 2.0)
    w = (torch.rand(d, device=dev) + 0.5).to(TORCH_DT[dtype])
    out = capi.rmsnorm(x, w, 1e-6)
    torch.cuda.synchronize()
    ref = oracle.rmsnorm(host(x), host(w), 1e-6, dtype)
    assert_within_ulp(host(out), ref, dtype, "rmsnorm")
    # in place (forward_inplace) gives the same bits
    y = x.clone()
    capi.rmsnorm(y, w, 1e-6, out=y)
    torch.cuda.synchronize()
    assert torch.equal(y, out)


def test_rmsnorm_strided_rows(oracle, dev):
    note("rmsnorm on a column slice (row stride > d)")
    big = rand_t((64, 3 * 1024), "bf16", dev, 2)
    x = big[:, 1024:2048]
    w = (torch.rand(1024, device=dev) + 0.5).to(torch.bfloat16)
    out = torch.empty((64, 2048), device=dev, dtype=torch.bfloat16)[:, :1024]
    capi.rmsnorm(x, w, 1e-5, out=out)
    torch.cuda.synchronize()
    ref = oracle.rmsnorm(host(x), host(w), 1e-5, "bf16")
    assert_within_ulp(host(out), ref, "bf16", "strided rmsnorm")


@pytest.mark.parametrize("rows,d,dtype", NORM_CASES)
def test_fused_add_rmsnorm(oracle, dev, rows, d, dtype):
    note(f"fused add rmsnorm rows={rows} d={d} {dtype}")
    x = rand_t((rows, d), dtype, dev, 3)
    r = rand_t((rows, d), dtype, dev, 4, 3.0)
    w = (torch.rand(d, device=dev) + 0.5).to(TORCH_DT[dtype])
    xo_ref, ro_ref = oracle.fused_add_rmsnorm(host(x), host(r), host(w), 1e-6, dtype)
    capi.fused_add_rmsnorm(x, r, w, 1e-6)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(r), ro_ref)
    if d <= 8192:
        assert_within_ulp(host(x), xo_ref, dtype, "fused add rmsnorm")
    else:
        # long rows normalise the rounded sum (second pass re-reads residual)
        assert_within_ulp(host(x), oracle.rmsnorm(ro_ref, host(w), 1e-6, dtype), dtype,
                          "fused add rmsnorm, long rows")


def test_fused_add_rmsnorm_strided(oracle, dev):
    note("fused add rmsnorm with strided x and residual")
    xb = rand_t((40, 4096 + 64), "bf16", dev, 5)
    rb = rand_t((40, 8192), "bf16", dev, 6)
    x, r = xb[:, 64:], rb[:, :4096]
    w = (torch.rand(4096, device=dev) + 0.5).to(torch.bfloat16)
    xo_ref, ro_ref = oracle.fused_add_rmsnorm(host(x), host(r), host(w), 1e-6, "bf16")
    rest = rb[:, 4096:].clone()
    capi.fused_add_rmsnorm(x, r, w, 1e-6)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(r), ro_ref)
    assert_within_ulp(host(x), xo_ref, "bf16", "strided fused add rmsnorm")
    assert torch.equal(rb[:, 4096:], rest)  # bytes past each row untouched


ACT_CASES = [
    (10, 128, "fp16"),     # the reference test's shape: [10, 256] -> [10, 128]
    (4096, 12288, "bf16"),  # Qwen3-8B MLP
    (1000, 768, "fp16"),   # Qwen3-30B-A3B expert width
    (77, 3072, "bf16"),
    (3, 1000, "bf16"),     # element path
    (5, 7, "fp16"),
]


@pytest.mark.parametrize("act", ["silu", "gelu"])
@pytest.mark.parametrize("tokens,d,dtype", ACT_CASES)
def test_act_and_mul(oracle, dev, act, tokens, d, dtype):
    note(f"{act}_and_mul tokens={tokens} d={d} {dtype}")
    inp = rand_t((tokens, 2 * d), dtype, dev, 7, 3.0)
    out = torch.empty((tokens, d), device=dev, dtype=TORCH_DT[dtype])
    (capi.silu_and_mul if act == "silu" else capi.gelu_and_mul)(out, inp)
    torch.cuda.synchronize()
    ref = oracle.act_and_mul(host(inp), act, dtype)
    assert_within_ulp(host(out), ref, dtype, f"{act}_and_mul")


def test_act_and_mul_strided(oracle, dev):
    note("silu_and_mul with padded input and output rows")
    big = rand_t((50, 2 * 1536 + 32), "bf16", dev, 8)
    inp = big[:, 16:16 + 2 * 1536]
    outb = torch.zeros((50, 1536 + 8), device=dev, dtype=torch.bfloat16)
    out = outb[:, :1536]
    capi.silu_and_mul(out, inp)
    torch.cuda.synchronize()
    ref = oracle.act_and_mul(host(inp), "silu", "bf16")
    assert_within_ulp(host(out), ref, "bf16", "strided silu_and_mul")
    assert torch.count_nonzero(outb[:, 1536:]) == 0


def test_residual_path_rejects_bad_arguments(dev):
    note("residual-path argument checks")
    x = torch.zeros((4, 64), device=dev, dtype=torch.float32)
    w = torch.ones(64, device=dev, dtype=torch.float32)
    with pytest.raises(ValueError):
        capi.rmsnorm(x, w, 1e-6)  # fp32 is not a built type
    xb = torch.zeros((4, 64), device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        capi.fused_add_rmsnorm(xb, torch.zeros((4, 64), device=dev, dtype=torch.float16),
                               w.to(torch.bfloat16), 1e-6)
    with pytest.raises(ValueError):
        capi.silu_and_mul(torch.empty((4, 31), device=dev, dtype=torch.bfloat16), xb)
