"""Shared helpers for the parity tests (bf16 <-> uint16, tolerances)."""
import numpy as np
import torch

ATOL = 2e-2  # attention outputs vs the fp32-softmax oracle (the stated parity tolerance)
RTOL = 1e-2


def u16(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> numpy uint16 bit patterns (host copy)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def from_u16(a: np.ndarray, device=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)
    return t if device is None else t.to(device)


def bf16_f32(a: np.ndarray) -> np.ndarray:
    return (a.astype(np.uint32) << 16).view(np.float32)


def bf16_ulp_dist(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in ulps between two uint16 arrays of bf16 (or fp16: the same
    sign-magnitude ordering) bit patterns."""
    def key(x):
        x = x.astype(np.int32)
        return np.where(x & 0x8000, -(x & 0x7FFF), x & 0x7FFF)
    return np.abs(key(a) - key(b))


def assert_attn_close(got: np.ndarray, ref: np.ndarray, atol=ATOL, rtol=RTOL, what=""):
    diff = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    bound = atol + rtol * np.abs(ref)
    bad = diff > bound
    if bad.any():
        i = np.unravel_index(np.argmax(diff - bound), diff.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {diff.size} elements out of tolerance "
            f"(atol {atol}, rtol {rtol}); worst at {i}: got {got[i]}, ref {ref[i]}")


def assert_bf16_close(got: np.ndarray, ref: np.ndarray, atol=1e-6, what: str = "",
                      max_ulp: int = 1, dtype: str = "bf16"):
    """bf16 results of fp32 math with the same rounding points: within one bf16
    ulp of the oracle, or within atol absolute where the fp32 result sits near
    zero after cancellation (x c - y s), where one fp32 ulp of difference in the
    inputs (fused multiply-add vs separate rounding) spans many bf16 ulps.
    atol may be an array (a per-element bound) broadcastable to ref. dtype
    "fp16": the same for fp16 bit patterns (ulps of fp16)."""
    val = bf16_f32 if dtype == "bf16" else (lambda x: x.view(np.float16).astype(np.float32))
    dist = bf16_ulp_dist(got, ref)
    diff = np.abs(val(got).astype(np.float64) - val(ref).astype(np.float64))
    bad = (dist > max_ulp) & (diff > atol)
    if bad.any():
        i = np.unravel_index(np.argmax(np.where(bad, diff, 0)), diff.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} elements differ by more "
                             f"than {max_ulp} {dtype} ulp and {atol}; worst at {i}: got "
                             f"{val(got)[i]}, ref {val(ref)[i]}")


def decode_ws_bytes(units: int, hq: int) -> int:
    """Decode workspace layout: a 256-byte header (status word), then fp32
    partial outputs [2 units, hq, 128], log2-sum-exp [2 units, hq] and the
    int32 request running into each unit [units], each padded to 256
    bytes."""
    npart = 2 * units * hq
    pad = lambda x: -(-x // 256) * 256
    return 256 + pad(npart * 512) + pad(npart * 4) + pad(units * 4)


def forced_plan(capi, kv_indptr, hq, hkv, unit):
    """A decode plan with a forced unit size (every unit `unit` tokens), so
    small batches exercise many split pieces."""
    plan = capi.decode_plan(kv_indptr, hq, hkv, 128)
    total = int(kv_indptr[-1])
    plan.kv_chunk_size = unit
    plan.min_chunk_size = unit
    plan.num_units = max(1, -(-total // unit))
    plan.max_total_tokens = plan.num_units * unit
    plan.split_kv = 1
    plan.workspace_bytes = decode_ws_bytes(plan.num_units, hq)
    return plan
