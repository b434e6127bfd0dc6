"""The C ABI library loads, exports every symbol include/sgl_attn.h declares,
and its host-side logic (argument checks, split-KV plan) behaves — all
without a GPU: none of these calls reaches the HIP runtime."""
import ctypes
import re
import subprocess

import pytest

from conftest import capi


def declared_symbols():
    text = capi.HEADER_PATH.read_text()
    return sorted(set(re.findall(r"\b(sgl_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared_symbols() == sorted(capi.exported_symbols())


def test_library_exports_every_declared_symbol():
    lib = capi.lib()
    out = subprocess.run(["nm", "-D", "--defined-only", str(capi.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (sgl_\w+)", out))
    for name in declared_symbols():
        assert name in exported, name
        getattr(lib, name)
    assert lib.sgl_abi_version() == capi.ABI_VERSION


def test_status_strings():
    lib = capi.lib()
    assert lib.sgl_status_string(0) == b"ok"
    assert lib.sgl_status_string(-1) == b"invalid argument"
    assert lib.sgl_status_string(-2) == b"unsupported configuration"
    assert lib.sgl_status_string(-3) == b"workspace or plan capacity exceeded"


def test_argument_checks_reject_before_launch():
    lib = capi.lib()
    # null pointers with work to do
    assert lib.sgl_store_kv(None, None, None, None, None, 0, 5, 64, 64, 64, None) == -1
    # empty work is a no-op success
    assert lib.sgl_store_kv(None, None, None, None, None, 0, 0, 64, 64, 64, None) == 0
    # row stride shorter than the row
    assert lib.sgl_store_kv(1, 1, 1, 1, 1, 0, 5, 64, 32, 64, None) == -1
    # bad index dtype
    assert lib.sgl_store_kv(16, 16, 16, 16, 16, 7, 5, 64, 64, 64, None) == -2
    assert lib.sgl_build_decode_indices(None, 4, 8, 8, None, None, None, 3, None) == -1
    assert lib.sgl_build_decode_indices(None, 4, 8, 8, None, None, None, 0, None) == 0
    assert lib.sgl_gather_int32_2d(None, 4, 2, 8, None, None, None, 3, None) == -1  # stride < cols
    assert lib.sgl_qk_rmsnorm(None, None, None, None, 3, 2, 1, 128, 0, 0, 0, 0,
                              ctypes.c_float(1e-6), 0, None) == -1
    assert lib.sgl_qk_rmsnorm(None, None, None, None, 3, 2, 1, 128, 0, 0, 0, 0,
                              ctypes.c_float(1e-6), 2, None) == -2  # dtype not built
    assert lib.sgl_rope(None, None, None, None, None, 3, 2, 1, 7, 128, 7, 0, 0, 0, 0,
                        0, None) == -1  # odd rotary_dim
    assert lib.sgl_rope(None, None, None, None, None, 3, 2, 1, 8, 128, 4, 0, 0, 0, 0,
                        2, None) == -2  # dtype not built
    # fused: head_dim not built
    assert lib.sgl_fused_qknorm_rope_store(16, 96 * 5, 16, 16, None, None, 16, 16, 16, 16, 4, 1,
                                           2, 96, ctypes.c_float(1e-6), 0, None) == -2
    # fused: unknown flag bit
    assert lib.sgl_fused_qknorm_rope_store(16, 128 * 4, 16, 16, None, None, 16, 16, 16, 16, 4, 2,
                                           1, 128, ctypes.c_float(1e-6), 2, None) == -1
    # fused: misaligned qkv
    assert lib.sgl_fused_qknorm_rope_store(18, 128 * 4, 16, 16, None, None, 16, 16, 16, 16, 4, 2,
                                           1, 128, ctypes.c_float(1e-6), 0, None) == -4
    assert lib.sgl_paged_prefill(16, 0, 0, 16, 16, 0, 0, 16, 16, 16, None, 2, 4, 16, 8, 64,
                                 ctypes.c_float(0.1), 16, 0, 0, None) == -2  # head_dim 64
    # batched int32 copies: too many entries, a null pointer with work, nothing to do
    copies = (capi.I32Copy * 9)()
    assert lib.sgl_copy_i32(copies, 9, None) == -1
    copies[0] = capi.I32Copy(None, 16, 5)
    assert lib.sgl_copy_i32(copies, 1, None) == -1
    copies[0] = capi.I32Copy(16, 16, -1)
    assert lib.sgl_copy_i32(copies, 1, None) == -1
    copies[0] = capi.I32Copy(None, None, 0)
    assert lib.sgl_copy_i32(copies, 1, None) == 0
    assert lib.sgl_copy_i32(None, 0, None) == 0


def ws_bytes(units, hq):
    """Workspace layout: 256-byte header, then fp32 partial o and lse (two
    slots per unit) and one int32 per unit."""
    npart = 2 * units * hq
    pad = lambda x: -(-x // 256) * 256
    return 256 + pad(npart * 512) + pad(npart * 4) + pad(units * 4)


def test_decode_plan_host_logic():
    # config 4 shape: 32q / 8kv, ragged lengths
    import numpy as np
    rng = np.random.default_rng(0)
    kv = rng.integers(128, 4097, 256)
    ip = np.concatenate([[0], np.cumsum(kv)])
    plan = capi.decode_plan(ip, 32, 8, 128)
    assert plan.kv_chunk_size % 16 == 0 and plan.kv_chunk_size >= 64
    W = plan.kv_chunk_size
    assert plan.min_chunk_size == 64
    # units cover the token stream exactly
    assert plan.num_units == -(-int(kv.sum()) // W)
    assert plan.max_total_tokens == plan.num_units * W >= int(kv.sum())
    # the unit size the device picks, and whether some request spans units
    w = min(W, max(plan.min_chunk_size, -(-(-(-int(kv.sum()) // plan.num_units)) // 16) * 16))
    pieces = [(ip[r + 1] - 1) // w - ip[r] // w + 1 for r in range(256)]
    assert plan.split_kv == (max(pieces) > 1)
    # partials: two slots per unit, independent of request lengths
    assert plan.workspace_bytes == ws_bytes(plan.num_units, 32)
    assert plan.workspace_bytes < 16 << 20
    # one unit per resident workgroup: 1 per CU at 8 kv heads on 256 CUs
    assert 250 <= plan.num_units <= 260
    # a batch shorter than one unit is a single unit; a request inside it is whole
    plan = capi.decode_plan([0, 20, 52], 16, 8, 128)
    assert plan.num_units == 1 and plan.split_kv == 0
    # graph-capture style plan: every request at the capture max length
    plan = capi.decode_plan(list(range(0, 8 * 32768 + 1, 32768)), 32, 8, 128)
    assert plan.max_total_tokens >= 8 * 32768
    with pytest.raises(capi.SglError):
        capi.decode_plan([0, 10], 48, 2, 128)  # group 24 > 16
    with pytest.raises(capi.SglError):
        capi.decode_plan([0, 10], 16, 8, 96)   # head_dim not built
    with pytest.raises(capi.SglError):
        capi.decode_plan([0, 10, 5], 16, 8, 128)  # negative length
    with pytest.raises(capi.SglError):
        capi.decode_plan([3, 10], 16, 8, 128)  # kv_indptr[0] != 0


def test_decode_plan_covers_any_batch_property():
    """Property over random batches (0-600 requests, lengths 0-40,000, GQA
    layouts): the plan's units of W tokens cover the batch, the unit size the
    device derives from kv_indptr (clamp(round16(ceil(total / units)),
    W_min, W)) also covers it, W is a 16-token multiple in [64, 8192], the
    plan accepts its own batch, and the workspace is two partial slots per
    unit. A uniform-by-construction check of the coupling between the host
    plan and the device's unit sizing."""
    import numpy as np
    from hypothesis import given, settings, strategies as st

    @settings(max_examples=300, deadline=None)
    @given(st.integers(0, 600), st.integers(0, 40000), st.sampled_from([(16, 8), (32, 8), (32, 4),
                                                                       (64, 4), (8, 8), (40, 8)]),
           st.integers(0, 2 ** 31 - 1))
    def check(n, max_len, heads, seed):
        hq, hkv = heads
        rng = np.random.default_rng(seed)
        lens = rng.integers(0, max_len + 1, n)
        ip = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
        plan = capi.decode_plan(ip, hq, hkv, 128)
        total = int(ip[-1])
        W = plan.kv_chunk_size
        assert W % 16 == 0 and 64 <= W <= 8192 and plan.min_chunk_size == 64
        assert plan.max_total_tokens == plan.num_units * W >= total
        w_dev = min(W, max(64, -(-(-(-total // plan.num_units)) // 16) * 16))
        assert plan.num_units * w_dev >= total
        assert capi.decode_plan_check(plan, ip) == 0
        assert plan.workspace_bytes == ws_bytes(plan.num_units, hq)

    check()


def test_mixed_split_heuristic():
    """Host logic, no GPU: the decode's CU share grows with its K/V bytes and shrinks with the
    prefill's flops, in multiples of 8 within [8, CUs]."""
    cus = capi.mixed_decode_cus(10 ** 6, 4, 128, 0.0)
    assert cus >= 8 and cus % 8 == 0
    a = capi.mixed_decode_cus(1_081_344, 4, 128, 171.8e9)  # config 5's layer
    assert 8 <= a < cus and a % 8 == 0
    assert capi.mixed_decode_cus(2_000_000, 4, 128, 171.8e9) >= a
    assert capi.mixed_decode_cus(1_081_344, 4, 128, 400e9) <= a
    assert capi.mixed_decode_cus(1, 4, 128, 1e15) == 8


def test_decode_plan_cus_host():
    """A plan for a decode sharing the device: about decode_cus x (8 / hkv)
    units, the usual capacity contract; kv-head counts that do not divide 8
    are refused."""
    import numpy as np
    rng = np.random.default_rng(3)
    kv = rng.integers(1024, 32769, 64)
    ip = np.concatenate([[0], np.cumsum(kv)])
    for cus, hq, hkv in ((160, 32, 4), (64, 32, 8), (8, 16, 1), (8, 16, 2), (32, 8, 1)):
        plan = capi.decode_plan_cus(ip, hq, hkv, 128, cus)
        # The fused launch stages each unit's slot indices (4 bytes a token)
        # and per kv head the Q rows (16 x 136 bf16) and a 4 KiB K tile in
        # LDS for 8 / hkv units per workgroup: all of it within the CU's
        # 160 KiB.
        wave = 16 * 136 * 2 + 4096
        assert (8 // hkv) * (hkv * wave + 4 * plan.kv_chunk_size) <= 160 * 1024
        # The longest unit that fits bounds the count from below.
        w_max = min(8192, ((160 * 1024 // (8 // hkv) - hkv * wave) // 4) // 16 * 16)
        target = max(cus * (8 // hkv), -(-int(kv.sum()) // w_max))
        assert target * 0.9 <= plan.num_units <= target
        assert plan.max_total_tokens == plan.num_units * plan.kv_chunk_size >= int(kv.sum())
        assert capi.decode_plan_check(plan, ip) == 0
    with pytest.raises(capi.SglError):
        capi.decode_plan_cus(ip, 48, 3, 128, 64)
    with pytest.raises(capi.SglError):
        capi.decode_plan_cus(ip, 32, 4, 128, 0)


def test_decode_plan_check_host():
    """A plan serves any batch with at most batch_size requests and
    max_total_tokens tokens, whatever the per-request lengths; beyond it the
    host check says CAPACITY."""
    plan = capi.decode_plan([0, 1000, 2000, 3000, 4000], 32, 4, 128)
    cap = plan.max_total_tokens
    assert capi.decode_plan_check(plan, [0, 1000, 2000, 3000, 4000]) == 0
    assert capi.decode_plan_check(plan, [0, cap]) == 0          # one request, all tokens
    assert capi.decode_plan_check(plan, [0, 1, 2, 3]) == 0
    assert capi.decode_plan_check(plan, [0, cap + 1]) == -3
    assert capi.decode_plan_check(plan, [0] * 6) == -3            # 5 requests > 4
    assert capi.decode_plan_check(plan, [0, 5, 4]) == -1          # negative length


def test_paged_decode_rejects_inconsistent_plan():
    """The launch validates the plan's derived fields before touching the GPU."""
    plan = capi.decode_plan([0, 100, 300], 16, 8, 128)
    bad = capi.DecodePlan.from_buffer_copy(plan)
    bad.max_total_tokens += 16
    lib = capi.lib()
    args = lambda pl, ws_bytes, ostride_h=128: (  # noqa: E731
        ctypes.byref(pl), 16, 16 * 128, 128, 16, 16, 8 * 128, 128, 16, 16, None, 2, 16, 8, 128,
        ctypes.c_float(0.1), 16, 16 * 128, ostride_h, 16, ws_bytes, None)
    assert lib.sgl_paged_decode(*args(bad, plan.workspace_bytes)) == -1
    # workspace smaller than the plan's
    assert lib.sgl_paged_decode(*args(plan, plan.workspace_bytes - 1)) == -3
    # output head stride not a multiple of 8 elements (16-byte row stores)
    assert lib.sgl_paged_decode(*args(plan, plan.workspace_bytes, 132)) == -4
