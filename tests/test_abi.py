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
                              ctypes.c_float(1e-6), None) == -1
    assert lib.sgl_rope(None, None, None, None, None, 3, 2, 1, 7, 128, 7, 0, 0, 0, 0,
                        None) == -1  # odd rotary_dim
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


def test_decode_plan_host_logic():
    # config 4 shape: 32q / 8kv, ragged lengths
    import numpy as np
    rng = np.random.default_rng(0)
    kv = rng.integers(128, 4097, 256)
    ip = np.concatenate([[0], np.cumsum(kv)])
    plan = capi.decode_plan(ip, 32, 8, 128)
    assert plan.kv_chunk_size % 16 == 0 and plan.kv_chunk_size >= 64
    W = plan.kv_chunk_size
    assert plan.min_chunk_size <= W and plan.min_chunk_size % 16 == 0
    # units cover the token stream exactly
    assert plan.num_units == -(-int(kv.sum()) // W)
    # the unit size the device picks, and the pieces per request it implies
    w = min(W, max(plan.min_chunk_size, -(-(-(-int(kv.sum()) // plan.num_units)) // 16) * 16))
    pieces = [(ip[r + 1] - 1) // w - ip[r] // w + 1 for r in range(256)]
    assert plan.max_chunks >= max(pieces)
    assert plan.max_chunks == -(-int(kv.max()) // plan.min_chunk_size) + 1 <= 128
    assert plan.split_kv == (max(pieces) > 1)
    npart = 256 * plan.max_chunks * 32
    assert plan.workspace_bytes == -(-npart * 512 // 256) * 256 + -(-npart * 4 // 256) * 256
    # one unit per resident workgroup: 1 per CU at 8 kv heads on 256 CUs
    assert 250 <= plan.num_units <= 260
    # a batch shorter than one unit is a single unit; a request inside it is whole
    plan = capi.decode_plan([0, 20, 52], 16, 8, 128)
    assert plan.num_units == 1 and plan.split_kv == 0
    # graph-capture style plan: every request at the capture max length; any
    # shorter replay batch fits its piece capacity
    plan = capi.decode_plan(list(range(0, 8 * 32768 + 1, 32768)), 32, 8, 128)
    assert (plan.max_chunks - 1) * plan.min_chunk_size >= 32768
    assert plan.max_chunks <= 128
    with pytest.raises(capi.SglError):
        capi.decode_plan([0, 10], 48, 2, 128)  # group 24 > 16
    with pytest.raises(capi.SglError):
        capi.decode_plan([0, 10], 16, 8, 96)   # head_dim not built
    with pytest.raises(capi.SglError):
        capi.decode_plan([0, 10, 5], 16, 8, 128)  # negative length
