"""ctypes binding of libsgl_attn.so (the C ABI in include/sgl_attn.h).

Thin tensor-level wrappers used by the tests and the bench: each function
checks shapes and dtypes the way the reference's TORCH_CHECKs do, passes
raw device pointers, strides and the current HIP stream, and raises
SglError on a non-zero status. There is no fallback: if the library is
not built, or a call is made on a tensor that is not on a HIP device,
the call raises.
"""
from __future__ import annotations

import ctypes
import math
import os
from pathlib import Path
from typing import Optional, Sequence

import torch

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libsgl_attn.so"
HEADER_PATH = PKG_DIR.parent / "include" / "sgl_attn.h"

SGL_INDEX_I32 = 0
SGL_INDEX_I64 = 1
SGL_DTYPE_BF16 = 0
SGL_DTYPE_F16 = 1
SGL_DTYPE_F32 = 2
ABI_VERSION = 15
FUSED_NO_K_WRITEBACK = 1  # SGL_FUSED_NO_K_WRITEBACK


class SglError(RuntimeError):
    def __init__(self, status: int, what: str):
        self.status = status
        super().__init__(f"{what} failed: status {status} ({status_string(status)})")


class DecodePlan(ctypes.Structure):
    _fields_ = [
        ("kv_chunk_size", ctypes.c_int32),
        ("min_chunk_size", ctypes.c_int32),
        ("num_units", ctypes.c_int32),
        ("split_kv", ctypes.c_int32),
        ("batch_size", ctypes.c_int32),
        ("num_qo_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("max_total_tokens", ctypes.c_int64),
        ("workspace_bytes", ctypes.c_int64),
    ]


class I32Copy(ctypes.Structure):
    """sgl_i32_copy_t."""
    _fields_ = [("src", ctypes.c_void_p), ("dst", ctypes.c_void_p), ("count", ctypes.c_int64)]


MAX_I32_COPIES = 8

_lib: Optional[ctypes.CDLL] = None

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float

_SIGNATURES = {
    "sgl_status_string": ([_i32], ctypes.c_char_p),
    "sgl_abi_version": ([], _i32),
    "sgl_store_kv": ([_vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _vp], _i32),
    "sgl_build_decode_indices": ([_vp, _i64, _i64, _i64, _vp, _vp, _vp, _i32, _vp], _i32),
    "sgl_build_prefill_indices": ([_vp, _i64, _i64, _i64, _vp, _vp, _vp, _i32, _vp], _i32),
    "sgl_write_token_pool": ([_vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp], _i32),
    "sgl_write_page_table": ([_vp, _i64, _i64, _i64, _vp, _i64, _vp, _i32, _i32, _vp], _i32),
    "sgl_gather_int32_2d": ([_vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp], _i32),
    "sgl_copy_i32": ([_vp, _i32, _vp], _i32),
    "sgl_rope_cos_sin_cache": ([_vp, _vp, _i64, _i32, _f32, _vp], _i32),
    "sgl_qk_rmsnorm": ([_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                        _f32, _i32, _vp], _i32),
    "sgl_rope": ([_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                  _i64, _i64, _i32, _vp], _i32),
    "sgl_fused_qknorm_rope_store": ([_vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64,
                                     _i32, _i32, _i32, _f32, _i32, _vp], _i32),
    "sgl_decode_plan": ([_vp, _i32, _i32, _i32, _i32, ctypes.POINTER(DecodePlan)], _i32),
    "sgl_decode_plan_check": ([ctypes.POINTER(DecodePlan), _vp, _i32], _i32),
    "sgl_decode_status": ([_vp, _vp, _vp], _i32),
    "sgl_paged_decode_noalloc": ([ctypes.POINTER(DecodePlan), _vp, _i64, _i64, _vp, _vp, _i64,
                                  _i64, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _f32, _vp, _i64,
                                  _i64, _vp], _i32),
    "sgl_paged_decode": ([ctypes.POINTER(DecodePlan), _vp, _i64, _i64, _vp, _vp, _i64, _i64,
                          _vp, _vp, _vp, _i32, _i32, _i32, _i32, _f32, _vp, _i64, _i64, _vp,
                          _i64, _vp], _i32),
    "sgl_rmsnorm": ([_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _f32, _vp], _i32),
    "sgl_fused_add_rmsnorm": ([_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _f32, _vp], _i32),
    "sgl_silu_and_mul": ([_vp, _vp, _i64, _i64, _i64, _i64, _i32, _vp], _i32),
    "sgl_gelu_and_mul": ([_vp, _vp, _i64, _i64, _i64, _i64, _i32, _vp], _i32),
    "sgl_softmax_temperature": ([_vp, _i64, _vp, _i64, _i32, _vp, _f32, _i64, _i64, _vp], _i32),
    "sgl_sampling_from_logits": ([_vp, _i64, _i32, _vp, _f32, _vp, _i32, _vp, _vp, _i32, _vp, _f32,
                                  _vp, _vp, _i32, _i32, _i32, _vp], _i32),
    "sgl_sampling_from_probs": ([_vp, _vp, _vp, _i32, _i32, _i32, _vp], _i32),
    "sgl_top_k_sampling_from_probs": ([_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32,
                                       _vp], _i32),
    "sgl_top_p_sampling_from_probs": ([_vp, _vp, _vp, _vp, _vp, _i32, _f32, _i32, _i32, _i32,
                                       _vp], _i32),
    "sgl_top_k_top_p_sampling_from_probs": ([_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _f32, _i32,
                                             _i32, _i32, _vp], _i32),
    "sgl_paged_prefill": ([_vp, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _vp, _vp, _vp, _i32,
                           _i32, _i32, _i32, _i32, _f32, _vp, _i64, _i64, _vp], _i32),
    "sgl_mixed_decode_cus": ([_i64, _i32, _i32, ctypes.c_double], _i32),
    "sgl_decode_plan_cus": ([_vp, _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(DecodePlan)], _i32),
    "sgl_paged_mixed": ([ctypes.POINTER(DecodePlan), _vp, _i64, _i64, _vp, _vp, _i64, _i64,
                         _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32,
                         _f32, _vp, _i64, _i64, _vp, _i64, _vp], _i32),
}


def lib() -> ctypes.CDLL:
    """Load the library once. Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                "(python sglang.cpp_amd/build.py)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = res
        if handle.sgl_abi_version() != ABI_VERSION:
            raise RuntimeError("libsgl_attn.so ABI version does not match capi.py")
        _lib = handle
    return _lib


def exported_symbols() -> Sequence[str]:
    return tuple(_SIGNATURES)


def status_string(status: int) -> str:
    try:
        return lib().sgl_status_string(status).decode()
    except Exception:  # library not loadable: still format the error
        return "unknown"


def _check(status: int, what: str) -> None:
    if status != 0:
        raise SglError(status, what)


def _p(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(dev: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _need_gpu(*ts: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("sgl_attn ops take HIP device tensors only")
        dev = t.device if dev is None else dev
        if t.device != dev:
            raise ValueError("all tensors must be on the same device")
    return dev


# ---------------------------------------------------------------- KV store

def store_kv(k_cache: torch.Tensor, v_cache: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
             out_loc: torch.Tensor) -> None:
    """MHAKVCache::store_kv semantics (src/kvcache/mha_kvcache.cu:111-155).

    k_cache/v_cache: one layer's [slots, Hkv, D]; k/v: [T, Hkv, D] or
    [T, Hkv*D] views with a contiguous last dim; out_loc int32/int64 [T].
    """
    dev = _need_gpu(k_cache, v_cache, k, v, out_loc)
    if k.dtype != v.dtype or k.dtype != k_cache.dtype or k.element_size() != 2:
        raise ValueError("key, val and cache must share a 2-byte dtype (bf16/fp16)")
    if k.stride(-1) != 1 or v.stride(-1) != 1:
        raise ValueError("key and val last dimension must be contiguous")
    if out_loc.dim() != 1:
        raise ValueError("out_loc must be rank 1")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("KV cache buffers must be contiguous")
    elems = k_cache.shape[1:].numel()
    T = k.shape[0]
    if v.shape[0] != T or out_loc.shape[0] != T:
        raise ValueError("key, val and out_loc token counts must match")
    if k.shape[1:].numel() != elems or v.shape[1:].numel() != elems:
        raise ValueError("key and val shape must match KV cache layout")
    if out_loc.dtype == torch.int32:
        idt = SGL_INDEX_I32
    elif out_loc.dtype == torch.int64:
        idt = SGL_INDEX_I64
    else:
        raise ValueError("out_loc must be int32 or int64")
    _check(lib().sgl_store_kv(_p(k_cache), _p(v_cache), _p(k), _p(v), _p(out_loc), idt, T, elems,
                              k.stride(0), v.stride(0), _stream(dev)), "sgl_store_kv")


# ---------------------------------------------------------------- metadata

def _table_args(t: torch.Tensor):
    if t.dtype != torch.int32 or t.dim() != 2 or t.stride(1) != 1:
        raise ValueError("page table / token pool must be a 2-D int32 tensor, unit column stride")
    return t.shape[0], t.stride(0), t.shape[1]


def build_decode_indices(page_table: torch.Tensor, table_indices: torch.Tensor,
                         kv_indptr: torch.Tensor, indices: torch.Tensor) -> None:
    dev = _need_gpu(page_table, table_indices, kv_indptr, indices)
    rows, stride, cols = _table_args(page_table)
    B = table_indices.shape[0]
    _check(lib().sgl_build_decode_indices(_p(page_table), rows, stride, cols, _p(table_indices),
                                          _p(kv_indptr), _p(indices), B, _stream(dev)),
           "sgl_build_decode_indices")


def build_prefill_indices(page_table: torch.Tensor, table_indices: torch.Tensor,
                          kv_indptr: torch.Tensor, indices: torch.Tensor) -> None:
    dev = _need_gpu(page_table, table_indices, kv_indptr, indices)
    rows, stride, cols = _table_args(page_table)
    B = table_indices.shape[0]
    _check(lib().sgl_build_prefill_indices(_p(page_table), rows, stride, cols, _p(table_indices),
                                           _p(kv_indptr), _p(indices), B, _stream(dev)),
           "sgl_build_prefill_indices")


def write_token_pool(pool: torch.Tensor, req_indices: torch.Tensor, positions: torch.Tensor,
                     tokens: torch.Tensor) -> None:
    """write_token_pool (src/kernels/token_pool.cu:53-93)."""
    dev = _need_gpu(pool, req_indices, positions, tokens)
    rows, stride, cols = _table_args(pool)
    for t in (req_indices, positions, tokens):
        if t.dtype != torch.int32 or t.dim() != 1:
            raise ValueError("req_indices, positions and tokens must be 1-D int32")
    if not (req_indices.numel() == positions.numel() == tokens.numel()):
        raise ValueError("req_indices, positions and tokens must have the same length")
    _check(lib().sgl_write_token_pool(_p(pool), rows, stride, cols, _p(req_indices),
                                      _p(positions), _p(tokens), tokens.numel(), _stream(dev)),
           "sgl_write_token_pool")


def write_page_table(page_table: torch.Tensor, page_starts: torch.Tensor,
                     alloc_info: torch.Tensor, page_size: int) -> None:
    """CacheManager::write_page_table on the device (src/scheduler/prefill.cc:144-187).
    alloc_info: int32 [n, 3] (table_idx, first_page, last_page)."""
    dev = _need_gpu(page_table, page_starts, alloc_info)
    rows, stride, cols = _table_args(page_table)
    if page_starts.dtype != torch.int32 or alloc_info.dtype != torch.int32:
        raise ValueError("page_starts and alloc_info must be int32")
    if not alloc_info.is_contiguous() or alloc_info.dim() != 2 or alloc_info.shape[1] != 3:
        raise ValueError("alloc_info must be a contiguous [n, 3] int32 tensor")
    _check(lib().sgl_write_page_table(_p(page_table), rows, stride, cols, _p(page_starts),
                                      page_starts.numel(), _p(alloc_info), alloc_info.shape[0],
                                      page_size, _stream(dev)), "sgl_write_page_table")


def copy_i32(pairs: Sequence) -> None:
    """sgl_copy_i32: dst[:n] = src[:n] for each (src, dst, n) in one launch
    (int32 device tensors, n elements from the start of each)."""
    if len(pairs) > MAX_I32_COPIES:
        raise ValueError(f"at most {MAX_I32_COPIES} copies per call")
    ts = [t for src, dst, _ in pairs for t in (src, dst)]
    dev = _need_gpu(*ts)
    arr = (I32Copy * max(1, len(pairs)))()
    for i, (src, dst, n) in enumerate(pairs):
        if src.dtype != torch.int32 or dst.dtype != torch.int32:
            raise ValueError("copy_i32 moves int32 tensors")
        if not (0 <= n <= min(src.numel(), dst.numel())):
            raise ValueError("count exceeds a tensor")
        arr[i] = I32Copy(src.data_ptr(), dst.data_ptr(), n)
    _check(lib().sgl_copy_i32(arr, len(pairs), _stream(dev)), "sgl_copy_i32")


def gather_int32_2d(table: torch.Tensor, req_indices: torch.Tensor,
                    positions: torch.Tensor) -> torch.Tensor:
    """gather_int32_2d (src/kernels/token_pool.cu:95-133)."""
    dev = _need_gpu(table, req_indices, positions)
    rows, stride, cols = _table_args(table)
    if req_indices.numel() != positions.numel():
        raise ValueError("req_indices and positions must have the same length")
    out = torch.empty(req_indices.numel(), dtype=torch.int32, device=dev)
    _check(lib().sgl_gather_int32_2d(_p(table), rows, stride, cols, _p(req_indices),
                                     _p(positions), _p(out), out.numel(), _stream(dev)),
           "sgl_gather_int32_2d")
    return out


# ---------------------------------------------------------------- RoPE / norm

def rope_cos_sin_cache(max_pos: int, rotary_dim: int, base: float,
                       device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
    cos = torch.empty((max_pos, rotary_dim // 2), dtype=torch.float32, device=device)
    sin = torch.empty_like(cos)
    _check(lib().sgl_rope_cos_sin_cache(_p(cos), _p(sin), max_pos, rotary_dim, base,
                                        _stream(cos.device)), "sgl_rope_cos_sin_cache")
    return cos, sin


def qk_rmsnorm(q: torch.Tensor, k: Optional[torch.Tensor], q_weight: torch.Tensor,
               k_weight: Optional[torch.Tensor], eps: float) -> None:
    """fused_qk_rmsnorm_inplace_3d_strided (src/layers/normalization.cu:318-384), in place."""
    dev = _need_gpu(q, k, q_weight, k_weight)
    if q.dim() != 3 or q.stride(2) != 1 or (k is not None and (k.dim() != 3 or k.stride(2) != 1)):
        raise ValueError("q/k must be rank-3 with a contiguous last dimension")
    dt = _dtype_code(*[t for t in (q, k, q_weight, k_weight) if t is not None])
    d = q.shape[2]
    kh = 0 if k is None else k.shape[1]
    _check(lib().sgl_qk_rmsnorm(_p(q), _p(k), _p(q_weight), _p(k_weight), q.shape[0], q.shape[1],
                                kh, d, q.stride(0), q.stride(1),
                                0 if k is None else k.stride(0), 0 if k is None else k.stride(1),
                                eps, dt, _stream(dev)), "sgl_qk_rmsnorm")


# ---------------------------------------------------------------- residual path

def _dtype_code(*ts: torch.Tensor) -> int:
    dt = ts[0].dtype
    if any(t.dtype != dt for t in ts):
        raise ValueError("tensors must share one dtype")
    if dt == torch.bfloat16:
        return SGL_DTYPE_BF16
    if dt == torch.float16:
        return SGL_DTYPE_F16
    raise ValueError("the 16-bit kernels take bf16 or fp16")


def _rows2d(t: torch.Tensor, what: str) -> tuple[int, int, int]:
    """(rows, d, row stride) of a tensor viewed as [rows, d] with contiguous rows."""
    if t.dim() < 2 or t.stride(-1) != 1:
        raise ValueError(f"{what} must have rank >= 2 and a contiguous last dimension")
    d = t.shape[-1]
    rows = t.numel() // d if d else 0
    if t.dim() == 2:
        return rows, d, t.stride(0)
    if not t.is_contiguous():
        raise ValueError(f"{what} of rank > 2 must be contiguous")
    return rows, d, d


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float,
            out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """RMSNorm::forward (src/layers/normalization.cu:236-241); out=x is forward_inplace."""
    out = torch.empty_like(x) if out is None else out
    dev = _need_gpu(x, weight, out)
    rows, d, xs = _rows2d(x, "x")
    _, _, os_ = _rows2d(out, "out")
    if out.shape != x.shape or weight.numel() != d:
        raise ValueError("out must match x; weight must have d elements")
    _check(lib().sgl_rmsnorm(_p(out), _p(x), _p(weight), rows, d, xs, os_,
                             _dtype_code(x, weight, out), eps, _stream(dev)), "sgl_rmsnorm")
    return out


def fused_add_rmsnorm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                      eps: float) -> None:
    """RMSNorm::fused_add_forward_inplace (src/layers/normalization.cu:386-416), in place."""
    dev = _need_gpu(x, residual, weight)
    if x.dim() != 2 or residual.dim() != 2 or x.shape != residual.shape:
        raise ValueError("FusedAddRMSNorm expects rank-2 tensors of one shape")
    rows, d, xs = _rows2d(x, "x")
    _, _, rs = _rows2d(residual, "residual")
    if weight.numel() != d:
        raise ValueError("weight must have d elements")
    _check(lib().sgl_fused_add_rmsnorm(_p(x), _p(residual), _p(weight), rows, d, xs, rs,
                                       _dtype_code(x, residual, weight), eps, _stream(dev)),
           "sgl_fused_add_rmsnorm")


def _act_and_mul(fn: str, out: torch.Tensor, input: torch.Tensor) -> None:
    dev = _need_gpu(out, input)
    if input.dim() != 2 or out.dim() != 2 or input.stride(1) != 1 or out.stride(1) != 1:
        raise ValueError("input / out must be rank-2 with contiguous rows")
    d = input.shape[1] // 2
    if input.shape[1] != 2 * d or out.shape[0] != input.shape[0] or out.shape[1] != d:
        raise ValueError("input must be [T, 2d] and out [T, d]")
    _check(getattr(lib(), fn)(_p(out), _p(input), input.shape[0], d, input.stride(0),
                              out.stride(0), _dtype_code(input, out), _stream(dev)), fn)


def silu_and_mul(out: torch.Tensor, input: torch.Tensor) -> None:
    """silu_and_mul (src/layers/activation.cu:15-45)."""
    _act_and_mul("sgl_silu_and_mul", out, input)


def gelu_and_mul(out: torch.Tensor, input: torch.Tensor) -> None:
    """gelu_and_mul (src/layers/activation.cu:47-77)."""
    _act_and_mul("sgl_gelu_and_mul", out, input)


def rope(positions: torch.Tensor, q: torch.Tensor, k: torch.Tensor, cos_cache: torch.Tensor,
         sin_cache: torch.Tensor, rotary_dim: Optional[int] = None) -> None:
    """RotaryEmbedding::forward_inplace (src/layers/rotary_embedding.cu:96-178), in place."""
    dev = _need_gpu(positions, q, k, cos_cache, sin_cache)
    head_dim = q.shape[2]
    rd = head_dim if rotary_dim is None else rotary_dim
    if positions.dtype != torch.int32:
        raise ValueError("positions must be int32")
    dt = _dtype_code(q, k)
    _check(lib().sgl_rope(_p(q), _p(k), _p(cos_cache), _p(sin_cache), _p(positions),
                          positions.shape[0], q.shape[1], k.shape[1], rd, head_dim,
                          cos_cache.shape[1], q.stride(0), q.stride(1), k.stride(0), k.stride(1),
                          dt, _stream(dev)), "sgl_rope")


def fused_qknorm_rope_store(qkv: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                            q_weight: Optional[torch.Tensor], k_weight: Optional[torch.Tensor],
                            cos_cache: torch.Tensor, sin_cache: torch.Tensor,
                            positions: torch.Tensor, out_loc: torch.Tensor, num_qo_heads: int,
                            num_kv_heads: int, head_dim: int, eps: float,
                            write_k_back: bool = True) -> None:
    """write_k_back=False leaves qkv's k part untouched (SGL_FUSED_NO_K_WRITEBACK)."""
    dev = _need_gpu(qkv, k_cache, v_cache, q_weight, k_weight, cos_cache, sin_cache, positions,
                    out_loc)
    if qkv.dtype != torch.bfloat16 or qkv.dim() != 2 or qkv.stride(1) != 1:
        raise ValueError("qkv must be a 2-D bf16 tensor with a contiguous last dimension")
    if out_loc.dtype != torch.int32 or positions.dtype != torch.int32:
        raise ValueError("positions and out_loc must be int32")
    _check(lib().sgl_fused_qknorm_rope_store(
        _p(qkv), qkv.stride(0), _p(k_cache), _p(v_cache), _p(q_weight), _p(k_weight),
        _p(cos_cache), _p(sin_cache), _p(positions), _p(out_loc), qkv.shape[0], num_qo_heads,
        num_kv_heads, head_dim, eps, 0 if write_k_back else FUSED_NO_K_WRITEBACK, _stream(dev)),
        "sgl_fused_qknorm_rope_store")


# ---------------------------------------------------------------- attention

def decode_plan(kv_indptr_host: Sequence[int], num_qo_heads: int, num_kv_heads: int,
                head_dim: int) -> DecodePlan:
    arr = (ctypes.c_int32 * len(kv_indptr_host))(*[int(x) for x in kv_indptr_host])
    plan = DecodePlan()
    _check(lib().sgl_decode_plan(ctypes.cast(arr, ctypes.c_void_p), len(kv_indptr_host) - 1,
                                 num_qo_heads, num_kv_heads, head_dim, ctypes.byref(plan)),
           "sgl_decode_plan")
    return plan


def mixed_decode_cus(decode_kv_tokens: int, num_kv_heads: int, head_dim: int,
                     prefill_flops: float) -> int:
    """CU share for the decode rows of a mixed step (sgl_mixed_decode_cus)."""
    return lib().sgl_mixed_decode_cus(int(decode_kv_tokens), num_kv_heads, head_dim,
                                      float(prefill_flops))


def decode_plan_cus(kv_indptr_host: Sequence[int], num_qo_heads: int, num_kv_heads: int,
                    head_dim: int, decode_cus: int) -> DecodePlan:
    """A decode plan whose units fill decode_cus CUs (sgl_decode_plan_cus)."""
    arr = (ctypes.c_int32 * len(kv_indptr_host))(*[int(x) for x in kv_indptr_host])
    plan = DecodePlan()
    _check(lib().sgl_decode_plan_cus(ctypes.cast(arr, ctypes.c_void_p), len(kv_indptr_host) - 1,
                                     num_qo_heads, num_kv_heads, head_dim, decode_cus,
                                     ctypes.byref(plan)), "sgl_decode_plan_cus")
    return plan


def paged_mixed(plan: DecodePlan, q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                dec_indices: torch.Tensor, dec_kv_indptr: torch.Tensor,
                dec_q_rows: Optional[torch.Tensor], pre_indices: torch.Tensor,
                pre_qo_indptr: torch.Tensor, pre_kv_indptr: torch.Tensor,
                pre_q_start: Optional[torch.Tensor], pre_max_qo_len: int, o: torch.Tensor,
                workspace: torch.Tensor, sm_scale: Optional[float] = None) -> None:
    """Decode rows and prefill rows of one mixed batch in one launch (sgl_paged_mixed)."""
    dev = _need_gpu(q, k_cache, v_cache, dec_indices, dec_kv_indptr, dec_q_rows, pre_indices,
                    pre_qo_indptr, pre_kv_indptr, pre_q_start, o, workspace)
    if q.dtype != torch.bfloat16 or k_cache.dtype != torch.bfloat16 or o.dtype != torch.bfloat16:
        raise ValueError("attention supports bf16 q / KV / o only")
    hq, D = q.shape[1], q.shape[2]
    hkv = k_cache.shape[1]
    ss, sh = _kv_strides(k_cache)
    if v_cache.stride() != k_cache.stride():
        raise ValueError("K and V caches must share strides")
    scale = 1.0 / math.sqrt(D) if sm_scale is None else sm_scale
    ws_bytes = workspace.numel() * workspace.element_size()
    _check(lib().sgl_paged_mixed(ctypes.byref(plan), _p(q), q.stride(0), q.stride(1),
                                 _p(k_cache), _p(v_cache), ss, sh, _p(dec_indices),
                                 _p(dec_kv_indptr), _p(dec_q_rows), dec_kv_indptr.shape[0] - 1,
                                 _p(pre_indices), _p(pre_qo_indptr), _p(pre_kv_indptr),
                                 _p(pre_q_start), pre_qo_indptr.shape[0] - 1, pre_max_qo_len,
                                 hq, hkv, D, scale, _p(o), o.stride(0), o.stride(1),
                                 _p(workspace), ws_bytes, _stream(dev)), "sgl_paged_mixed")


def decode_plan_check(plan: DecodePlan, kv_indptr_host: Sequence[int]) -> int:
    """SGL_OK (0) when the batch fits the plan, SGL_ERR_CAPACITY (-3) when not."""
    arr = (ctypes.c_int32 * len(kv_indptr_host))(*[int(x) for x in kv_indptr_host])
    return lib().sgl_decode_plan_check(ctypes.byref(plan), ctypes.cast(arr, ctypes.c_void_p),
                                       len(kv_indptr_host) - 1)


def decode_workspace(plan: DecodePlan, device: torch.device) -> torch.Tensor:
    """Allocates the split-KV workspace a plan needs."""
    return torch.empty(int(plan.workspace_bytes), dtype=torch.uint8, device=device)


def decode_status(workspace: Optional[torch.Tensor]) -> int:
    """Status word of the last decode call on this workspace (waits for the
    stream); None reads the no-alloc entry point's scratch on the current
    device."""
    dev = _need_gpu(workspace) if workspace is not None else _need_gpu()
    st = ctypes.c_int32(-100)
    _check(lib().sgl_decode_status(_p(workspace), ctypes.byref(st), _stream(dev)),
           "sgl_decode_status")
    return st.value


def _kv_strides(k_cache: torch.Tensor):
    if k_cache.dim() != 3 or k_cache.stride(2) != 1:
        raise ValueError("KV cache layer must be [slots, Hkv, D] with a contiguous last dim")
    return k_cache.stride(0), k_cache.stride(1)


def paged_decode(plan: DecodePlan, q: torch.Tensor, k_cache: torch.Tensor,
                 v_cache: torch.Tensor, indices: torch.Tensor, kv_indptr: torch.Tensor,
                 o: torch.Tensor, workspace: Optional[torch.Tensor],
                 sm_scale: Optional[float] = None,
                 q_indptr: Optional[torch.Tensor] = None) -> None:
    dev = _need_gpu(q, k_cache, v_cache, indices, kv_indptr, o, workspace, q_indptr)
    if q.dtype != torch.bfloat16 or k_cache.dtype != torch.bfloat16 or o.dtype != torch.bfloat16:
        raise ValueError("decode supports bf16 q / KV / o only")
    hq, D = q.shape[1], q.shape[2]
    hkv = k_cache.shape[1]
    ss, sh = _kv_strides(k_cache)
    if v_cache.stride() != k_cache.stride():
        raise ValueError("K and V caches must share strides")
    B = kv_indptr.shape[0] - 1
    scale = 1.0 / math.sqrt(D) if sm_scale is None else sm_scale
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _check(lib().sgl_paged_decode(ctypes.byref(plan), _p(q), q.stride(0), q.stride(1),
                                  _p(k_cache), _p(v_cache), ss, sh, _p(indices), _p(kv_indptr),
                                  _p(q_indptr), B, hq, hkv, D, scale, _p(o), o.stride(0),
                                  o.stride(1), _p(workspace), ws_bytes, _stream(dev)),
           "sgl_paged_decode")


DECODE_SCRATCH_BYTES = 32 << 20  # SGL_DECODE_SCRATCH_BYTES


def paged_decode_noalloc(plan: DecodePlan, q: torch.Tensor, k_cache: torch.Tensor,
                         v_cache: torch.Tensor, indices: torch.Tensor, kv_indptr: torch.Tensor,
                         o: torch.Tensor, sm_scale: Optional[float] = None,
                         q_indptr: Optional[torch.Tensor] = None) -> None:
    """sgl_paged_decode with the library's own device scratch (no workspace)."""
    dev = _need_gpu(q, k_cache, v_cache, indices, kv_indptr, o, q_indptr)
    if q.dtype != torch.bfloat16 or k_cache.dtype != torch.bfloat16 or o.dtype != torch.bfloat16:
        raise ValueError("decode supports bf16 q / KV / o only")
    hq, D = q.shape[1], q.shape[2]
    hkv = k_cache.shape[1]
    ss, sh = _kv_strides(k_cache)
    if v_cache.stride() != k_cache.stride():
        raise ValueError("K and V caches must share strides")
    B = kv_indptr.shape[0] - 1
    scale = 1.0 / math.sqrt(D) if sm_scale is None else sm_scale
    _check(lib().sgl_paged_decode_noalloc(ctypes.byref(plan), _p(q), q.stride(0), q.stride(1),
                                          _p(k_cache), _p(v_cache), ss, sh, _p(indices),
                                          _p(kv_indptr), _p(q_indptr), B, hq, hkv, D, scale,
                                          _p(o), o.stride(0), o.stride(1), _stream(dev)),
           "sgl_paged_decode_noalloc")


def paged_prefill(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  indices: torch.Tensor, qo_indptr: torch.Tensor, kv_indptr: torch.Tensor,
                  max_qo_len: int, o: torch.Tensor, sm_scale: Optional[float] = None,
                  q_start: Optional[torch.Tensor] = None) -> None:
    dev = _need_gpu(q, k_cache, v_cache, indices, qo_indptr, kv_indptr, o, q_start)
    if q.dtype != torch.bfloat16 or k_cache.dtype != torch.bfloat16 or o.dtype != torch.bfloat16:
        raise ValueError("prefill supports bf16 q / KV / o only")
    hq, D = q.shape[1], q.shape[2]
    hkv = k_cache.shape[1]
    ss, sh = _kv_strides(k_cache)
    if v_cache.stride() != k_cache.stride():
        raise ValueError("K and V caches must share strides")
    B = qo_indptr.shape[0] - 1
    scale = 1.0 / math.sqrt(D) if sm_scale is None else sm_scale
    _check(lib().sgl_paged_prefill(_p(q), q.stride(0), q.stride(1), _p(k_cache), _p(v_cache), ss,
                                   sh, _p(indices), _p(qo_indptr), _p(kv_indptr), _p(q_start), B,
                                   max_qo_len,
                                   hq, hkv, D, scale, _p(o), o.stride(0), o.stride(1),
                                   _stream(dev)), "sgl_paged_prefill")


# ---------------------------------------------------------------- sampling

def softmax_temperature(logits: torch.Tensor, temperatures: Optional[torch.Tensor] = None,
                        temperature: float = 1.0,
                        out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The probabilities Sampler::sample hands to the sampling kernels:
    softmax(logits.float() / temperatures, -1) (src/engine/engine.cc:306-308),
    one pass. logits: [batch, vocab] bf16, fp16 or fp32 with contiguous rows;
    temperatures: float32 [batch] (or [batch, 1]), else the scalar
    temperature. Returns (or fills) float32 [batch, vocab]."""
    dev = _need_gpu(logits, temperatures, out)
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be [batch, vocab] with contiguous rows")
    codes = {torch.bfloat16: SGL_DTYPE_BF16, torch.float16: SGL_DTYPE_F16,
             torch.float32: SGL_DTYPE_F32}
    if logits.dtype not in codes:
        raise ValueError("logits must be bf16, fp16 or float32")
    b, v = logits.shape
    if temperatures is not None:
        if temperatures.dtype != torch.float32 or temperatures.numel() != b:
            raise ValueError("temperatures must be float32 with one value per row")
        temperatures = temperatures.reshape(b).contiguous()
    elif not temperature > 0:
        raise ValueError("temperature must be positive")
    if out is None:
        out = torch.empty((b, v), dtype=torch.float32, device=dev)
    elif out.shape != (b, v) or out.dtype != torch.float32 or out.stride(1) != 1:
        raise ValueError("out must be float32 [batch, vocab] with contiguous rows")
    _check(lib().sgl_softmax_temperature(_p(out), out.stride(0), _p(logits), logits.stride(0),
                                         codes[logits.dtype], _p(temperatures),
                                         float(temperature), b, v, _stream(dev)),
           "sgl_softmax_temperature")
    return out


def sampling_from_logits(logits: torch.Tensor, uniform_samples: torch.Tensor, mode: str,
                         temperatures: Optional[torch.Tensor] = None, temperature: float = 1.0,
                         top_k: Optional[torch.Tensor] = None, top_k_val: int = 0,
                         top_p: Optional[torch.Tensor] = None, top_p_val: float = 0.0):
    """Sampler::sample's probabilities and draw in one launch (engine.cc:306-333):
    mode "plain" (uniform [batch]), "top_k" (top_k float32 [batch]), "top_p",
    "top_k_top_p" (top_k int32 [batch]); the filtered modes take uniform
    [max_rounds, batch]. Returns (samples int32 [batch], success bool [batch]
    or None for the plain draw); equal to softmax_temperature followed by
    the mode's draw from probabilities."""
    m = {"plain": 0, "top_k": 1, "top_p": 2, "top_k_top_p": 3}[mode]
    dev = _need_gpu(logits, uniform_samples, temperatures, top_k, top_p)
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be [batch, vocab] with contiguous rows")
    codes = {torch.bfloat16: SGL_DTYPE_BF16, torch.float16: SGL_DTYPE_F16,
             torch.float32: SGL_DTYPE_F32}
    if logits.dtype not in codes:
        raise ValueError("logits must be bf16, fp16 or float32")
    b, v = logits.shape
    dims = 1 if m == 0 else 2
    if (uniform_samples.dtype != torch.float32 or not uniform_samples.is_contiguous()
            or uniform_samples.dim() != dims or uniform_samples.shape[-1] != b):
        raise ValueError("uniform_samples must be contiguous float32 "
                         + ("[batch]" if dims == 1 else "[max_rounds, batch]"))
    if temperatures is not None:
        temperatures = temperatures.to(torch.float32).reshape(b).contiguous()
    elif not temperature > 0:
        raise ValueError("temperature must be positive")
    tkf = _opt(top_k, torch.float32, b, "top_k") if m == 1 else None
    tki = _opt(top_k, torch.int32, b, "top_k") if m == 3 else None
    tp = _opt(top_p, torch.float32, b, "top_p") if m >= 2 else None
    out = torch.empty(b, dtype=torch.int32, device=dev)
    succ = None if m == 0 else torch.empty(b, dtype=torch.bool, device=dev)
    rounds = 1 if m == 0 else uniform_samples.shape[0]
    _check(lib().sgl_sampling_from_logits(_p(logits), logits.stride(0), codes[logits.dtype],
                                          _p(temperatures), float(temperature),
                                          _p(uniform_samples), m, _p(tkf), _p(tki),
                                          int(top_k_val), _p(tp), float(top_p_val), _p(out),
                                          _p(succ), b, v, rounds, _stream(dev)),
           "sgl_sampling_from_logits")
    return out, succ


def _check_probs(probs: torch.Tensor, uniform: torch.Tensor, dims: int) -> None:
    if probs.dim() != 2 or not probs.is_contiguous() or probs.dtype != torch.float32:
        raise ValueError("probs must be a contiguous float32 [batch, vocab] tensor")
    if uniform.dtype != torch.float32 or not uniform.is_contiguous() or uniform.dim() != dims:
        raise ValueError("uniform_samples must be contiguous float32 with "
                         + ("shape [batch]" if dims == 1 else "shape [max_rounds, batch]"))
    if uniform.shape[-1] != probs.shape[0]:
        raise ValueError("uniform_samples must cover every row")


def _opt(t: Optional[torch.Tensor], dtype, n: int, what: str):
    if t is None:
        return None
    if t.dtype != dtype or not t.is_contiguous() or t.numel() != n:
        raise ValueError(f"{what} must be a contiguous {dtype} tensor with shape [batch]")
    return t


def sampling_from_probs(probs: torch.Tensor, uniform_samples: torch.Tensor,
                        deterministic: bool = False) -> torch.Tensor:
    """flashinfer_sample_from_probs (src/engine/sampling.cu:65-84)."""
    dev = _need_gpu(probs, uniform_samples)
    _check_probs(probs, uniform_samples, 1)
    out = torch.empty(probs.shape[0], dtype=torch.int32, device=dev)
    _check(lib().sgl_sampling_from_probs(_p(probs), _p(uniform_samples), _p(out), probs.shape[0],
                                         probs.shape[1], int(deterministic), _stream(dev)),
           "sgl_sampling_from_probs")
    return out


def top_k_sampling_from_probs(probs, uniform_samples, top_k: Optional[torch.Tensor],
                              top_k_value: int = 0, deterministic: bool = False):
    """flashinfer_top_k_sample_from_probs (src/engine/sampling.cu:86-116): top_k is
    float32 [batch] or None (then top_k_value). Returns (samples, success)."""
    dev = _need_gpu(probs, uniform_samples, top_k)
    _check_probs(probs, uniform_samples, 2)
    B = probs.shape[0]
    top_k = _opt(top_k, torch.float32, B, "top_k")
    out = torch.empty(B, dtype=torch.int32, device=dev)
    ok = torch.empty(B, dtype=torch.bool, device=dev)
    _check(lib().sgl_top_k_sampling_from_probs(_p(probs), _p(uniform_samples), _p(out), _p(ok),
                                               _p(top_k), B, int(top_k_value), probs.shape[1],
                                               uniform_samples.shape[0], int(deterministic),
                                               _stream(dev)), "sgl_top_k_sampling_from_probs")
    return out, ok


def top_p_sampling_from_probs(probs, uniform_samples, top_p: Optional[torch.Tensor],
                              top_p_value: float = 0.0, deterministic: bool = False):
    """flashinfer_top_p_sample_from_probs (src/engine/sampling.cu:118-148)."""
    dev = _need_gpu(probs, uniform_samples, top_p)
    _check_probs(probs, uniform_samples, 2)
    B = probs.shape[0]
    top_p = _opt(top_p, torch.float32, B, "top_p")
    out = torch.empty(B, dtype=torch.int32, device=dev)
    ok = torch.empty(B, dtype=torch.bool, device=dev)
    _check(lib().sgl_top_p_sampling_from_probs(_p(probs), _p(uniform_samples), _p(out), _p(ok),
                                               _p(top_p), B, float(top_p_value), probs.shape[1],
                                               uniform_samples.shape[0], int(deterministic),
                                               _stream(dev)), "sgl_top_p_sampling_from_probs")
    return out, ok


def top_k_top_p_sampling_from_probs(probs, uniform_samples, top_k: Optional[torch.Tensor],
                                    top_k_value: int, top_p: Optional[torch.Tensor],
                                    top_p_value: float, deterministic: bool = False):
    """flashinfer_top_k_top_p_sample_from_probs (src/engine/sampling.cu:150-192):
    top_k is int32 [batch] here, as the reference passes it."""
    dev = _need_gpu(probs, uniform_samples, top_k, top_p)
    _check_probs(probs, uniform_samples, 2)
    B = probs.shape[0]
    top_k = _opt(top_k, torch.int32, B, "top_k")
    top_p = _opt(top_p, torch.float32, B, "top_p")
    out = torch.empty(B, dtype=torch.int32, device=dev)
    ok = torch.empty(B, dtype=torch.bool, device=dev)
    _check(lib().sgl_top_k_top_p_sampling_from_probs(
        _p(probs), _p(uniform_samples), _p(top_k), _p(top_p), _p(out), _p(ok), B,
        int(top_k_value), float(top_p_value), probs.shape[1], uniform_samples.shape[0],
        int(deterministic), _stream(dev)), "sgl_top_k_top_p_sampling_from_probs")
    return out, ok
