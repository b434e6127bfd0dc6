"""ctypes front end of the CPU oracle (oracle.c) — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
this module, always as the checker and never as the thing measured or
shipped. Arrays are numpy; bf16 is carried as uint16 bit patterns.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle.so"

_lib = None


def build() -> Path:
    res = subprocess.run(["make", "-C", str(ORACLE_DIR), "-s"], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stdout}\n{res.stderr}")
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        _lib.oracle_threads.restype = ctypes.c_int
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    return a.ctypes.data_as(ctypes.c_void_p)


def _row_stride(a: np.ndarray) -> int:
    """Row stride in elements of a 2-D array whose rows are contiguous."""
    assert a.ndim == 2
    if a.size == 0:
        return a.shape[1]
    assert a.strides[1] == a.itemsize, "rows must be contiguous"
    return a.strides[0] // a.itemsize


I64 = ctypes.c_int64
F32 = ctypes.c_float


# ---------------------------------------------------------------- bf16 helpers

def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_bf16(_p(x), _p(out), I64(x.size))
    return out


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def threads() -> int:
    return lib().oracle_threads()


def set_threads(n: int) -> None:
    lib().oracle_set_threads(ctypes.c_int(n))


# ---------------------------------------------------------------- kernels

def store_kv(k_cache, v_cache, k, v, out_loc) -> None:
    """k_cache/v_cache: contiguous uint16 [slots, elems]; k/v: uint16 [T, >= elems]
    row-strided views (e.g. slices of a qkv row); the first elems of each row are stored."""
    out_loc = np.ascontiguousarray(out_loc, dtype=np.int64)
    assert k_cache.flags["C_CONTIGUOUS"] and v_cache.flags["C_CONTIGUOUS"]
    elems = k_cache.shape[1]
    assert k.shape[1] >= elems and v.shape[1] >= elems
    lib().oracle_store_kv(_p(k_cache), _p(v_cache), _p(k), _p(v), _p(out_loc), I64(len(out_loc)),
                          I64(elems), I64(_row_stride(k)), I64(_row_stride(v)))


def build_indices(page_table, table_indices, kv_indptr) -> np.ndarray:
    pt = np.ascontiguousarray(page_table, dtype=np.int32)
    ti = np.ascontiguousarray(table_indices, dtype=np.int32)
    ip = np.ascontiguousarray(kv_indptr, dtype=np.int32)
    out = np.zeros(int(ip[-1]) if len(ip) else 0, dtype=np.int32)
    lib().oracle_build_indices(_p(pt), I64(pt.shape[0]), I64(pt.shape[1]), I64(pt.shape[1]),
                               _p(ti), _p(ip), _p(out), ctypes.c_int(len(ti)))
    return out


def write_token_pool(pool, req, pos, tok) -> None:
    req = np.ascontiguousarray(req, np.int32)
    pos = np.ascontiguousarray(pos, np.int32)
    tok = np.ascontiguousarray(tok, np.int32)
    lib().oracle_write_token_pool(_p(pool), I64(pool.shape[0]), I64(pool.shape[1]),
                                  I64(pool.shape[1]), _p(req), _p(pos), _p(tok), I64(len(tok)))


def gather_int32_2d(table, req, pos) -> np.ndarray:
    table = np.ascontiguousarray(table, np.int32)
    req = np.ascontiguousarray(req, np.int32)
    pos = np.ascontiguousarray(pos, np.int32)
    out = np.empty(len(req), np.int32)
    lib().oracle_gather_int32_2d(_p(table), I64(table.shape[0]), I64(table.shape[1]),
                                 I64(table.shape[1]), _p(req), _p(pos), _p(out), I64(len(req)))
    return out


def write_page_table(table, page_starts, alloc, page_size: int) -> int:
    """In place on the int32 [rows, cols] table; alloc is [n, 3] (table_idx,
    first_page, last_page). Returns the page starts consumed (-1 if short)."""
    ps = np.ascontiguousarray(page_starts, np.int32)
    al = np.ascontiguousarray(np.asarray(alloc, np.int32).reshape(-1, 3))
    fn = lib().oracle_write_page_table
    fn.restype = ctypes.c_int64
    return fn(_p(table), I64(table.shape[0]), I64(table.shape[1]), I64(table.shape[1]), _p(ps),
              I64(len(ps)), _p(al), I64(al.shape[0]), ctypes.c_int(page_size))


def pages_to_tokens(page_starts, page_size: int) -> np.ndarray:
    ps = np.ascontiguousarray(page_starts, np.int32)
    out = np.empty(len(ps) * page_size, np.int32)
    lib().oracle_pages_to_tokens(_p(ps), I64(len(ps)), ctypes.c_int(page_size), _p(out))
    return out


def cos_sin_cache(max_pos: int, rotary_dim: int, base: float):
    cos = np.empty((max_pos, rotary_dim // 2), np.float32)
    sin = np.empty_like(cos)
    lib().oracle_cos_sin_cache(_p(cos), _p(sin), I64(max_pos), ctypes.c_int(rotary_dim), F32(base))
    return cos, sin


def qk_rmsnorm(q, k, qw, kw, eps: float, dtype: str = "bf16") -> None:
    """In place on uint16 bit patterns (bf16 or fp16) q [T, Hq, D], k [T, Hk, D]
    (contiguous)."""
    T, qh, d = q.shape
    kh = 0 if k is None else k.shape[1]
    lib().oracle_qk_rmsnorm(_p(q), _p(k), _p(qw), _p(kw), I64(T), I64(qh), I64(kh), I64(d),
                            I64(qh * d), I64(d), I64(kh * d), I64(d), F32(eps),
                            ctypes.c_int(_DT[dtype]))


def rope(q, k, cos, sin, positions, rotary_dim: int | None = None, dtype: str = "bf16") -> None:
    T, qh, d = q.shape
    kh = k.shape[1]
    rd = d if rotary_dim is None else rotary_dim
    pos = np.ascontiguousarray(positions, np.int32)
    rc = lib().oracle_rope(_p(q), _p(k), _p(cos), _p(sin), _p(pos), I64(T), I64(qh), I64(kh),
                           I64(rd), I64(cos.shape[1]), I64(qh * d), I64(d), I64(kh * d), I64(d),
                           ctypes.c_int(_DT[dtype]))
    assert rc == 0


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> IEEE binary16 bit patterns (round to nearest even), the oracle's encoding."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().oracle_f16_bits(_p(x), _p(out), I64(x.size))
    return out


def f16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(b, np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().oracle_f16_values(_p(b), _p(out), I64(b.size))
    return out


def decode(q, k_cache, v_cache, indices, kv_indptr, sm_scale: float, q_indptr=None) -> np.ndarray:
    """q: uint16 [rows, Hq, D]; caches: uint16 [slots, Hkv, D]. Returns fp32 [rows, Hq, D]."""
    rows, hq, D = q.shape
    hkv = k_cache.shape[1]
    B = len(kv_indptr) - 1
    out = np.zeros((rows, hq, D), np.float32)
    qi = None if q_indptr is None else np.ascontiguousarray(q_indptr, np.int32)
    lib().oracle_decode(_p(np.ascontiguousarray(q)), I64(hq * D), I64(D),
                        _p(k_cache), _p(v_cache), I64(hkv * D), I64(D),
                        _p(np.ascontiguousarray(indices, np.int32)),
                        _p(np.ascontiguousarray(kv_indptr, np.int32)), _p(qi), ctypes.c_int(B),
                        ctypes.c_int(hq), ctypes.c_int(hkv), ctypes.c_int(D), F32(sm_scale),
                        _p(out))
    return out


def prefill(q, k_cache, v_cache, indices, qo_indptr, kv_indptr, sm_scale: float) -> np.ndarray:
    rows, hq, D = q.shape
    hkv = k_cache.shape[1]
    B = len(qo_indptr) - 1
    out = np.zeros((rows, hq, D), np.float32)
    lib().oracle_prefill(_p(np.ascontiguousarray(q)), I64(hq * D), I64(D),
                         _p(k_cache), _p(v_cache), I64(hkv * D), I64(D),
                         _p(np.ascontiguousarray(indices, np.int32)),
                         _p(np.ascontiguousarray(qo_indptr, np.int32)),
                         _p(np.ascontiguousarray(kv_indptr, np.int32)), ctypes.c_int(B),
                         ctypes.c_int(hq), ctypes.c_int(hkv), ctypes.c_int(D), F32(sm_scale),
                         _p(out))
    return out


# ---------------------------------------------------------------- residual path
# Values are fp32 arrays holding numbers representable in T (bf16 or fp16);
# dtype is "bf16" or "fp16". Outputs are fp32 arrays of T-rounded values.

_DT = {"bf16": 0, "fp16": 1}


def _f32c(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def rmsnorm(x, w, eps: float, dtype: str) -> np.ndarray:
    """RMSNorm::forward (src/layers/normalization.cu:236-269) on [rows, d]."""
    x, w = _f32c(x), _f32c(w)
    out = np.empty_like(x)
    rows, d = x.shape
    lib().oracle_rmsnorm(_p(x), _p(w), _p(out), I64(rows), I64(d), F32(eps),
                         ctypes.c_int(_DT[dtype]))
    return out


def fused_add_rmsnorm(x, residual, w, eps: float, dtype: str):
    """RMSNorm::fused_add_forward_inplace (src/layers/normalization.cu:386-416).
    Returns (x_out, residual_out)."""
    x, r, w = _f32c(x), _f32c(residual), _f32c(w)
    xo, ro = np.empty_like(x), np.empty_like(x)
    rows, d = x.shape
    lib().oracle_fused_add_rmsnorm(_p(x), _p(r), _p(w), _p(xo), _p(ro), I64(rows), I64(d),
                                   F32(eps), ctypes.c_int(_DT[dtype]))
    return xo, ro


def act_and_mul(inp, act: str, dtype: str) -> np.ndarray:
    """silu_and_mul / gelu_and_mul (src/layers/activation.cu:8-77) on [T, 2d] -> [T, d]."""
    inp = _f32c(inp)
    T, d2 = inp.shape
    out = np.empty((T, d2 // 2), np.float32)
    lib().oracle_act_and_mul(_p(inp), _p(out), I64(T), I64(d2 // 2),
                             ctypes.c_int({"silu": 0, "gelu": 1}[act]), ctypes.c_int(_DT[dtype]))
    return out


def round_t(x, dtype: str) -> np.ndarray:
    """The oracle's rounding to the nearest T value (ties to even), as fp32."""
    x = _f32c(x)
    out = np.empty_like(x)
    lib().oracle_round_t(_p(x), _p(out), I64(x.size), ctypes.c_int(_DT[dtype]))
    return out


# ---------------------------------------------------------------- sampling

def sample(probs, uniform, mode: str, top_k=None, top_k_val: int = 0, top_p=None,
           top_p_val: float = 0.0):
    """src/engine/sampling.cu:65-194. probs fp32 [B, d]; uniform fp32 [B] (plain)
    or [rounds, B]. top_k: fp32 [B] for "top_k", int32 [B] for "top_k_top_p".
    Returns (samples int32 [B], success bool [B] or None)."""
    probs = _f32c(probs)
    uniform = _f32c(uniform)
    B, d = probs.shape
    m = {"plain": 0, "top_k": 1, "top_p": 2, "top_k_top_p": 3}[mode]
    rounds = 1 if m == 0 else uniform.shape[0]
    out = np.empty(B, np.int32)
    succ = None if m == 0 else np.empty(B, np.uint8)
    tkf = _f32c(top_k) if (top_k is not None and m == 1) else None
    tki = np.ascontiguousarray(top_k, np.int32) if (top_k is not None and m == 3) else None
    tp = _f32c(top_p) if top_p is not None else None
    lib().oracle_sample(_p(probs), _p(uniform), _p(out), _p(succ), I64(B), I64(d),
                        ctypes.c_int(rounds), ctypes.c_int(m), _p(tkf), _p(tki),
                        ctypes.c_int(top_k_val), _p(tp), F32(top_p_val))
    return out, (None if succ is None else succ.astype(bool))


def softmax_temperature(logits_f32: np.ndarray, temperatures) -> np.ndarray:
    """The probabilities of Sampler::sample (src/engine/engine.cc:306-308):
    y = logits.to(float32) / temperatures in float32 (an IEEE division per
    element, as LibTorch computes it), then softmax over the vocabulary,
    here in float64 (max-shifted). logits_f32: [batch, vocab] float32 (the
    widened logits); temperatures: [batch] or a scalar. Returns float64."""
    x = np.ascontiguousarray(logits_f32, dtype=np.float32)
    t = np.asarray(temperatures, dtype=np.float32).reshape(-1, 1) if np.ndim(temperatures) \
        else np.float32(temperatures)
    y = (x / t).astype(np.float64)  # float32 division, then widened
    y = y - y.max(axis=1, keepdims=True)
    e = np.exp(y)
    return e / e.sum(axis=1, keepdims=True)
