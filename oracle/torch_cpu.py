"""LibTorch-CPU fp32 attention — the CPU baseline leg, TEST INFRASTRUCTURE ONLY.

The reference has no CPU attention path of its own; the baseline it plans for
this path is a LibTorch-CPU fp32 restatement on the same inputs: per request
and per kv-head group, gather the request's K/V rows from the pool, then
matmul -> (causal-masked) softmax -> matmul (the semantics of
src/attention/flashinfer_backend.cu:553-595 for decode and :596-679 for
causal prefill, bottom-right aligned). PyTorch's CPU operators are LibTorch's.
The fused store is the same elementwise operations plus index_put_: q/k
RMSNorm (src/layers/normalization.cu:138-170, bf16-rounded), NeoX RoPE
(src/layers/rotary_embedding.cu:50-66, half-width cos/sin table), then the
K/V store (src/kvcache/mha_kvcache.cu:13-41).
Only bench.py's cpu_baseline leg and tests/ use this module, never the
product path. Tensors are CPU torch tensors: q [rows, Hq, D] bf16, caches
[slots, Hkv, D] bf16, index arrays int64.
"""
from __future__ import annotations

import os
import platform
import time

import torch

QUERY_BLOCK = 512  # query tokens per score block (bounds the [Hkv, rows, kv] scores)


def decode(q, k_cache, v_cache, indices, kv_indptr, sm_scale, out=None):
    """o[r, h] = softmax(q[r, h] . K[idx] * scale) . V[idx], fp32; returns fp32 [B, Hq, D]."""
    B, hq, D = q.shape
    hkv = k_cache.shape[1]
    G = hq // hkv
    out = torch.empty((B, hq, D), dtype=torch.float32) if out is None else out
    for r in range(B):
        b, e = int(kv_indptr[r]), int(kv_indptr[r + 1])
        if e <= b:
            out[r].zero_()
            continue
        idx = indices[b:e]
        k = k_cache.index_select(0, idx).float().permute(1, 2, 0)   # [Hkv, D, n]
        v = v_cache.index_select(0, idx).float().permute(1, 0, 2)   # [Hkv, n, D]
        qq = q[r].float().view(hkv, G, D)
        p = torch.softmax(torch.matmul(qq, k) * sm_scale, dim=-1)   # [Hkv, G, n]
        out[r] = torch.matmul(p, v).reshape(hq, D)
    return out


def prefill(q, k_cache, v_cache, indices, qo_indptr, kv_indptr, sm_scale, out=None):
    """Causal prefill (query i of a request sees kv j <= i + kv_len - qo_len); fp32 out."""
    rows, hq, D = q.shape
    hkv = k_cache.shape[1]
    G = hq // hkv
    out = torch.empty((rows, hq, D), dtype=torch.float32) if out is None else out
    for r in range(len(qo_indptr) - 1):
        q0, q1 = int(qo_indptr[r]), int(qo_indptr[r + 1])
        b, e = int(kv_indptr[r]), int(kv_indptr[r + 1])
        qo, kv = q1 - q0, e - b
        if qo <= 0:
            continue
        if kv <= 0:
            out[q0:q1].zero_()
            continue
        idx = indices[b:e]
        k = k_cache.index_select(0, idx).float().permute(1, 2, 0)   # [Hkv, D, kv]
        v = v_cache.index_select(0, idx).float().permute(1, 0, 2)   # [Hkv, kv, D]
        off = kv - qo
        j = torch.arange(kv)
        for t0 in range(0, qo, QUERY_BLOCK):
            t1 = min(qo, t0 + QUERY_BLOCK)
            n = t1 - t0
            qq = q[q0 + t0:q0 + t1].float().view(n, hkv, G, D).permute(1, 0, 2, 3)
            s = torch.matmul(qq.reshape(hkv, n * G, D), k) * sm_scale   # [Hkv, n G, kv]
            i = torch.arange(t0, t1).repeat_interleave(G)
            s.masked_fill_(j[None, :] > (i[:, None] + off), float("-inf"))
            p = torch.softmax(s, dim=-1)
            o = torch.matmul(p, v).view(hkv, n, G, D).permute(1, 0, 2, 3)
            out[q0 + t0:q0 + t1] = o.reshape(n, hq, D)
    return out


def fused_qknorm_rope_store(qkv, k_cache, v_cache, q_weight, k_weight, cos, sin, positions,
                            out_loc, num_qo_heads, num_kv_heads, eps):
    """In place: q part of qkv [T, (Hq + 2 Hkv) D] bf16 normalised and rotated;
    k normalised, rotated and stored at k_cache[out_loc]; v stored raw at
    v_cache[out_loc]. cos/sin fp32 [max_pos, D/2]; positions, out_loc int64."""
    T = qkv.shape[0]
    D = q_weight.shape[0]
    hq, hkv = num_qo_heads, num_kv_heads
    q = qkv[:, :hq * D].view(T, hq, D)
    k = qkv[:, hq * D:(hq + hkv) * D].view(T, hkv, D)
    v = qkv[:, (hq + hkv) * D:].view(T, hkv, D)
    c = cos.index_select(0, positions).unsqueeze(1)
    s = sin.index_select(0, positions).unsqueeze(1)

    def norm(x, w):
        xf = x.float()
        r = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
        return (xf * r * w.float()).to(torch.bfloat16)

    def rope(x):
        xf = x.float()
        x1, x2 = xf[..., :D // 2], xf[..., D // 2:]
        return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], -1).to(torch.bfloat16)

    q.copy_(rope(norm(q, q_weight)))
    k_cache.index_put_((out_loc,), rope(norm(k, k_weight)))
    v_cache.index_put_((out_loc,), v)


def host_info() -> dict:
    """CPU model and the threads LibTorch uses."""
    model = platform.processor() or "unknown"
    ident = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key = line.split(":", 1)[0].strip()
                if key == "model name":
                    model = line.split(":", 1)[1].strip()
                elif key in ("cpu family", "model", "stepping", "cpu MHz") and key not in ident:
                    ident[key] = line.split(":", 1)[1].strip()
                elif not line.strip() and ident:
                    break  # first processor's block only
    except OSError:
        pass
    if ident:  # a virtualised host may report only the vendor in "model name"
        model += " (family {}, model {}, stepping {}, {} MHz)".format(
            ident.get("cpu family", "?"), ident.get("model", "?"), ident.get("stepping", "?"),
            ident.get("cpu MHz", "?"))
    return {"cpu_model": model, "threads": torch.get_num_threads(),
            "host_cpus": len(os.sched_getaffinity(0))}


def median_time(fn, runs: int = 5) -> tuple[float, list[float]]:
    """One warm-up call, then the median wall time of `runs` calls (seconds)."""
    fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts_sorted = sorted(ts)
    return ts_sorted[len(ts) // 2], ts
