"""Seeded synthetic inputs for the attention hot path (the five benchmark configurations).

Page tables are built the way the reference's scheduler builds them:
CacheManager hands out page starts (slot of a page's first token,
src/scheduler/prefill.cc:55-67,88-101) from a free list — here a seeded
random permutation of pages — and write_page_table expands each page to
page_size consecutive token slots in the request's row
(src/scheduler/prefill.cc:144-206). Prefill metadata follows
FlashInferBackend::prepare_metadata (src/attention/flashinfer_backend.cu:466-519):
qo_len = max(1, extend_len), kv_len = device_len, indices = the row prefix.
Positions of the new tokens are cached_len .. device_len-1 and out_loc is
the page-table gather at those positions (src/scheduler/scheduler.cc:295-332).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np


def align_up(x: int, a: int) -> int:
    return (x + a - 1) // a * a


@dataclass
class PagedBatch:
    cached_lens: np.ndarray  # [B] int32
    device_lens: np.ndarray  # [B] int32 (kv_len)
    page_size: int
    num_pages: int           # allocatable pages (the pool has one spare page after them)
    page_table: np.ndarray   # [B + 1, W] int32, token-granular slots
    table_idx: np.ndarray    # [B] int32
    qo_indptr: np.ndarray
    kv_indptr: np.ndarray
    indices: np.ndarray      # [sum kv] int32
    positions: np.ndarray    # [sum qo] int32 (new-token positions)
    out_loc: np.ndarray      # [sum qo] int32 (slots of the new tokens)
    is_decode: bool = False

    @property
    def batch_size(self) -> int:
        return int(self.device_lens.shape[0])

    @property
    def qo_lens(self) -> np.ndarray:
        return np.diff(self.qo_indptr).astype(np.int32)

    @property
    def kv_lens(self) -> np.ndarray:
        return np.diff(self.kv_indptr).astype(np.int32)

    @property
    def num_slots(self) -> int:
        return (self.num_pages + 1) * self.page_size


def make_paged_batch(rng: np.random.Generator, cached_lens, device_lens, page_size: int,
                     decode: bool = False, spare_pages: int = 0) -> PagedBatch:
    cached = np.asarray(cached_lens, dtype=np.int64)
    dev = np.asarray(device_lens, dtype=np.int64)
    assert cached.shape == dev.shape and np.all(cached <= dev) and np.all(dev >= 0)
    B = dev.shape[0]
    pages_per_req = (dev + page_size - 1) // page_size
    num_pages = int(pages_per_req.sum()) + spare_pages
    free_pages = rng.permutation(num_pages).astype(np.int64)
    width = align_up(int(dev.max()) if B else 1, 32)
    page_table = np.zeros((B + 1, width), dtype=np.int32)
    cursor = 0
    for r in range(B):
        n = int(pages_per_req[r])
        starts = free_pages[cursor:cursor + n] * page_size
        cursor += n
        slots = (starts[:, None] + np.arange(page_size)[None, :]).reshape(-1)
        page_table[r, :dev[r]] = slots[:dev[r]]
    # The spare row is the graph-capture dummy: every column at the spare slot.
    page_table[B, :] = num_pages * page_size
    table_idx = np.arange(B, dtype=np.int32)
    if decode:
        qo_lens = np.ones(B, dtype=np.int64)
    else:
        qo_lens = np.maximum(1, dev - cached)
    qo_indptr = np.concatenate([[0], np.cumsum(qo_lens)]).astype(np.int32)
    kv_indptr = np.concatenate([[0], np.cumsum(dev)]).astype(np.int32)
    indices = np.concatenate([page_table[r, :dev[r]] for r in range(B)]).astype(np.int32) \
        if B else np.zeros(0, np.int32)
    pos, loc = [], []
    for r in range(B):
        q0 = int(dev[r] - qo_lens[r])
        p = np.arange(q0, dev[r], dtype=np.int32)
        pos.append(p)
        loc.append(page_table[r, p])
    positions = np.concatenate(pos).astype(np.int32) if B else np.zeros(0, np.int32)
    out_loc = np.concatenate(loc).astype(np.int32) if B else np.zeros(0, np.int32)
    return PagedBatch(cached.astype(np.int32), dev.astype(np.int32), page_size, num_pages,
                      page_table, table_idx, qo_indptr, kv_indptr, indices, positions, out_loc,
                      decode)


@dataclass
class AttnShape:
    num_qo_heads: int
    num_kv_heads: int
    head_dim: int = 128

    @property
    def group(self) -> int:
        return self.num_qo_heads // self.num_kv_heads

    @property
    def qkv_width(self) -> int:
        return (self.num_qo_heads + 2 * self.num_kv_heads) * self.head_dim


QWEN3_0_6B = AttnShape(16, 8)
QWEN3_8B = AttnShape(32, 8)
QWEN3_30B_A3B = AttnShape(32, 4)


@dataclass
class Workload:
    name: str
    shape: AttnShape
    batch: PagedBatch
    layers: int = 1
    extra: dict = field(default_factory=dict)


def cfg1_decode_small(seed: int = 0) -> Workload:
    """Config 1: decode, 16q/8kv, B=4 x 512 cached tokens, page_size 1."""
    rng = np.random.default_rng(seed)
    b = make_paged_batch(rng, [511] * 4, [512] * 4, page_size=1, decode=True)
    return Workload("cfg1_decode_qwen3_0.6b_b4_kv512_p1", QWEN3_0_6B, b)


def cfg2_prefill_prefix(seed: int = 0) -> Workload:
    """Config 2: causal prefill, 16q/8kv, B=8, 256 cached + 128 new tokens, page_size 16."""
    rng = np.random.default_rng(seed)
    b = make_paged_batch(rng, [256] * 8, [384] * 8, page_size=16)
    return Workload("cfg2_prefill_qwen3_0.6b_b8_prefix256_ext128_p16", QWEN3_0_6B, b)


def cfg3_fused_store(seed: int = 0, tokens: int = 8192, requests: int = 64) -> Workload:
    """Config 3: fused RoPE + qk-RMSNorm + KV store, 8192 tokens over 64 requests.

    Positions ~ U[0, 8192), destination slots a seeded permutation of an
    8192-slot pool; heads 16q/8kv (Qwen3-0.6B).
    """
    rng = np.random.default_rng(seed)
    positions = rng.integers(0, 8192, size=tokens).astype(np.int32)
    out_loc = rng.permutation(tokens).astype(np.int32)
    per = tokens // requests
    qo_indptr = (np.arange(requests + 1) * per).astype(np.int32)
    qo_indptr[-1] = tokens
    b = PagedBatch(np.zeros(requests, np.int32), np.diff(qo_indptr).astype(np.int32), 1,
                   tokens - 1, np.zeros((1, 1), np.int32), np.zeros(requests, np.int32),
                   qo_indptr, qo_indptr.copy(), out_loc.copy(), positions, out_loc)
    return Workload("cfg3_fused_rope_qknorm_store_t8192", QWEN3_0_6B, b,
                    extra={"theta": 1e6, "eps": 1e-6, "max_pos": 8192})


def cfg4_decode_large(seed: int = 0, batch: int = 256) -> Workload:
    """Config 4: ragged decode, 32q/8kv, B=256, kv ~ U[128, 4096], page_size 16."""
    rng = np.random.default_rng(seed)
    kv = rng.integers(128, 4097, size=batch)
    b = make_paged_batch(rng, kv - 1, kv, page_size=16, decode=True)
    return Workload("cfg4_decode_qwen3_8b_b256_kv128-4096_p16", QWEN3_8B, b)


def cfg5_mixed(seed: int = 0, layers: int = 48, decode_reqs: int = 64) -> Workload:
    """Config 5: 64 decode requests (kv ~ U[1024, 32768]) + one 2048-token
    prefill chunk on a 4096-token cached prefix, 32q/4kv, page_size 16, 48 layers."""
    rng = np.random.default_rng(seed)
    kv = rng.integers(1024, 32769, size=decode_reqs)
    cached = np.concatenate([kv - 1, [4096]])
    dev = np.concatenate([kv, [4096 + 2048]])
    b = make_paged_batch(rng, cached, dev, page_size=16)
    return Workload("cfg5_mixed_qwen3_30b_a3b_64dec_kv1k-32k_plus_prefill2048_on4096_p16",
                    QWEN3_30B_A3B, b, layers=layers)


def cfg5_prefill_chunk(seed: int = 0) -> Workload:
    """The prefill part of config 5 on its own: one 2048-token chunk on a
    4096-token cached prefix, 32q/4kv, page_size 16 (one layer)."""
    rng = np.random.default_rng(seed)
    b = make_paged_batch(rng, [4096], [4096 + 2048], page_size=16)
    return Workload("cfg5_prefill_chunk_qwen3_30b_a3b_2048_on4096_p16", QWEN3_30B_A3B, b)


def attention_bytes(shape: AttnShape, qo_lens, kv_lens, page_size: int) -> int:
    """Algorithmic HBM bytes: K+V bf16 once, Q in + O out bf16, one int32 index per page."""
    kv = np.asarray(kv_lens, dtype=np.int64)
    qo = np.asarray(qo_lens, dtype=np.int64)
    D = shape.head_dim
    pages = (kv + page_size - 1) // page_size
    return int(4 * shape.num_kv_heads * D * kv.sum() + 4 * shape.num_qo_heads * D * qo.sum()
               + 4 * pages.sum())


def causal_pairs(qo_len: int, kv_len: int) -> int:
    """Visible (query, key) pairs of one request under bottom-right causal alignment."""
    off = kv_len - qo_len
    i = np.arange(qo_len, dtype=np.int64)
    return int(np.minimum(i + off + 1, kv_len).clip(min=0).sum())


def attention_flops(shape: AttnShape, qo_lens, kv_lens, causal: bool) -> int:
    pairs = 0
    for q, k in zip(np.asarray(qo_lens), np.asarray(kv_lens)):
        pairs += causal_pairs(int(q), int(k)) if causal else int(q) * int(k)
    return 4 * shape.head_dim * shape.num_qo_heads * pairs


def fused_store_bytes(shape: AttnShape, tokens: int) -> int:
    D, hq, hkv = shape.head_dim, shape.num_qo_heads, shape.num_kv_heads
    return (tokens * D * (2 * hq + 2 * hkv) * 2 + tokens * hkv * D * 2 * 2
            + 8 * tokens * (D // 2) + 8 * tokens)
