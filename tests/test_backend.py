"""The C++ backend (HipAttnBackend, MHAKVCache, AttentionLayer) against the
CPU oracle, through the reference's BaseAttnBackend call sequence
(prepare_metadata -> forward; init_capture_graph -> prepare_for_capture ->
capture -> prepare_for_replay -> replay), as the reference's engine drives it
(src/engine/engine.cc:557-561 and GraphRunner, src/engine/engine.cc:670-743)."""
import math
import sys

import numpy as np
import pytest
import torch

from conftest import capi, pkg, wl
from helpers import assert_attn_close, u16

D = 128


def note(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def sb():
    return pkg.backend.load()


def test_backend_module_surface(sb):
    """Loads on CPU too: every reference-named class is exported."""
    for name in ["Req", "Batch", "MHAKVCache", "HipAttnBackend", "RMSNorm", "RotaryEmbedding",
                 "AttentionLayer", "fused_qk_rmsnorm_inplace_3d_strided", "silu_and_mul",
                 "gelu_and_mul", "flashinfer_sample_from_probs",
                 "flashinfer_top_k_sample_from_probs", "flashinfer_top_p_sample_from_probs",
                 "flashinfer_top_k_top_p_sample_from_probs", "write_page_table"]:
        assert hasattr(sb, name), name
    r = sb.Req(3, 10, 25)
    assert (r.table_idx, r.cached_len, r.device_len(), r.extend_len()) == (3, 10, 25, 15)


def _gen(dev, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return g


def _randn(shape, dev, g, scale=1.0):
    return (torch.randn(shape, device=dev, generator=g) * scale).to(torch.bfloat16)


class Setup:
    """Pool + backend + batch for a PagedBatch."""

    def __init__(self, sb, dev, b, hq, hkv, seed, layers=2):
        self.b, self.hq, self.hkv = b, hq, hkv
        self.cache = sb.MHAKVCache(hkv, layers, D, b.num_pages + 1, b.page_size, 0)
        g = _gen(dev, seed)
        buf = self.cache.buffer()
        buf.copy_(_randn(tuple(buf.shape), dev, g))
        self.backend = sb.HipAttnBackend(self.cache, hq, hkv, D)
        self.backend.set_page_table(torch.from_numpy(b.page_table).to(dev))
        reqs = [sb.Req(int(b.table_idx[i]), int(b.cached_lens[i]), int(b.device_lens[i]))
                for i in range(b.batch_size)]
        self.batch = sb.Batch(not b.is_decode, reqs, torch.from_numpy(b.positions).to(dev),
                              torch.from_numpy(b.out_loc).to(dev))
        T = int(b.qo_indptr[-1])
        self.q = _randn((T, hq * D), dev, g)
        self.k = _randn((T, hkv * D), dev, g)
        self.v = _randn((T, hkv * D), dev, g)

    def expected(self, oracle, layer, scale):
        """Oracle: store the new tokens in a host copy of the pool, then attend."""
        b = self.b
        kc = u16(self.k_before[layer]).copy()
        vc = u16(self.v_before[layer]).copy()
        T = self.q.shape[0]
        kc[b.out_loc] = u16(self.k).reshape(T, self.hkv, D)
        vc[b.out_loc] = u16(self.v).reshape(T, self.hkv, D)
        q = u16(self.q).reshape(T, self.hq, D).copy()
        if b.is_decode:
            ref = oracle.decode(q, kc, vc, b.indices, b.kv_indptr, scale)
        else:
            ref = oracle.prefill(q, kc, vc, b.indices, b.qo_indptr, b.kv_indptr, scale)
        return ref.reshape(T, -1), kc, vc

    def snapshot(self):
        L = self.cache.buffer().shape[1]
        self.k_before = [self.cache.k_cache(l).clone() for l in range(L)]
        self.v_before = [self.cache.v_cache(l).clone() for l in range(L)]


def _run_forward(oracle, s, layer=1):
    s.snapshot()
    s.backend.prepare_metadata(s.batch)
    o = s.backend.forward(s.q, s.k, s.v, layer, s.batch)
    torch.cuda.synchronize()
    ref, kc, vc = s.expected(oracle, layer, 1 / math.sqrt(D))
    assert_attn_close(o.float().cpu().numpy(), ref, what="backend forward")
    # the store is bit exact, and only this layer's pool changed
    np.testing.assert_array_equal(u16(s.cache.k_cache(layer)), kc)
    np.testing.assert_array_equal(u16(s.cache.v_cache(layer)), vc)
    other = 1 - layer
    assert torch.equal(s.cache.k_cache(other), s.k_before[other])
    return o


@pytest.mark.gpu
@pytest.mark.parametrize("hq,hkv", [(16, 8), (32, 4)])
def test_backend_decode_forward(oracle, dev, sb, hq, hkv):
    note(f"backend decode forward {hq}/{hkv}")
    rng = np.random.default_rng(40)
    lens = [1, 37, 900, 4096, 129]
    b = wl.make_paged_batch(rng, [x - 1 for x in lens], lens, page_size=16, decode=True)
    s = Setup(sb, dev, b, hq, hkv, 41)
    _run_forward(oracle, s)
    assert s.batch.num_decode_rows() == len(lens) and s.batch.num_prefill_rows() == 0
    # decode: get_last_indices = kv_indptr[1..bs] - 1 (as the reference's metadata)
    got = s.batch.get_last_indices(len(lens)).cpu().numpy()
    np.testing.assert_array_equal(got, b.kv_indptr[1:] - 1)


@pytest.mark.gpu
def test_backend_prefill_no_cache_hit(oracle, dev, sb):
    note("backend prefill, no cache hit")
    rng = np.random.default_rng(42)
    lens = [1, 77, 640, 2000]
    b = wl.make_paged_batch(rng, [0] * 4, lens, page_size=16)
    s = Setup(sb, dev, b, 16, 8, 43)
    _run_forward(oracle, s)
    # the length-1 request goes through the decode kernel
    assert s.batch.num_decode_rows() == 1 and s.batch.num_prefill_rows() == 3
    np.testing.assert_array_equal(s.batch.get_last_indices(4).cpu().numpy(),
                                  b.qo_indptr[1:] - 1)


@pytest.mark.gpu
@pytest.mark.parametrize("hq,hkv", [(32, 8), (32, 4)])
def test_backend_prefill_prefix_and_mixed(oracle, dev, sb, hq, hkv):
    """Prefix hits, a chunked-prefill chunk and extend-1 rows in one batch."""
    note(f"backend mixed prefill {hq}/{hkv}")
    rng = np.random.default_rng(44)
    cached = [0, 100, 2047, 1024, 5, 3000]
    dev_lens = [300, 101, 2048, 2048, 6, 3100]
    b = wl.make_paged_batch(rng, cached, dev_lens, page_size=1)
    s = Setup(sb, dev, b, hq, hkv, 45)
    _run_forward(oracle, s, layer=0)
    assert s.batch.num_decode_rows() == 3 and s.batch.num_prefill_rows() == 3
    np.testing.assert_array_equal(s.batch.qo_indptr_host(), b.qo_indptr)
    np.testing.assert_array_equal(s.batch.get_last_indices(6).cpu().numpy(),
                                  b.qo_indptr[1:] - 1)


@pytest.mark.gpu
def test_backend_rejects_fp16_q(dev, sb):
    rng = np.random.default_rng(46)
    b = wl.make_paged_batch(rng, [9], [10], page_size=16, decode=True)
    s = Setup(sb, dev, b, 16, 8, 47)
    s.backend.prepare_metadata(s.batch)
    with pytest.raises(RuntimeError, match="bf16"):
        s.backend.attend(s.q.to(torch.float16), 0, s.batch)


@pytest.mark.gpu
def test_attention_layer_matches_unfused_modules(dev, sb):
    """AttentionLayer (fused qk-norm + RoPE + store, then attention) equals the
    reference's module sequence: fused_qk_rmsnorm, RotaryEmbedding, forward."""
    note("attention layer fused vs modules")
    rng = np.random.default_rng(48)
    hq, hkv = 32, 8
    b = wl.make_paged_batch(rng, [0, 50, 999], [33, 51, 1400], page_size=16)
    s1 = Setup(sb, dev, b, hq, hkv, 49)
    s2 = Setup(sb, dev, b, hq, hkv, 49)
    g = _gen(dev, 50)
    rot = sb.RotaryEmbedding(D, D, 8192, 1e6, 0)
    qn, kn = sb.RMSNorm(D, 1e-6, 0), sb.RMSNorm(D, 1e-6, 0)
    qn.weight = _randn((D,), dev, g, 0.5) + 1
    kn.weight = _randn((D,), dev, g, 0.5) + 1
    T = s1.q.shape[0]
    qkv = torch.cat([s1.q, s1.k, s1.v], dim=1)
    layer = sb.AttentionLayer(1, hq, hkv, D, s1.backend, rot, qn, kn)
    s1.backend.prepare_metadata(s1.batch)
    o1 = layer.forward(qkv.clone(), s1.batch.positions, s1.batch)

    qkv2 = qkv.clone()
    q = qkv2[:, :hq * D].view(T, hq, D)
    k = qkv2[:, hq * D:(hq + hkv) * D].view(T, hkv, D)
    v = qkv2[:, (hq + hkv) * D:].view(T, hkv, D)
    sb.fused_qk_rmsnorm_inplace_3d_strided(q, k, qn, kn)
    rot.forward_inplace(s2.batch.positions, q, k)
    s2.backend.prepare_metadata(s2.batch)
    o2 = s2.backend.forward(q, k, v, 1, s2.batch)
    torch.cuda.synchronize()
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))
    assert torch.equal(s1.cache.buffer().view(torch.int16), s2.cache.buffer().view(torch.int16))


@pytest.mark.gpu
def test_norm_and_rope_modules_fp16(dev, sb):
    """The reference's RMSNorm / fused qk-norm / RotaryEmbedding dispatch fp16
    as well as bf16 (normalization.cu:346-372, rotary_embedding.cu:124-168):
    the modules on fp16 tensors equal the C ABI calls (pinned to the oracle in
    test_gpu_parity), bit for bit, and mixed dtypes are refused."""
    note("fp16 norm / rope modules")
    g = _gen(dev, 55)
    T, hq, hkv = 9, 16, 8
    q = (torch.randn((T, hq, D), device=dev, generator=g)).to(torch.float16)
    k = (torch.randn((T, hkv, D), device=dev, generator=g)).to(torch.float16)
    qn, kn = sb.RMSNorm(D, 1e-6, 0), sb.RMSNorm(D, 1e-6, 0)
    qn.weight = (torch.rand(D, device=dev, generator=g) + 0.5).to(torch.float16)
    kn.weight = (torch.rand(D, device=dev, generator=g) + 0.5).to(torch.float16)
    rot = sb.RotaryEmbedding(D, D, 4096, 1e6, 0)
    pos = torch.randint(0, 4096, (T,), device=dev, generator=g, dtype=torch.int32)
    q1, k1, q2, k2 = q.clone(), k.clone(), q.clone(), k.clone()
    sb.fused_qk_rmsnorm_inplace_3d_strided(q1, k1, qn, kn)
    rot.forward_inplace(pos, q1, k1)
    capi.qk_rmsnorm(q2, k2, qn.weight, kn.weight, 1e-6)
    capi.rope(pos, q2, k2, rot.cos_cache(), rot.sin_cache())
    torch.cuda.synchronize()
    assert torch.equal(q1.view(torch.int16), q2.view(torch.int16))
    assert torch.equal(k1.view(torch.int16), k2.view(torch.int16))
    assert not torch.equal(q1.view(torch.int16), q.view(torch.int16))
    with pytest.raises(RuntimeError, match="share one dtype"):
        sb.fused_qk_rmsnorm_inplace_3d_strided(q1, k1.to(torch.bfloat16), qn, kn)
    with pytest.raises(RuntimeError, match="share one dtype"):
        rot.forward_inplace(pos, q1, k1.to(torch.bfloat16))


@pytest.mark.gpu
def test_missing_context_raises_without_side_effects(dev, sb):
    """The reference's layer test expects a throw when the context is missing
    (tests/layers/test_attention_layer.cpp:7-22): here a backend without a page
    table refuses prepare_metadata, and a layer or backend forward on a batch
    without metadata raises before anything reaches the pool."""
    note("missing context")
    rng = np.random.default_rng(53)
    hq, hkv = 16, 8
    b = wl.make_paged_batch(rng, [3, 0], [4, 20], page_size=16)
    s = Setup(sb, dev, b, hq, hkv, 54)
    bare = sb.HipAttnBackend(s.cache, hq, hkv, D)
    with pytest.raises(RuntimeError, match="set_page_table"):
        bare.prepare_metadata(s.batch)
    rot = sb.RotaryEmbedding(D, D, 8192, 1e6, 0)
    layer = sb.AttentionLayer(0, hq, hkv, D, s.backend, rot, None, None)
    qkv = torch.cat([s.q, s.k, s.v], dim=1)
    qkv_before = qkv.clone()
    pool_before = s.cache.buffer().clone()
    with pytest.raises(RuntimeError, match="prepare_metadata"):
        layer.forward(qkv, s.batch.positions, s.batch)
    with pytest.raises(RuntimeError, match="prepare_metadata"):
        s.backend.forward(s.q, s.k, s.v, 0, s.batch)
    torch.cuda.synchronize()
    assert torch.equal(qkv.view(torch.int16), qkv_before.view(torch.int16))
    assert torch.equal(s.cache.buffer().view(torch.int16), pool_before.view(torch.int16))


@pytest.mark.gpu
def test_backend_decode_graph_capture_replay(oracle, dev, sb):
    """Capture forward once at the worst case, replay on batches of new lengths;
    every replay matches the oracle and the eager forward of the same batch."""
    note("backend decode graph capture / replay")
    hq, hkv, max_seq, bs = 32, 8, 1024, 8
    rng = np.random.default_rng(51)
    # one page-table row per request at max_seq, plus the spare row
    full = wl.make_paged_batch(rng, [max_seq - 1] * bs, [max_seq] * bs, page_size=16,
                               decode=True)
    cache = sb.MHAKVCache(hkv, 1, D, full.num_pages + 1, 16, 0)
    g = _gen(dev, 52)
    cache.buffer().copy_(_randn(tuple(cache.buffer().shape), dev, g))
    backend = sb.HipAttnBackend(cache, hq, hkv, D)
    page_table = torch.from_numpy(full.page_table).to(dev)
    backend.set_page_table(page_table)
    backend.init_capture_graph(max_seq, [4, bs])

    static_q = torch.zeros(bs, hq * D, device=dev, dtype=torch.bfloat16)
    static_k = torch.zeros(bs, hkv * D, device=dev, dtype=torch.bfloat16)
    static_v = torch.zeros_like(static_k)
    static_loc = torch.from_numpy(full.out_loc).to(dev)
    reqs = [sb.Req(i, max_seq - 1, max_seq) for i in range(bs)]
    cap = sb.Batch(False, reqs, torch.zeros(bs, dtype=torch.int32, device=dev), static_loc)
    backend.prepare_for_capture(cap)
    assert cap.uses_capture_buffers()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        backend.forward(static_q, static_k, static_v, 0, cap)  # warm-up
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_o = backend.forward(static_q, static_k, static_v, 0, cap)

    scale = 1 / math.sqrt(D)
    pt = full.page_table
    for it in range(5):
        lens = rng.integers(1, max_seq + 1, bs)
        if it == 3:
            lens[:] = max_seq
        if it == 4:
            lens[:] = 1  # every request at its first token
        loc = np.array([pt[i, lens[i] - 1] for i in range(bs)], np.int32)
        q = _randn((bs, hq * D), dev, g)
        k = _randn((bs, hkv * D), dev, g)
        v = _randn((bs, hkv * D), dev, g)
        rb = sb.Batch(False, [sb.Req(i, int(n) - 1, int(n)) for i, n in enumerate(lens)],
                      torch.from_numpy(lens.astype(np.int32) - 1).to(dev),
                      torch.from_numpy(loc).to(dev))
        backend.prepare_metadata(rb)
        backend.prepare_for_replay(rb)
        static_q.copy_(q)
        static_k.copy_(k)
        static_v.copy_(v)
        static_loc.copy_(rb.out_loc)
        graph.replay()
        torch.cuda.synchronize()
        got = static_o.float().cpu().numpy()
        kc, vc = u16(cache.k_cache(0)), u16(cache.v_cache(0))
        ip = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        idx = np.concatenate([pt[i, :lens[i]] for i in range(bs)]).astype(np.int32)
        ref = oracle.decode(u16(q).reshape(bs, hq, D).copy(), kc, vc, idx, ip, scale)
        assert_attn_close(got, ref.reshape(bs, -1), what=f"replay {it}")
        # eager forward of the same batch (the store rewrites the same values)
        eb = sb.Batch(False, [sb.Req(i, int(n) - 1, int(n)) for i, n in enumerate(lens)],
                      rb.positions, rb.out_loc)
        backend.prepare_metadata(eb)
        o_eager = backend.forward(q, k, v, 0, eb)
        torch.cuda.synchronize()
        assert_attn_close(o_eager.float().cpu().numpy(), ref.reshape(bs, -1),
                          what=f"eager {it}")

    # An eager batch that needs a larger split workspace than any captured
    # plan (64 requests over the same table rows) must not move the buffer
    # the graph was captured with.
    big = sb.Batch(False, [sb.Req(i % bs, max_seq - 1, max_seq) for i in range(64)],
                   torch.full((64,), max_seq - 1, dtype=torch.int32, device=dev),
                   static_loc.repeat(8))
    backend.prepare_metadata(big)
    qb = _randn((64, hq * D), dev, g)
    kb = torch.cat([k] * 8)
    vb = torch.cat([v] * 8)
    backend.forward(qb, kb, vb, 0, big)
    torch.cuda.synchronize()
    lens = np.full(bs, max_seq)
    loc = np.array([pt[i, max_seq - 1] for i in range(bs)], np.int32)
    rb = sb.Batch(False, [sb.Req(i, max_seq - 1, max_seq) for i in range(bs)],
                  torch.full((bs,), max_seq - 1, dtype=torch.int32, device=dev),
                  torch.from_numpy(loc).to(dev))
    backend.prepare_metadata(rb)
    backend.prepare_for_replay(rb)
    q = _randn((bs, hq * D), dev, g)
    static_q.copy_(q)
    static_k.copy_(k)
    static_v.copy_(v)
    static_loc.copy_(rb.out_loc)
    graph.replay()
    torch.cuda.synchronize()
    kc, vc = u16(cache.k_cache(0)), u16(cache.v_cache(0))
    ip = (np.arange(bs + 1) * max_seq).astype(np.int32)
    idx = np.concatenate([pt[i, :max_seq] for i in range(bs)]).astype(np.int32)
    ref = oracle.decode(u16(q).reshape(bs, hq, D).copy(), kc, vc, idx, ip, scale)
    assert_attn_close(static_o.float().cpu().numpy(), ref.reshape(bs, -1),
                      what="replay after workspace growth")


@pytest.mark.gpu
def test_backend_mixed_batch_overlap_and_graph_replay(oracle, dev, sb):
    """A mixed batch (qo=1 rows beside a prefill chunk): with separate
    launches the side-stream overlap gives the same bits as the serial order;
    the one-launch path (decode rows on a CU share) matches the oracle; and a
    captured graph of the step replays to the eager result every time."""
    note("backend mixed batch: overlap, one launch and graph replay")
    rng = np.random.default_rng(53)
    kv = [900, 3000, 17, 4096 + 512]
    cached = [899, 2999, 16, 4096]
    b = wl.make_paged_batch(rng, cached, kv, page_size=16)
    s = Setup(sb, dev, b, 32, 4, 54, layers=1)
    s.snapshot()
    s.backend.set_fused_mixed(False)
    s.backend.prepare_metadata(s.batch)
    assert s.batch.num_decode_rows() == 3 and s.batch.num_prefill_rows() == 1
    assert s.batch.fused_mixed_cus() == 0
    s.backend.set_overlap_mixed(False)
    o_serial = s.backend.forward(s.q, s.k, s.v, 0, s.batch).clone()
    s.backend.set_overlap_mixed(True)
    o_overlap = s.backend.forward(s.q, s.k, s.v, 0, s.batch).clone()
    torch.cuda.synchronize()
    assert torch.equal(o_serial.view(torch.int16), o_overlap.view(torch.int16))
    ref, _, _ = s.expected(oracle, 0, 1 / math.sqrt(D))
    assert_attn_close(o_overlap.float().cpu().numpy(), ref, what="mixed overlap")
    s.backend.set_fused_mixed(True)
    s.backend.prepare_metadata(s.batch)
    assert s.batch.fused_mixed_cus() >= 8
    o_fused = s.backend.forward(s.q, s.k, s.v, 0, s.batch).clone()
    torch.cuda.synchronize()
    assert_attn_close(o_fused.float().cpu().numpy(), ref, what="mixed one launch")

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        s.backend.forward(s.q, s.k, s.v, 0, s.batch)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        o_graph = s.backend.forward(s.q, s.k, s.v, 0, s.batch)
    for it in range(3):
        o_graph.zero_()
        graph.replay()
        # eager work between replays, as a serving loop would have
        o_eager = s.backend.forward(s.q, s.k, s.v, 0, s.batch)
        torch.cuda.synchronize()
        assert torch.equal(o_graph.view(torch.int16), o_eager.view(torch.int16)), f"replay {it}"
    # An eager decode batch whose plan needs a larger split workspace than the
    # one the graph recorded: the backend grows its workspace, and the graph's
    # buffer must stay alive and private to it.
    big = sb.Batch(False, [sb.Req(1, 2999, 3000) for _ in range(200)],
                   torch.full((200,), 2999, dtype=torch.int32, device=dev),
                   torch.zeros(200, dtype=torch.int32, device=dev))
    s.backend.prepare_metadata(big)
    assert big.decode_plan()["num_units"] > 100
    g = _gen(dev, 55)
    s.backend.attend(_randn((200, 32 * D), dev, g), 0, big)
    torch.cuda.synchronize()
    o_graph.zero_()
    graph.replay()
    o_eager = s.backend.forward(s.q, s.k, s.v, 0, s.batch)
    torch.cuda.synchronize()
    assert torch.equal(o_graph.view(torch.int16), o_eager.view(torch.int16)), "after growth"


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_residual_modules_match_c_abi(dev, sb, dtype):
    """RMSNorm.forward / forward_inplace / fused_add_forward_inplace and
    silu_and_mul / gelu_and_mul (the reference's layer API, as
    qwen3.cc:24-31,62 and utils.cc:49 call it) give the C ABI's bits; the
    shapes are the reference tests' (test_normalization.cpp:5-19,
    test_activation.cpp:5-29) and a Qwen3-8B layer's."""
    from conftest import capi
    note(f"residual modules {dtype}")
    g = _gen(dev, 90)
    for rows, d in [(10, 128), (300, 4096)]:
        norm = sb.RMSNorm(d, 1e-6, 0)
        norm.weight = (torch.rand(d, device=dev, generator=g) + 0.5).to(dtype)
        x = torch.randn((rows, d), device=dev, generator=g).to(dtype)
        r = torch.randn((rows, d), device=dev, generator=g).to(dtype)
        want = capi.rmsnorm(x, norm.weight, 1e-6)
        assert torch.equal(norm.forward(x), want)
        y = x.clone()
        norm.forward_inplace(y)
        assert torch.equal(y, want)
        x1, r1 = x.clone(), r.clone()
        norm.fused_add_forward_inplace(x1, r1)
        x2, r2 = x.clone(), r.clone()
        capi.fused_add_rmsnorm(x2, r2, norm.weight, 1e-6)
        assert torch.equal(x1, x2) and torch.equal(r1, r2)
        assert torch.equal(r1, (x.float() + r.float()).to(dtype))
    for fn, cfn in [(sb.silu_and_mul, capi.silu_and_mul), (sb.gelu_and_mul, capi.gelu_and_mul)]:
        for tokens, d in [(10, 128), (64, 12288)]:
            inp = torch.randn((tokens, 2 * d), device=dev, generator=g).to(dtype)
            a = torch.empty((tokens, d), device=dev, dtype=dtype)
            b = torch.empty_like(a)
            fn(a, inp)
            cfn(b, inp)
            assert torch.equal(a, b)
    torch.cuda.synchronize()


@pytest.mark.gpu
def test_sampling_probs_matches_c_abi(dev, sb):
    """Sampler::sample's probabilities (engine.cc:306-308: temperatures as
    given by BatchSamplingArgs, [batch, 1] after the view) through the C++
    layer equal the C ABI's, bit for bit."""
    from conftest import capi
    note("sampling probs")
    g = _gen(dev, 17)
    B, V = 5, 151936
    logits = (torch.randn((B, V), device=dev, generator=g) * 2).to(torch.bfloat16)
    temps = torch.tensor([[0.7], [1.0], [1.3], [0.5], [0.9]], device=dev, dtype=torch.float16)
    a = sb.sampling_probs(logits, temps)
    b = capi.softmax_temperature(logits, temps.float().view(B))
    assert torch.equal(a, b)


@pytest.mark.gpu
def test_sample_from_logits_matches_c_abi(dev, sb):
    """Sampler::sample's dispatch (engine.cc:310-333: top_k int32 beside
    top_p, float32 alone; uniform [batch] for the plain draw) through the
    C++ layer gives the C ABI's draws from logits."""
    from conftest import capi
    note("sample from logits")
    g = _gen(dev, 23)
    B, V = 6, 151936
    logits = (torch.randn((B, V), device=dev, generator=g) * 3).to(torch.bfloat16)
    temps = torch.linspace(0.6, 1.2, B, device=dev)
    u1 = torch.rand(B, device=dev, generator=g)
    u = torch.rand((32, B), device=dev, generator=g)
    k = torch.randint(1, 64, (B,), device=dev, generator=g)
    tp = torch.rand(B, device=dev, generator=g) * 0.5 + 0.45
    s, ok = sb.sample_from_logits(logits, temps, u1)
    assert ok is None and torch.equal(s, capi.sampling_from_logits(logits, u1, "plain", temps)[0])
    s, ok = sb.sample_from_logits(logits, temps, u, k, tp)
    r = capi.sampling_from_logits(logits, u, "top_k_top_p", temps, top_k=k.int(), top_p=tp)
    assert torch.equal(s, r[0]) and torch.equal(ok, r[1])
    s, ok = sb.sample_from_logits(logits, temps, u, k, None)
    r = capi.sampling_from_logits(logits, u, "top_k", temps, top_k=k.float())
    assert torch.equal(s, r[0]) and torch.equal(ok, r[1])


@pytest.mark.gpu
def test_sampling_functions_match_c_abi(dev, sb):
    """The reference's sampling API (include/sglang/engine/sampling.h:7-36) as
    the Sampler calls it (engine.cc:300-345: uniform [32, batch], top_k float32
    for top-k, int32 for top-k + top-p) gives the C ABI's draws."""
    from conftest import capi
    note("sampling functions")
    g = _gen(dev, 91)
    B, V = 16, 151936
    probs = torch.softmax(torch.randn((B, V), device=dev, generator=g) * 3, -1).contiguous()
    u1 = torch.rand(B, device=dev, generator=g)
    u = torch.rand((32, B), device=dev, generator=g)
    k = torch.randint(1, 64, (B,), device=dev, generator=g)
    tp = torch.rand(B, device=dev, generator=g) * 0.5 + 0.45
    assert torch.equal(sb.flashinfer_sample_from_probs(probs, u1, False),
                       capi.sampling_from_probs(probs, u1))
    a = sb.flashinfer_top_k_sample_from_probs(probs, u, k.float(), 0, False)
    b = capi.top_k_sampling_from_probs(probs, u, k.float())
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    a = sb.flashinfer_top_p_sample_from_probs(probs, u, tp, 0.0, False)
    b = capi.top_p_sampling_from_probs(probs, u, tp)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    a = sb.flashinfer_top_k_top_p_sample_from_probs(probs, u, k.int(), 0.0, tp, 0.0, False)
    b = capi.top_k_top_p_sampling_from_probs(probs, u, k.int(), 0, tp, 0.0)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    a = sb.flashinfer_top_k_sample_from_probs(probs, u, None, 5, False)
    assert bool(a[1].all())
    with pytest.raises(Exception):
        sb.flashinfer_top_k_top_p_sample_from_probs(probs, u, k.float(), 0.0, tp, 0.0, False)
    torch.cuda.synchronize()


@pytest.mark.gpu
def test_write_page_table_module(oracle, dev, sb):
    """The reference's CacheManager::write_page_table call (host page list and
    (table_idx, first_page, last_page) tuples, prefill.cc:144-187) writes what
    the oracle writes, and refuses a page count that does not match."""
    note("backend write_page_table")
    rng = np.random.default_rng(95)
    P = 16
    table = torch.zeros((9, 64 * P), dtype=torch.int32, device=dev)
    alloc = [(0, 0, 64), (3, 10, 12), (8, 5, 6)]
    n = sum(b - a for _, a, b in alloc)
    pages = [int(x) * P for x in rng.permutation(5000)[:n]]
    sb.write_page_table(table, pages, alloc, P)
    torch.cuda.synchronize()
    want = np.zeros((9, 64 * P), np.int32)
    assert oracle.write_page_table(want, np.array(pages, np.int32), alloc, P) == n
    np.testing.assert_array_equal(table.cpu().numpy(), want)
    with pytest.raises(RuntimeError, match="page count mismatch"):
        sb.write_page_table(table, pages[:-1], alloc, P)
