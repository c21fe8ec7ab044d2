"""The dispatch-layer entry points that round out the drop-in boundary
(ComputeDispatch's gemm, gpu_ffn_fused, flush_token / resume_token,
init_gpu_pool, init_kv_cache, pre_allocate_activation_buffer and
preload_all_buffers) through the C-ABI on the GPU: compute ops against
numpy / the oracle, the rest by their effects."""
import ctypes as C

import numpy as np
import pytest

import nexus_amd
import oracle
from conftest import f16, rel_err
from test_gpu_kernels import up

pytestmark = pytest.mark.gpu
L = oracle.lib


@pytest.mark.parametrize("M,N,K", [(1, 70, 131), (37, 70, 131), (64, 64, 16), (256, 512, 1024), (8, 4096, 4096)])
def test_gemm_f32(ctx, M, N, K):
    rng = np.random.default_rng(M * 7 + N + K)
    A = rng.normal(0, 1, (M, K)).astype(np.float32)
    B = rng.normal(0, 1, (K, N)).astype(np.float32)
    cb = ctx.alloc(M * N * 4)
    ctx.check(ctx.L.nx_gemm_f32(ctx.h, up(ctx, A), up(ctx, B), cb, M, N, K), "gemm_f32")
    got = ctx.download(cb, (M, N), np.float32)
    want = A.astype(np.float64) @ B.astype(np.float64)
    # fp32 products and sums: a few ulps of the row's magnitude
    assert rel_err(got, want) < 1e-5


def test_gemm_f32_rejects_short_buffers(ctx):
    a = ctx.alloc(16)
    with pytest.raises(nexus_amd.NxError):
        ctx.check(ctx.L.nx_gemm_f32(ctx.h, a, a, a, 4, 4, 4), "gemm_f32")


def _ffn_weights(rng, d, F):
    g, u, dn = (rng.normal(0, 0.02, s).astype(np.float32) for s in ((F, d), (F, d), (d, F)))
    (cg, sg), (cu, su), (cd, sd) = oracle.quantize(g), oracle.quantize(u), oracle.quantize(dn)
    w13 = np.empty((2 * F, cg.shape[1]), np.uint8)
    s13 = np.empty((2 * F, sg.shape[1]), np.uint16)
    w13[0::2], s13[0::2], w13[1::2], s13[1::2] = cg, sg, cu, su
    return w13, s13, cd, sd, ((cg, sg), (cu, su), (cd, sd))


@pytest.mark.parametrize("d,F,B", [(256, 688, 1), (256, 688, 3), (4096, 14336, 1), (4096, 14336, 8)])
def test_ffn_int4_g32(ctx, d, F, B):
    """W2(fp16(silu(W1 x) * W3 x)), accumulated into y, against the oracle's
    GEMVs on the same int4-g32 weights."""
    print(f"[case] ffn d={d} F={F} batch={B}", flush=True)
    rng = np.random.default_rng(d + F + B)
    w13, s13, w2, s2, ((cg, sg), (cu, su), (cd, sd)) = _ffn_weights(rng, d, F)
    x = rng.normal(0, 1, (B, d)).astype(np.float16)
    y0 = rng.normal(0, 1, (B, d)).astype(np.float32)
    yb = up(ctx, y0)
    bufs = [up(ctx, a) for a in (x.view(np.uint16), w13, s13, w2, s2)]
    ctx.check(ctx.L.nx_ffn_int4_g32(ctx.h, *bufs, yb, d, F, B, 1), "ffn")
    got = ctx.download(yb, (B, d), np.float32)
    xf = x.astype(np.float32)
    gv, uv = oracle.gemv(cg, sg, xf, F, d), oracle.gemv(cu, su, xf, F, d)
    act = (gv / (1.0 + np.exp(-gv.astype(np.float64))) * uv).astype(np.float16).astype(np.float32)
    want = y0 + oracle.gemv(cd, sd, act, d, F)
    assert rel_err(got - y0, want - y0) < 1e-3
    for b in bufs + [yb]:
        ctx.free(b)


def test_token_flush_and_resume(ctx):
    """flush runs what the token batch captured so far (its result can be
    read), resume captures the rest; both segments replay on later tokens."""
    n = 4096
    rng = np.random.default_rng(3)
    for rep in range(3):
        a = rng.normal(0, 1, n).astype(np.float32)
        b = rng.normal(0, 1, n).astype(np.float32)
        ab, bb = up(ctx, a), up(ctx, b)
        cb, db = ctx.alloc(n * 4), ctx.alloc(n * 4)
        ctx.check(ctx.L.nx_token_begin(ctx.h), "begin")
        ctx.check(ctx.L.nx_residual_add(ctx.h, ab, bb, cb, n), "add1")
        ctx.check(ctx.L.nx_token_flush(ctx.h), "flush")
        ctx.check(ctx.L.nx_token_flush(ctx.h), "flush again (no-op)")
        mid = ctx.download(cb, n, np.float32)
        assert np.array_equal(mid, a + b)
        ctx.check(ctx.L.nx_token_resume(ctx.h), "resume")
        ctx.check(ctx.L.nx_token_resume(ctx.h), "resume again (no-op)")
        ctx.check(ctx.L.nx_residual_add(ctx.h, cb, bb, db, n), "add2")
        ctx.check(ctx.L.nx_token_end(ctx.h), "end")
        assert np.array_equal(ctx.download(db, n, np.float32), (a + b) + b)
        for x in (ab, bb, cb, db):
            ctx.free(x)
    assert ctx.L.nx_token_flush(ctx.h) == 5  # NX_ERR_STATE outside a token batch
    assert ctx.L.nx_token_resume(ctx.h) == 5


def test_gpu_pool_sizes(ctx):
    pool = nexus_amd.GpuPool()
    ctx.check(ctx.L.nx_init_gpu_pool(ctx.h, 4096, 4096, 1024, 14336, 128256, 2, C.byref(pool)), "pool")
    want = {"hidden": 2 * 4096 * 4, "residual": 2 * 4096 * 4, "norm": 2 * 4096 * 2, "q": 2 * 4096 * 4,
            "k": 2 * 1024 * 4, "v": 2 * 1024 * 4, "attn_out": 2 * 4096 * 2, "ffn_gate": 2 * 14336 * 4,
            "ffn_up": 2 * 14336 * 4, "ffn_act": 2 * 14336 * 2, "ffn_out": 2 * 4096 * 4,
            "logits": 2 * 128256 * 4, "token": 2 * 4}
    for name, nbytes in want.items():
        sz = C.c_size_t()
        buf = getattr(pool, name)
        ctx.check(ctx.L.nx_buffer_size(ctx.h, buf, C.byref(sz)), name)
        assert sz.value == nbytes, name
        assert not ctx.download(buf, nbytes, np.uint8).any(), name
    for name in want:
        ctx.free(getattr(pool, name))


def test_kv_cache_feeds_the_paged_entry_points(ctx):
    """Pages from nx_init_kv_cache: K/V appended position by position, then
    paged attention over them equals the oracle's on the same pages."""
    layers, max_seq, hkv, hd, B, hq = 2, 80, 2, 64, 2, 4
    kp = (C.c_uint64 * layers)()
    vp = (C.c_uint64 * layers)()
    bt, mb, nb = C.c_uint64(), C.c_int(), C.c_int()
    ctx.check(ctx.L.nx_init_kv_cache(ctx.h, layers, max_seq, hkv, hd, B, kp, vp, C.byref(bt), C.byref(mb),
                                     C.byref(nb)), "kv cache")
    assert mb.value == 5 and nb.value == 10
    table = ctx.download(bt.value, (B, mb.value), np.int32)
    assert np.array_equal(table, np.arange(10, dtype=np.int32).reshape(B, 5))
    rng = np.random.default_rng(9)
    lens = np.array([37, 70], np.int32)
    for p in range(int(lens.max())):
        pos = np.minimum(p, lens - 1).astype(np.int32)
        k = rng.normal(0, 1, (B, hkv, hd)).astype(np.float32)
        v = rng.normal(0, 1, (B, hkv, hd)).astype(np.float32)
        ctx.check(ctx.L.nx_kv_append_f16(ctx.h, up(ctx, k), up(ctx, v), kp[1], vp[1], bt.value, up(ctx, pos), B,
                                         hkv, hd, mb.value, nb.value), "append")
    q = rng.normal(0, 1, (B, hq, hd)).astype(np.float32)
    ob = ctx.alloc(B * hq * hd * 2)
    ctx.check(ctx.L.nx_attn_decode_paged_f16(ctx.h, up(ctx, q), kp[1], vp[1], bt.value, up(ctx, lens), ob, B, hq,
                                             hkv, hd, mb.value, nb.value), "attn")
    got = f16(ctx.download(ob, (B, hq, hd), np.uint16))
    pool_elems = nb.value * hkv * 16 * hd
    kh = ctx.download(kp[1], pool_elems, np.uint16)
    vh = ctx.download(vp[1], pool_elems, np.uint16)
    want = np.empty_like(q)
    L.nxo_attn_decode_paged_f16(q, kh, vh, table, mb.value, lens, B, hq, hkv, hd, want)
    assert rel_err(got, want) < 1e-3
    # layer 0 was never written: still zero
    assert not ctx.download(kp[0], pool_elems * 2, np.uint8).any()


def test_reserved_workspace_allows_capture(ctx):
    """After nx_reserve_workspace, the FFN and the sampler run inside a token
    batch (graph capture) without growing a workspace."""
    d, F, V = 256, 688, 4096
    fresh = nexus_amd.Context(0)
    try:
        rng = np.random.default_rng(12)
        w13, s13, w2, s2, _ = _ffn_weights(rng, d, F)
        x = rng.normal(0, 1, (1, d)).astype(np.float16)
        bufs = [fresh.upload(np.ascontiguousarray(a)) for a in (x.view(np.uint16), w13, s13, w2, s2)]
        y = fresh.alloc(d * 4)
        logits = fresh.upload(rng.normal(0, 3, V).astype(np.float32))
        tok = fresh.alloc(4)
        # without a reservation the first FFN call cannot grow its workspace under capture
        fresh.check(fresh.L.nx_token_begin(fresh.h), "begin")
        assert fresh.L.nx_ffn_int4_g32(fresh.h, *bufs, y, d, F, 1, 0) == 5
        fresh.check(fresh.L.nx_token_end(fresh.h), "end")
        fresh.check(fresh.L.nx_reserve_workspace(fresh.h, 1, F, V, 4, 2, 64, 256), "reserve")
        fresh.check(fresh.L.nx_token_begin(fresh.h), "begin")
        fresh.check(fresh.L.nx_ffn_int4_g32(fresh.h, *bufs, y, d, F, 1, 0), "ffn in capture")
        fresh.check(fresh.L.nx_sample(fresh.h, logits, tok, V, 1, 0.8, 40, 0.9, 7), "sample in capture")
        fresh.check(fresh.L.nx_token_end(fresh.h), "end")
        direct = fresh.alloc(d * 4)
        fresh.check(fresh.L.nx_ffn_int4_g32(fresh.h, *bufs, direct, d, F, 1, 0), "ffn")
        assert np.array_equal(fresh.download(y, d, np.float32), fresh.download(direct, d, np.float32))
        t = fresh.download(tok, 1, np.int32)[0]
        assert 0 <= t < V
        n = C.c_size_t()
        fresh.check(fresh.L.nx_preload_all_buffers(fresh.h, C.byref(n)), "preload")
        assert n.value == 0
    finally:
        fresh.close()


def test_preload_counts_cached_weights(ctx):
    fresh = nexus_amd.Context(0)
    try:
        w = [np.arange(1000, dtype=np.float32) + i for i in range(3)]
        for a in w:
            b = C.c_uint64()
            fresh.check(fresh.L.nx_weight_cache(fresh.h, a.ctypes.data, a.ctypes.data, a.nbytes, C.byref(b)), "wc")
        n = C.c_size_t()
        fresh.check(fresh.L.nx_preload_all_buffers(fresh.h, C.byref(n)), "preload")
        assert n.value == 3
    finally:
        fresh.close()
