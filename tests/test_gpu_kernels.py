"""GPU parity tests of the decode kernels through the C-ABI, against the
oracle on identical inputs.  Integer and byte outputs (unpacked int4 codes,
quantized weights, fp16 KV bits, TurboQuant codes and norms, routed expert
ids) must match bit for bit; floating-point outputs must satisfy
max|gpu - oracle| / max|oracle| < 1e-3 (fp32 accumulation)."""
import numpy as np
import pytest

import nexus_amd
import oracle
from conftest import f16, rel_err

pytestmark = pytest.mark.gpu
L = oracle.lib
TOL = 1e-3


def up(ctx, a):
    return ctx.upload(np.ascontiguousarray(a))


# ------------------------------------------------------------------- int4 --
def test_unpack_bit_exact(ctx):
    rng = np.random.default_rng(0)
    packed = rng.integers(0, 256, 4096, dtype=np.uint8)
    packed[:256] = np.arange(256)
    cb = ctx.alloc(8192)
    ctx.check(ctx.L.nx_unpack_int4(ctx.h, up(ctx, packed), cb, 8192), "unpack")
    got = ctx.download(cb, 8192, np.uint8)
    want = np.empty(8192, np.uint8)
    L.nxo_unpack_int4(packed, 8192, want)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("N,K", [(33, 32), (64, 96), (17, 688), (256, 4096)])
def test_device_quantizer_bit_exact(ctx, N, K):
    rng = np.random.default_rng(N * K)
    w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    w[1] = 0.0
    w[2, 5] = 1.0
    G = (K + 31) // 32
    cb, sb = ctx.alloc(N * G * 16), ctx.alloc(N * G * 2)
    ctx.check(ctx.L.nx_quantize_int4_g32(ctx.h, up(ctx, w), cb, sb, N, K), "quantize")
    codes, scales = oracle.quantize(w)
    assert np.array_equal(ctx.download(cb, codes.shape, np.uint8), codes)
    assert np.array_equal(ctx.download(sb, scales.shape, np.uint16), scales)


def _gemv_case(ctx, N, K, B, codes, scales, seed):
    rng = np.random.default_rng(seed)
    x16 = rng.normal(0, 1, (B, K)).astype(np.float16)
    xb, wb, sb = up(ctx, x16.view(np.uint16)), up(ctx, codes), up(ctx, scales)
    want = oracle.gemv(codes, scales, x16.astype(np.float32), N, K)
    yb = ctx.alloc(B * N * 2)
    ctx.gemv(xb, wb, sb, yb, N, K, B)
    y16 = f16(ctx.download(yb, (B, N), np.uint16))
    y32b = ctx.alloc(B * N * 4)
    ctx.gemv_f32(xb, wb, sb, y32b, N, K, B)
    y32 = ctx.download(y32b, (B, N), np.float32)
    ctx.gemv_f32(xb, wb, sb, y32b, N, K, B, accumulate=True)
    y2 = ctx.download(y32b, (B, N), np.float32)
    for b in (xb, wb, sb, yb, y32b):
        ctx.free(b)
    return y16, y32, y2, want


@pytest.mark.parametrize("N,K,B", [(64, 96, 1), (256, 256, 1), (1376, 256, 1), (256, 688, 1),
                                   (256, 688, 3), (1024, 4096, 1), (4096, 4096, 2), (512, 14336, 1),
                                   (300, 14336, 8), (130, 8192, 5),
                                   # batch 2-8 scale-load forms: 16-byte loads clamped at the
                                   # stage end (24 groups), 2-byte loads (12 groups, G % 8 != 0),
                                   # several stages with G % 8 != 0 (132 groups)
                                   (160, 768, 4), (200, 384, 4), (96, 4224, 6)])
def test_gemv_parity(ctx, N, K, B):
    rng = np.random.default_rng(N + K + B)
    w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    codes, scales = oracle.quantize(w)
    y16, y32, y2, want = _gemv_case(ctx, N, K, B, codes, scales, N * K)
    assert rel_err(y16, want) < TOL
    assert rel_err(y32, want) < 1e-5
    assert rel_err(y2, 2 * want) < 1e-5


# The five Llama-3-8B projection shapes (out x in) of the GEMV microbench.
SHAPES_8B = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336), (128256, 4096)]


@pytest.mark.parametrize("N,K", SHAPES_8B)
@pytest.mark.parametrize("B", [1, 8])
def test_gemv_parity_8b_shapes(ctx, N, K, B):
    codes, scales = oracle.gen_quant_rows(0, N, K, 0x5EED, 900 + N % 97, 0.02)
    y16, y32, _, want = _gemv_case(ctx, N, K, B, codes, scales, N + B)
    assert rel_err(y16, want) < TOL
    assert rel_err(y32, want) < 1e-5


# 70B-class projections (d 8192, FFN 28672): the down projection's K = 28672
# runs the batch-1 kernel with x in LDS and the batch-8 matrix-core kernel's
# K split; gate/up (N = 28672, K = 8192) the ordinary forms.  Plus K = 28672
# with a ragged row count at batch 3 and a K that is not a multiple of 256.
@pytest.mark.parametrize("N,K,B", [(8192, 28672, 1), (8192, 28672, 8), (28672, 8192, 1), (28672, 8192, 8),
                                   (300, 28672, 3), (200, 20000, 1)])
def test_gemv_parity_70b_shapes(ctx, N, K, B):
    codes, scales = oracle.gen_quant_rows(0, N, K, 0x70B, N % 97 + K % 89, 0.02)
    y16, y32, y2, want = _gemv_case(ctx, N, K, B, codes, scales, N + K + B)
    assert rel_err(y16, want) < TOL
    assert rel_err(y32, want) < 1e-5
    assert rel_err(y2, 2 * want) < 1e-5


def test_gemv_rejects_bad_shapes(ctx):
    xb, wb, sb, yb = ctx.alloc(64), ctx.alloc(64), ctx.alloc(64), ctx.alloc(64)
    with pytest.raises(nexus_amd.NxError):
        ctx.gemv(xb, wb, sb, yb, 4096, 4096, 1)  # buffers far too small
    with pytest.raises(nexus_amd.NxError):
        ctx.gemv(xb, wb, sb, yb, 1, 32, 9)  # batch above 8
    with pytest.raises(nexus_amd.NxError):
        ctx.gemv(xb, wb, sb, 12345, 1, 32, 1)  # unknown buffer
    big = [ctx.alloc(1 << 20) for _ in range(4)]
    with pytest.raises(nexus_amd.NxError) as e:
        ctx.gemv(big[0], big[1], big[2], big[3], 1, 28704, 1)  # K above 28672
    assert e.value.code == 4
    for b in big:
        ctx.free(b)


# ------------------------------------------------------------ elementwise --
def test_rmsnorm_swiglu_residual_argmax(ctx):
    rng = np.random.default_rng(3)
    B, d = 3, 4096
    x = rng.normal(0, 2, (B, d)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, d).astype(np.float32)
    ob = ctx.alloc(B * d * 2)
    ctx.check(ctx.L.nx_rmsnorm(ctx.h, up(ctx, x), up(ctx, w), ob, d, 1e-5, B), "rmsnorm")
    got = f16(ctx.download(ob, (B, d), np.uint16))
    for b in range(B):
        want = np.empty(d, np.float32)
        L.nxo_rmsnorm(np.ascontiguousarray(x[b]), w.ctypes.data, d, 1e-5, want)
        assert rel_err(got[b], want) < TOL

    g = rng.normal(0, 3, (B, 700)).astype(np.float32)
    u = rng.normal(0, 1, (B, 700)).astype(np.float32)
    sb = ctx.alloc(B * 700 * 2)
    ctx.check(ctx.L.nx_swiglu(ctx.h, up(ctx, g), up(ctx, u), sb, 700, B), "swiglu")
    want = np.empty_like(g)
    L.nxo_swiglu(g.reshape(-1), u.reshape(-1), g.size, want.reshape(-1))
    assert rel_err(f16(ctx.download(sb, (B, 700), np.uint16)), want) < TOL

    a = rng.normal(0, 1, 1000).astype(np.float32)
    c = rng.normal(0, 1, 1000).astype(np.float32)
    rb = ctx.alloc(4000)
    ctx.check(ctx.L.nx_residual_add(ctx.h, up(ctx, a), up(ctx, c), rb, 1000), "residual")
    assert np.array_equal(ctx.download(rb, 1000, np.float32), a + c)

    logits = rng.normal(0, 1, (4, 128256)).astype(np.float32)
    logits[1, 77] = logits[1, 99] = 50.0  # tie: first maximum wins
    logits[2, :] = -3.0
    ib = ctx.alloc(16)
    ctx.check(ctx.L.nx_argmax(ctx.h, up(ctx, logits), ib, 128256, 4), "argmax")
    got = ctx.download(ib, 4, np.int32)
    assert list(got) == [L.nxo_argmax(np.ascontiguousarray(r), 128256) for r in logits]
    assert got[1] == 77 and got[2] == 0


def test_rope(ctx):
    hd, heads, B, theta, maxp = 128, 8, 2, 500000.0, 300
    cos = np.empty((maxp, hd // 2), np.float32)
    sin = np.empty((maxp, hd // 2), np.float32)
    L.nxo_rope_table(maxp, hd, theta, cos, sin)
    rng = np.random.default_rng(4)
    x = rng.normal(0, 1, (B, heads * hd)).astype(np.float32)
    pos = np.array([0, 257], np.int32)
    xb = up(ctx, x)
    ctx.check(ctx.L.nx_rope(ctx.h, xb, up(ctx, pos), up(ctx, cos), up(ctx, sin), heads, hd, B, maxp), "rope")
    got = ctx.download(xb, x.shape, np.float32)
    for b in range(B):
        want = x[b].copy()
        L.nxo_rope(want, heads, hd, int(pos[b]), cos, sin)
        assert rel_err(got[b], want) < 1e-6
    with pytest.raises(nexus_amd.NxError):
        ctx.check(ctx.L.nx_rope(ctx.h, xb, up(ctx, np.array([0, maxp], np.int32)), up(ctx, cos),
                                up(ctx, sin), heads, hd, B, maxp), "rope out of table")


# ---------------------------------------------------------- paged fp16 KV --
def _pools(rng, B, hkv, hd, lens, seed=7):
    max_blocks = max(1, -(-max(lens) // 16)) + 1
    nblk = B * max_blocks
    perm = np.empty(nblk, np.int32)
    L.nxo_shuffle_perm(perm, nblk, seed, 7)
    bt = np.ascontiguousarray(perm.reshape(B, max_blocks))
    kp = np.zeros((nblk, hkv, 16, hd), np.float16)  # K pages token-major
    vp = np.zeros((nblk, hkv, hd, 16), np.float16)  # V pages dimension-major
    for b in range(B):
        n = lens[b]
        K = rng.normal(0, 1, (n, hkv, hd)).astype(np.float16)
        V = rng.normal(0, 1, (n, hkv, hd)).astype(np.float16)
        for p in range(n):
            blk = bt[b, p // 16]
            kp[blk, :, p % 16, :] = K[p]
            vp[blk, :, :, p % 16] = V[p]
    return max_blocks, nblk, bt, kp.view(np.uint16), vp.view(np.uint16)


@pytest.mark.parametrize("hq,hkv,hd,lens", [
    (4, 2, 64, [1]), (4, 2, 64, [17]), (4, 2, 64, [16, 100]), (32, 8, 128, [4096]),
    (32, 8, 128, [1, 15, 300]), (8, 8, 128, [33]), (32, 4, 128, [64, 129]), (32, 8, 128, [4096] * 8),
    # 256-long heads: one page pair (short contexts) and the one-pair loop
    # (20000 positions, 20 pages per split), query groups of 1 to 8
    (8, 2, 256, [1]), (16, 4, 256, [300, 17]), (16, 2, 256, [33]), (4, 4, 256, [70]),
    (8, 1, 256, [20000]), (32, 8, 256, [4096] * 2)])
def test_attention_f16_parity(ctx, hq, hkv, hd, lens):
    rng = np.random.default_rng(hq + hd + sum(lens))
    B = len(lens)
    max_blocks, nblk, bt, kp, vp = _pools(rng, B, hkv, hd, lens)
    q = rng.normal(0, 1, (B, hq, hd)).astype(np.float32)
    ln = np.array(lens, np.int32)
    ob = ctx.alloc(B * hq * hd * 2)
    ctx.check(ctx.L.nx_attn_decode_paged_f16(ctx.h, up(ctx, q), up(ctx, kp), up(ctx, vp), up(ctx, bt),
                                             up(ctx, ln), ob, B, hq, hkv, hd, max_blocks, nblk), "attn")
    got = f16(ctx.download(ob, (B, hq, hd), np.uint16))
    want = np.empty_like(q)
    L.nxo_attn_decode_paged_f16(q, np.ascontiguousarray(kp.reshape(-1)), np.ascontiguousarray(vp.reshape(-1)),
                                bt, max_blocks, ln, B, hq, hkv, hd, want)
    for b in range(B):
        assert rel_err(got[b], want[b]) < TOL


def test_attention_rejects_bad_table(ctx):
    rng = np.random.default_rng(1)
    max_blocks, nblk, bt, kp, vp = _pools(rng, 1, 2, 64, [20])
    bad = bt.copy()
    bad[0, 1] = nblk + 5
    q = np.zeros((1, 4, 64), np.float32)
    with pytest.raises(nexus_amd.NxError):
        ctx.check(ctx.L.nx_attn_decode_paged_f16(ctx.h, up(ctx, q), up(ctx, kp), up(ctx, vp), up(ctx, bad),
                                                 up(ctx, np.array([20], np.int32)), ctx.alloc(512), 1, 4, 2, 64,
                                                 max_blocks, nblk), "attn")
    with pytest.raises(nexus_amd.NxError):
        ctx.check(ctx.L.nx_attn_decode_paged_f16(ctx.h, up(ctx, q), up(ctx, kp), up(ctx, vp), up(ctx, bt),
                                                 up(ctx, np.array([max_blocks * 16 + 1], np.int32)),
                                                 ctx.alloc(512), 1, 4, 2, 64, max_blocks, nblk), "attn")


def test_kv_append_bit_exact(ctx):
    rng = np.random.default_rng(5)
    B, hkv, hd, max_blocks = 3, 8, 128, 4
    nblk = B * max_blocks
    perm = np.empty(nblk, np.int32)
    L.nxo_shuffle_perm(perm, nblk, 3, 7)
    bt = np.ascontiguousarray(perm.reshape(B, max_blocks))
    k = rng.normal(0, 10, (B, hkv * hd)).astype(np.float32)
    v = rng.normal(0, 10, (B, hkv * hd)).astype(np.float32)
    k[0, :4] = [65519.0, 1e-7, -6.1e-5, 3e-8]
    pos = np.array([0, 17, 63], np.int32)
    size = nblk * hkv * 16 * hd
    kb, vb = ctx.alloc(size * 2), ctx.alloc(size * 2)
    ctx.check(ctx.L.nx_kv_append_f16(ctx.h, up(ctx, k), up(ctx, v), kb, vb, up(ctx, bt), up(ctx, pos), B, hkv,
                                     hd, max_blocks, nblk), "kv_append")
    kw = np.zeros(size, np.uint16)
    vw = np.zeros(size, np.uint16)
    for b in range(B):
        L.nxo_kv_append_f16(np.ascontiguousarray(k[b]), np.ascontiguousarray(v[b]), kw, vw, bt, max_blocks, b,
                            int(pos[b]), hkv, hd)
    assert np.array_equal(ctx.download(kb, size, np.uint16), kw)
    assert np.array_equal(ctx.download(vb, size, np.uint16), vw)


# ------------------------------------------------------------- TurboQuant --
def _tq_vectors(rng, n):
    x = rng.normal(0, 1, (n, 128)).astype(np.float32)
    x[1] = 0.0
    x[2] *= 1e-20
    x[3] *= 1e4
    ch = rng.choice(128, 4, replace=False)
    x[4:, ch] *= 10.0
    x[5] = np.where(np.arange(128) == 9, 1.0, 0.0)
    return x


def test_tq_encode_bit_exact(ctx):
    rng = np.random.default_rng(6)
    n = 4099
    x = _tq_vectors(rng, n)
    signs = oracle.tq_signs(0x5EED, 0x108)
    c4b, c3b, nb = ctx.alloc(n * 32), ctx.alloc(n * 24), ctx.alloc(n * 2)
    ctx.check(ctx.L.nx_tq_encode(ctx.h, up(ctx, x), up(ctx, signs), c4b, c3b, nb, n), "tq_encode")
    k4, k3, nr, _ = oracle.tq_encode(x, signs)
    assert np.array_equal(ctx.download(c4b, (n, 32), np.uint8), k4)
    assert np.array_equal(ctx.download(c3b, (n, 24), np.uint8), k3)
    assert np.array_equal(ctx.download(nb, n, np.uint16), nr)


def _tq_pools(rng, B, hkv, lens, ks, vs):
    c4, b4 = oracle.codebook(4)
    c3, b3 = oracle.codebook(3)
    max_blocks = max(1, -(-max(lens) // 16)) + 1
    nblk = B * max_blocks
    perm = np.empty(nblk, np.int32)
    L.nxo_shuffle_perm(perm, nblk, 5, 7)
    bt = np.ascontiguousarray(perm.reshape(B, max_blocks))
    nv = nblk * hkv * 16
    pools = [np.zeros((nv, 32), np.uint8), np.zeros((nv, 24), np.uint8), np.zeros(nv, np.uint16),
             np.zeros((nv, 32), np.uint8), np.zeros((nv, 24), np.uint8), np.zeros(nv, np.uint16)]
    for b in range(B):
        n = lens[b]
        # N(0,1) with 4 outlier channels x10 (norms stay inside fp16 range)
        K = rng.normal(0, 1, (n, hkv, 128)).astype(np.float32)
        K[:, :, rng.choice(128, 4, replace=False)] *= 10.0
        V = rng.normal(0, 1, (n, hkv, 128)).astype(np.float32)
        # encode in bulk, then place by the block table
        for src, signs, off in ((K, ks, 0), (V, vs, 3)):
            k4, k3, nr, _ = oracle.tq_encode(src.reshape(-1, 128), signs)
            p = np.repeat(np.arange(n), hkv)
            h = np.tile(np.arange(hkv), n)
            idx = (bt[b, p // 16] * hkv + h) * 16 + p % 16
            pools[off][idx], pools[off + 1][idx], pools[off + 2][idx] = k4, k3, nr
    return max_blocks, nblk, bt, pools, (c4, c3)


@pytest.mark.parametrize("hq,hkv,lens", [(4, 1, [1]), (4, 1, [40]), (32, 8, [300, 17]), (32, 8, [2048]),
                                         (16, 8, [129])])
def test_tq_attention_parity(ctx, hq, hkv, lens):
    rng = np.random.default_rng(hq * 7 + sum(lens))
    B = len(lens)
    ks, vs = oracle.tq_signs(1, 11), oracle.tq_signs(1, 12)
    max_blocks, nblk, bt, pools, (c4, c3) = _tq_pools(rng, B, hkv, lens, ks, vs)
    q = rng.normal(0, 1, (B, hq, 128)).astype(np.float32)
    ln = np.array(lens, np.int32)
    bufs = [up(ctx, p) for p in pools]
    ob = ctx.alloc(B * hq * 128 * 2)
    ctx.check(ctx.L.nx_attn_decode_paged_tq(ctx.h, up(ctx, q), *bufs, up(ctx, ks), up(ctx, vs), up(ctx, bt),
                                            up(ctx, ln), ob, B, hq, hkv, max_blocks, nblk), "attn_tq")
    got = f16(ctx.download(ob, (B, hq, 128), np.uint16))
    want = np.empty_like(q)
    L.nxo_attn_decode_paged_tq(q, *[np.ascontiguousarray(p) for p in pools], ks, vs, c4, c3, bt, max_blocks, ln, B,
                               hq, hkv, want)
    for b in range(B):
        assert rel_err(got[b], want[b]) < TOL


def test_tq_append_bit_exact(ctx):
    rng = np.random.default_rng(8)
    B, hkv, max_blocks = 2, 8, 3
    nblk = B * max_blocks
    bt = np.arange(nblk, dtype=np.int32)[::-1].copy().reshape(B, max_blocks)
    ks, vs = oracle.tq_signs(2, 11), oracle.tq_signs(2, 12)
    _, b4 = oracle.codebook(4)
    _, b3 = oracle.codebook(3)
    k = _tq_vectors(rng, B * hkv).reshape(B, hkv * 128)
    v = rng.normal(0, 1, (B, hkv * 128)).astype(np.float32)
    pos = np.array([5, 40], np.int32)
    nv = nblk * hkv * 16
    bufs = [ctx.alloc(nv * 32), ctx.alloc(nv * 24), ctx.alloc(nv * 2), ctx.alloc(nv * 32), ctx.alloc(nv * 24),
            ctx.alloc(nv * 2)]
    ctx.check(ctx.L.nx_tq_append(ctx.h, up(ctx, k), up(ctx, v), up(ctx, ks), up(ctx, vs), *bufs, up(ctx, bt),
                                 up(ctx, pos), B, hkv, max_blocks, nblk), "tq_append")
    want = [np.zeros((nv, 32), np.uint8), np.zeros((nv, 24), np.uint8), np.zeros(nv, np.uint16),
            np.zeros((nv, 32), np.uint8), np.zeros((nv, 24), np.uint8), np.zeros(nv, np.uint16)]
    for b in range(B):
        L.nxo_tq_append(np.ascontiguousarray(k[b]), np.ascontiguousarray(v[b]), hkv, ks, vs, b4, b3, *want, bt,
                        max_blocks, b, int(pos[b]))
    for buf, w in zip(bufs, want):
        assert np.array_equal(ctx.download(buf, w.shape, w.dtype), w)


# -------------------------------------------------------------------- MoE --
def test_moe_route(ctx):
    rng = np.random.default_rng(9)
    B, E, k = 8, 8, 2
    logits = rng.normal(0, 1, (B, E)).astype(np.float32)
    logits[3] = [0.5, 1.0, 1.0, 1.0, 0, 0, 0, 0]
    ib, wb = ctx.alloc(B * k * 4), ctx.alloc(B * k * 4)
    ctx.check(ctx.L.nx_moe_route_topk(ctx.h, up(ctx, logits), ib, wb, E, k, B), "route")
    ids, w = ctx.download(ib, (B, k), np.int32), ctx.download(wb, (B, k), np.float32)
    for b in range(B):
        oi, ow = np.empty(k, np.int32), np.empty(k, np.float32)
        L.nxo_moe_route(np.ascontiguousarray(logits[b]), E, k, oi, ow)
        assert np.array_equal(ids[b], oi)
        assert np.allclose(w[b], ow, rtol=2e-6, atol=0)


@pytest.mark.parametrize("B,E,k", [(8, 256, 16), (3, 64, 10), (64, 128, 2)])
def test_moe_route_wide(ctx, B, E, k):
    """Routing over up to 256 experts, top-16 and 64 sequences: ids equal the
    oracle's, weights within 2e-6."""
    rng = np.random.default_rng(E * 7 + k)
    logits = (rng.normal(0, 1, (B, E)) * 2).astype(np.float32)
    ib, wb = ctx.alloc(B * k * 4), ctx.alloc(B * k * 4)
    ctx.check(ctx.L.nx_moe_route_topk(ctx.h, up(ctx, logits), ib, wb, E, k, B), "route")
    ids, w = ctx.download(ib, (B, k), np.int32), ctx.download(wb, (B, k), np.float32)
    for b in range(B):
        oi, ow = np.empty(k, np.int32), np.empty(k, np.float32)
        L.nxo_moe_route(np.ascontiguousarray(logits[b]), E, k, oi, ow)
        assert np.array_equal(ids[b], oi)
        assert np.allclose(w[b], ow, rtol=2e-6, atol=0)


def test_moe_expert_ffn(ctx):
    rng = np.random.default_rng(10)
    d, F, E, k, B = 256, 688, 4, 2, 3
    Gd, Gf = d // 32, (F + 31) // 32
    w13 = np.zeros((E, 2 * F, Gd * 16), np.uint8)
    s13 = np.zeros((E, 2 * F, Gd), np.uint16)
    w2 = np.zeros((E, d, Gf * 16), np.uint8)
    s2 = np.zeros((E, d, Gf), np.uint16)
    mats = []
    for e in range(E):
        g, u, dn = (rng.normal(0, 0.02, s).astype(np.float32) for s in ((F, d), (F, d), (d, F)))
        cg, sg = oracle.quantize(g)
        cu, su = oracle.quantize(u)
        cd, sd = oracle.quantize(dn)
        w13[e, 0::2], s13[e, 0::2], w13[e, 1::2], s13[e, 1::2] = cg, sg, cu, su
        w2[e], s2[e] = cd, sd
        mats.append(((cg, sg), (cu, su), (cd, sd)))
    x = rng.normal(0, 1, (B, d)).astype(np.float16)
    ids = np.array([[0, 3], [3, 1], [2, 0]], np.int32)
    wts = rng.uniform(0.1, 0.9, (B, k)).astype(np.float32)
    out0 = rng.normal(0, 1, (B, d)).astype(np.float32)
    ob = up(ctx, out0)
    ctx.check(ctx.L.nx_moe_expert_ffn(ctx.h, up(ctx, x.view(np.uint16)), up(ctx, w13), up(ctx, s13), up(ctx, w2),
                                      up(ctx, s2), up(ctx, ids), up(ctx, wts), ob, d, F, E, k, B, 1), "moe_ffn")
    got = ctx.download(ob, (B, d), np.float32)
    for b in range(B):
        acc = np.zeros(d, np.float32)
        xf = x[b].astype(np.float32)
        for j in range(k):
            (cg, sg), (cu, su), (cd, sd) = mats[ids[b, j]]
            gv, uv = oracle.gemv(cg, sg, xf, F, d)[0], oracle.gemv(cu, su, xf, F, d)[0]
            a = np.empty(F, np.float32)
            L.nxo_swiglu(gv, uv, F, a)
            a = a.astype(np.float16).astype(np.float32)
            acc += wts[b, j] * oracle.gemv(cd, sd, a, d, F)[0]
        assert rel_err(got[b] - out0[b], acc) < TOL


# ------------------------------------------------------------ token graph --
def test_token_batch_graph_matches_eager(ctx):
    rng = np.random.default_rng(11)
    N, K = 512, 1024
    codes, scales = oracle.quantize(rng.normal(0, 0.02, (N, K)).astype(np.float32))
    wb, sb = up(ctx, codes), up(ctx, scales)
    xb, yb, hb = ctx.alloc(K * 2), ctx.alloc(N * 4), ctx.alloc(K * 4)
    for rep in range(4):
        h = rng.normal(0, 1, K).astype(np.float32)
        ctx.upload(h, hb)
        ctx.check(ctx.L.nx_token_begin(ctx.h), "begin")
        ctx.check(ctx.L.nx_rmsnorm(ctx.h, hb, 0, xb, K, 1e-5, 1), "rmsnorm")
        ctx.gemv_f32(xb, wb, sb, yb, N, K, 1)
        ctx.check(ctx.L.nx_token_end(ctx.h), "end")
        got = ctx.download(yb, N, np.float32)
        xn = np.empty(K, np.float32)
        L.nxo_rmsnorm(h, None, K, 1e-5, xn)
        want = oracle.gemv(codes, scales, xn.astype(np.float16).astype(np.float32), N, K)[0]
        assert rel_err(got, want) < TOL
    # ops that cannot be captured are refused inside a token batch
    ctx.check(ctx.L.nx_token_begin(ctx.h), "begin")
    assert ctx.L.nx_upload(ctx.h, hb, 0, h.ctypes.data, 16) == 5
    ctx.check(ctx.L.nx_token_end(ctx.h), "end")
    assert ctx.L.nx_token_end(ctx.h) == 5
