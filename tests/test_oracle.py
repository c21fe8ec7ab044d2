"""CPU tests that pin the oracle before it is trusted as the checker.

Each oracle function is checked against (a) golden vectors produced by the
reference's own functions (tests/golden, see make_golden.py), (b) the live
reference checker oracle/_ref when it is built, and/or (c) what mathematics
fixes: published tables, closed forms and fp64 brute force.
"""
from pathlib import Path

import numpy as np
import pytest

import oracle
from conftest import rel_err

GOLD = Path(__file__).resolve().parent / "golden"
L = oracle.lib


def gold(name):
    return np.load(GOLD / name)


# ------------------------------------------------------------------- fp16 --
def test_f32_to_f16_rne_matches_ieee():
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    vals = bits.view(np.float32)
    vals = vals[np.isfinite(vals)]
    edge = np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, 6.1035156e-05, 6.097555e-05,
                     5.9604645e-08, 2.9802322e-08, 2.9802326e-08, 8.940697e-08, 1.0009766,
                     1.0004883, -1.0004883, 2049.0, 2051.0], np.float32)
    for v in (vals, edge, rng.normal(0, 1, 50000).astype(np.float32)):
        got = oracle.f16_bits(v)
        want = v.astype(np.float16).view(np.uint16)  # numpy rounds to nearest even
        assert np.array_equal(got, want)


def test_f16_to_f32_exact_all_values():
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = np.array([L.nxo_f16_to_f32(int(h)) for h in allh[::7]], np.float32)
    want = allh[::7].view(np.float16).astype(np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))


def test_reference_kv_conversion_golden():
    g = gold("kv_fp16.npz")
    got = np.array([L.nxo_f32_to_f16_trunc(float(v)) for v in g["f32"]], np.uint16)
    assert np.array_equal(got, g["f16_trunc"])
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    back = np.array([L.nxo_f16_to_f32_ref(int(h)) for h in allh], np.float32)
    ref = g["f16_to_f32"]
    # NaN payloads do not survive the trip through a Python float; compare the rest bitwise
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(back), nan)
    assert np.array_equal(back[~nan].view(np.uint32), ref[~nan].view(np.uint32))


# -------------------------------------------------------------------- RNG --
def test_rng_determinism_and_moments():
    a = oracle.gen_normal(1 << 20, 7, 123, 0.02)
    b = oracle.gen_normal(1 << 20, 7, 123, 0.02)
    c = oracle.gen_normal(1 << 20, 7, 124, 0.02)
    assert np.array_equal(a, b)
    assert not np.array_equal(a, c)
    assert abs(a.mean()) < 1e-4
    assert abs(a.std() / 0.02 - 1) < 3e-3
    # Irwin-Hall(4): excess kurtosis -0.3, bounded support |z| <= sqrt(12)
    z = a.astype(np.float64) / 0.02
    kurt = np.mean(z**4) / np.mean(z**2) ** 2 - 3
    assert abs(kurt + 0.3) < 0.02
    assert np.max(np.abs(z)) <= np.sqrt(12) + 1e-3


def test_gen_quant_rows_matches_full_generation():
    K, N = 96, 40
    w = oracle.gen_normal(N * K, 3, 9, 0.02).reshape(N, K)
    codes, scales = oracle.quantize(w)
    c2, s2 = oracle.gen_quant_rows(11, 17, K, 3, 9, 0.02)
    assert np.array_equal(c2, codes[11:28])
    assert np.array_equal(s2, scales[11:28])


# -------------------------------------------------------------- int4 g32 --
def test_dequant_int4_golden():
    g = gold("dequant_int4.npz")
    scales16 = g["scales"].astype(np.float16).view(np.uint16)
    codes = np.ascontiguousarray(g["data"][None, :])
    out = oracle.dequantize(codes, scales16[None, :], 1, 256)
    assert np.array_equal(out[0].view(np.uint32), g["out"].view(np.uint32))


def test_dequant_int4_live_reference():
    R = oracle.ref()
    if R is None:
        pytest.skip("reference checker not built")
    rng = np.random.default_rng(5)
    data = rng.integers(0, 256, 512, dtype=np.uint8)
    s16 = rng.uniform(1e-4, 1, 32).astype(np.float16)
    out_ref = np.empty(1024, np.float32)
    R.ref_dequant_int4(out_ref, data, s16.astype(np.float32), np.full(32, 8.0, np.float32), 1024, 32)
    out = oracle.dequantize(data[None, :], s16.view(np.uint16)[None, :], 1, 1024)
    assert np.array_equal(out[0].view(np.uint32), out_ref.view(np.uint32))


def test_unpack_int4_all_bytes():
    allb = np.arange(256, dtype=np.uint8)
    codes = np.empty(512, np.uint8)
    L.nxo_unpack_int4(allb, 512, codes)
    assert np.array_equal(codes[0::2], allb & 15)
    assert np.array_equal(codes[1::2], allb >> 4)


@pytest.mark.parametrize("K", [32, 96, 688, 4096])
def test_quantizer_invariants(K):
    rng = np.random.default_rng(K)
    N = 33
    w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    w[3] = 0.0
    w[5, :7] = 0.5  # outliers in one group
    codes, scales = oracle.quantize(w)
    deq = oracle.dequantize(codes, scales, N, K)
    s = scales.view(np.float16).astype(np.float32)
    s_el = np.repeat(s, 32, axis=1)[:, :K]
    assert np.all(np.abs(deq - w) <= s_el * 0.5000001 + 1e-12)
    assert np.all(scales[3] == 0) and np.all(deq[3] == 0)
    # codes of a ragged tail hold 8
    G = (K + 31) // 32
    if K % 32:
        un = np.empty(G * 32 * N, np.uint8)
        L.nxo_unpack_int4(np.ascontiguousarray(codes), un.size, un)
        un = un.reshape(N, G * 32)
        assert np.all(un[:, K:] == 8)


@pytest.mark.parametrize("N,K,B", [(64, 96, 1), (256, 688, 2), (128, 4096, 3)])
def test_gemv_vs_fp64(N, K, B):
    rng = np.random.default_rng(N + K)
    w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    codes, scales = oracle.quantize(w)
    x = rng.normal(0, 1, (B, K)).astype(np.float16).astype(np.float32)
    y = oracle.gemv(codes, scales, x, N, K)
    deq = oracle.dequantize(codes, scales, N, K).astype(np.float64)
    want = x.astype(np.float64) @ deq.T
    assert rel_err(y, want) < 1e-5


# ------------------------------------------------------------ elementwise --
def test_rmsnorm_vs_fp64():
    rng = np.random.default_rng(2)
    x = rng.normal(0, 3, 4096).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 4096).astype(np.float32)
    out = np.empty_like(x)
    L.nxo_rmsnorm(x, w.ctypes.data, 4096, 1e-5, out)
    xd = x.astype(np.float64)
    want = xd / np.sqrt(np.mean(xd**2) + 1e-5) * w
    assert rel_err(out, want) < 1e-6


def test_head_rmsnorm_vs_fp64():
    """The Q/K norm (hybrid_model.cpp:1325-1349): every head_dim slice is
    normalized by its own RMS with the shared head_dim weights.  Heads of
    scales 1e-2 .. 1e2 make a norm over the whole vector (or over the wrong
    slice) fail; with unit weights each head's RMS is sqrt(m / (m + eps)), m
    its mean square."""
    heads, hd, eps = 5, 128, 1e-5
    rng = np.random.default_rng(12)
    x = (rng.normal(0, 1, (heads, hd)) * (10.0 ** np.arange(-2, 3))[:, None]).astype(np.float32)
    w = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    y = x.reshape(-1).copy()
    L.nxo_head_rmsnorm(y, heads, hd, w.ctypes.data, eps)
    xd = x.astype(np.float64)
    ms = np.mean(xd ** 2, axis=1, keepdims=True)
    want = xd / np.sqrt(ms + eps) * w
    assert rel_err(y.reshape(heads, hd), want) < 1e-6
    for h in range(heads):  # per head, not only overall
        assert rel_err(y.reshape(heads, hd)[h], want[h]) < 1e-6
    whole = xd / np.sqrt(np.mean(xd ** 2) + eps) * w
    assert rel_err(y.reshape(heads, hd), whole) > 0.5
    u = x.reshape(-1).copy()
    L.nxo_head_rmsnorm(u, heads, hd, None, eps)
    rms = np.sqrt(np.mean(u.reshape(heads, hd).astype(np.float64) ** 2, axis=1))
    assert np.allclose(rms, np.sqrt(ms[:, 0] / (ms[:, 0] + eps)), rtol=1e-6, atol=0)


def test_rope_is_complex_rotation():
    hd, heads, pos, theta = 64, 3, 37, 10000.0
    cos = np.empty((128, hd // 2), np.float32)
    sin = np.empty((128, hd // 2), np.float32)
    L.nxo_rope_table(128, hd, theta, cos, sin)
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, heads * hd).astype(np.float32)
    y = x.copy()
    L.nxo_rope(y, heads, hd, pos, cos, sin)
    z = x.astype(np.float64).reshape(heads, hd // 2, 2)
    zc = z[..., 0] + 1j * z[..., 1]
    ang = pos * theta ** (-(2.0 * np.arange(hd // 2)) / hd)
    r = zc * np.exp(1j * ang)
    want = np.stack([r.real, r.imag], -1).reshape(-1)
    assert rel_err(y, want) < 1e-6
    # position 0 is the identity
    y0 = x.copy()
    L.nxo_rope(y0, heads, hd, 0, cos, sin)
    assert np.array_equal(y0, x)


def test_swiglu_vs_fp64():
    rng = np.random.default_rng(4)
    g = rng.normal(0, 3, 1000).astype(np.float32)
    u = rng.normal(0, 1, 1000).astype(np.float32)
    out = np.empty_like(g)
    L.nxo_swiglu(g, u, 1000, out)
    gd = g.astype(np.float64)
    want = gd / (1 + np.exp(-gd)) * u
    assert rel_err(out, want) < 1e-6


def test_argmax_first_maximum():
    v = np.array([1.0, 3.0, -2.0, 3.0, 0.5], np.float32)
    assert L.nxo_argmax(v, 5) == 1


# -------------------------------------------------------- paged attention --
def _attn_fp64(q, K, V, hq, hkv, hd):
    grp = hq // hkv
    out = np.zeros((hq, hd))
    for h in range(hq):
        kvh = h // grp
        s = K[:, kvh, :] @ q[h] / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = p @ V[:, kvh, :]
    return out


def _paged_setup(rng, B, hkv, hd, max_blocks, ctx_lens):
    nblk = B * max_blocks
    perm = np.empty(nblk, np.int32)
    L.nxo_shuffle_perm(perm, nblk, 11, 7)
    bt = np.ascontiguousarray(perm.reshape(B, max_blocks))
    kpool = np.zeros(nblk * hkv * 16 * hd, np.uint16)
    vpool = np.zeros_like(kpool)
    raw = []
    for b in range(B):
        K = rng.normal(0, 1, (ctx_lens[b], hkv, hd)).astype(np.float32)
        V = rng.normal(0, 1, (ctx_lens[b], hkv, hd)).astype(np.float32)
        for p in range(ctx_lens[b]):
            L.nxo_kv_append_f16(np.ascontiguousarray(K[p]), np.ascontiguousarray(V[p]), kpool, vpool,
                                bt, max_blocks, b, p, hkv, hd)
        raw.append((K, V))
    return bt, kpool, vpool, raw


@pytest.mark.parametrize("hq,hkv,hd", [(4, 2, 64), (8, 2, 128), (8, 2, 256)])
def test_paged_attention_vs_fp64(hq, hkv, hd):
    rng = np.random.default_rng(hq * hd)
    B, max_blocks = 3, 4
    ctx = np.array([1, 17, 64], np.int32)
    bt, kp, vp, raw = _paged_setup(rng, B, hkv, hd, max_blocks, ctx)
    q = rng.normal(0, 1, (B, hq, hd)).astype(np.float32)
    out = np.empty_like(q)
    L.nxo_attn_decode_paged_f16(q, kp, vp, bt, max_blocks, ctx, B, hq, hkv, hd, out)
    for b in range(B):
        K, V = raw[b]
        Kh = K.astype(np.float16).astype(np.float64)
        Vh = V.astype(np.float16).astype(np.float64)
        want = _attn_fp64(q[b].astype(np.float64), Kh, Vh, hq, hkv, hd)
        assert rel_err(out[b], want) < 1e-5


def test_paged_gather_golden_and_shuffle_invariance():
    g = gold("paged_gather.npz")
    hkv, hd = int(g["hkv"]), int(g["hd"])
    # the reference gather returns positions in order: contiguous == input
    assert np.array_equal(g["k_out"], g["k"]) and np.array_equal(g["v_out"], g["v"])
    npos = g["k"].shape[0]
    max_blocks = (npos + 15) // 16
    for seed in (1, 2, 3):
        perm = np.empty(max_blocks, np.int32)
        L.nxo_shuffle_perm(perm, max_blocks, seed, 7)
        kp = np.zeros(max_blocks * hkv * 16 * hd, np.uint16)
        vp = np.zeros_like(kp)
        for p in range(npos):
            L.nxo_kv_append_f16(np.ascontiguousarray(g["k"][p]), np.ascontiguousarray(g["v"][p]),
                                kp, vp, perm, max_blocks, 0, p, hkv, hd)
        q = np.random.default_rng(seed).normal(0, 1, (1, 2 * hkv, hd)).astype(np.float32)
        out = np.empty_like(q)
        L.nxo_attn_decode_paged_f16(q, kp, vp, perm, max_blocks, np.array([npos], np.int32), 1,
                                    2 * hkv, hkv, hd, out)
        Kc = g["k_out"].astype(np.float16).astype(np.float32)
        Vc = g["v_out"].astype(np.float16).astype(np.float32)
        want = np.empty_like(q)
        L.nxo_attn_decode_contig(np.ascontiguousarray(q[0]), np.ascontiguousarray(Kc),
                                 np.ascontiguousarray(Vc), npos, 2 * hkv, hkv, hd, want[0])
        assert np.array_equal(out, want)


# ------------------------------------------------------------- TurboQuant --
# Max (1960) Lloyd-Max quantizers for N(0, 1), output levels (positive half).
MAX_8 = [0.2451, 0.7560, 1.3440, 2.1520]
MAX_16 = [0.1284, 0.3881, 0.6568, 0.9424, 1.2562, 1.6181, 2.0690, 2.7326]


def test_codebook_matches_reference_golden():
    g = gold("tq_codebook.npz")
    for bits in (3, 4):
        c, b = oracle.codebook(bits)
        assert np.array_equal(c.view(np.uint32), g[f"c{bits}"].view(np.uint32))
        assert np.array_equal(b.view(np.uint32), g[f"b{bits}"].view(np.uint32))


def test_codebook_live_reference():
    R = oracle.ref()
    if R is None:
        pytest.skip("reference checker not built")
    for d in (64, 128, 256):
        for bits in (2, 3, 4):
            n = 1 << bits
            c, b = np.empty(n, np.float32), np.empty(n - 1, np.float32)
            rc, rb = np.empty(n, np.float32), np.empty(n - 1, np.float32)
            L.nxo_tq_codebook(d, bits, c, b)
            R.ref_tq_codebook(d, bits, rc, rb)
            assert np.array_equal(c.view(np.uint32), rc.view(np.uint32))
            assert np.array_equal(b.view(np.uint32), rb.view(np.uint32))


def test_codebook_is_lloyd_max_iteration():
    """The codebook is the Lloyd-Max iteration for N(0, 1/128) run from a
    uniform start in +-3 sigma with +-10 sigma tails for at most 100 steps
    (it stops short of the fixed point, as the reference does); checked in
    fp64 with scipy's normal pdf/cdf, and against Max's (1960) table."""
    from scipy.stats import norm
    sigma = 1 / np.sqrt(128)
    for bits, table in ((3, MAX_8), (4, MAX_16)):
        n = 1 << bits
        c, b = oracle.codebook(bits)
        c64 = c.astype(np.float64)
        assert np.allclose(b, 0.5 * (c64[:-1] + c64[1:]), atol=1e-7)
        cm = -3 * sigma + 6 * sigma * (np.arange(n) + 0.5) / n
        for _ in range(100):
            bd = 0.5 * (cm[:-1] + cm[1:])
            edges = np.concatenate([[-10 * sigma], bd, [10 * sigma]])
            new = sigma**2 * (norm.pdf(edges[:-1], scale=sigma) - norm.pdf(edges[1:], scale=sigma)) / (
                norm.cdf(edges[1:], scale=sigma) - norm.cdf(edges[:-1], scale=sigma))
            delta = np.max(np.abs(new - cm))
            cm = new
            if delta < 1e-7 * sigma:
                break
        assert np.allclose(c64, cm, atol=2e-6)
        half = np.sort(np.abs(c64))[::2] * np.sqrt(128)
        assert np.allclose(half, table, atol=2e-2)


def test_encode_rule_golden():
    g = gold("tq_encode.npz")
    for bits in (3, 4):
        _, b = oracle.codebook(bits)
        got = np.array([L.nxo_tq_encode_scalar(float(x), b, 1 << bits) for x in g[f"x{bits}"]], np.uint8)
        assert np.array_equal(got, g[f"code{bits}"])


def test_pack_golden_and_roundtrip():
    g = gold("tq_pack.npz")
    for bits in (3, 4):
        for n in (8, 37, 64, 128):
            codes = g[f"codes_{bits}_{n}"]
            packed = np.zeros((n * bits + 7) // 8, np.uint8)
            L.nxo_pack_codes(packed, np.ascontiguousarray(codes), n, bits)
            assert np.array_equal(packed, g[f"packed_{bits}_{n}"])
            back = np.empty(n, np.uint8)
            L.nxo_unpack_codes(back, packed, n, bits)
            assert np.array_equal(back, codes)


def test_quantize_composition_golden():
    """norm -> normalize -> encode -> pack, as TurboQuantKV::quantize does it."""
    g = gold("tq_quantize.npz")
    for bits in (3, 4):
        _, b = oracle.codebook(bits)
        x = g[f"x{bits}"]
        nbytes = (128 * bits + 7) // 8
        for v in range(x.shape[0]):
            nrm = g[f"norms{bits}"][v]
            assert np.isclose(nrm, np.sqrt(np.sum(x[v].astype(np.float64) ** 2)), rtol=1e-6)
            if nrm > 1e-12:
                inv = np.float32(1.0) / np.float32(nrm)
                y = (x[v] * inv).astype(np.float32)
            else:
                y = np.zeros(128, np.float32)
            codes = np.array([L.nxo_tq_encode_scalar(float(t), b, 1 << bits) for t in y], np.uint8)
            packed = np.zeros(nbytes, np.uint8)
            L.nxo_pack_codes(packed, codes, 128, bits)
            assert np.array_equal(packed, g[f"packed{bits}"][v * nbytes:(v + 1) * nbytes])


def test_fwht_is_sylvester_hadamard():
    from scipy.linalg import hadamard
    H = hadamard(128).astype(np.float64)
    u = np.random.default_rng(6).normal(0, 1, 128).astype(np.float32)
    v = u.copy()
    L.nxo_fwht128(v)
    assert rel_err(v, H @ u.astype(np.float64)) < 1e-6
    L.nxo_fwht128(v)  # H H = 128 I
    assert rel_err(v / 128.0, u) < 1e-6


def test_tq_sumsq_tree_is_exact_sum():
    x = np.random.default_rng(7).normal(0, 1, 128).astype(np.float32)
    assert np.isclose(L.nxo_tq_sumsq(x), np.sum(x.astype(np.float64) ** 2), rtol=1e-6)


def test_tq_roundtrip_distortion():
    rng = np.random.default_rng(8)
    x = rng.normal(0, 1, (2000, 128)).astype(np.float32)
    signs = oracle.tq_signs(5, 0x108)
    k4, k3, nr, cu = oracle.tq_encode(x, signs)
    xh = oracle.tq_decode(k4, k3, nr, signs)
    err = np.sum((xh - x) ** 2, 1) / np.sum(x**2, 1)
    # Gaussian Lloyd-Max distortion: 0.009497 (16 levels), 0.03454 (8 levels); average 0.0220
    assert 0.018 < err.mean() < 0.026
    # the codes index both halves correctly and the norm is stored in fp16
    assert cu[:, :64].max() <= 15 and cu[:, 64:].max() <= 7
    assert np.allclose(nr.view(np.float16).astype(np.float32), np.linalg.norm(x, axis=1), rtol=1e-3)
    # zero vector -> norm 0, reconstruction 0
    z = np.zeros((1, 128), np.float32)
    zk4, zk3, znr, _ = oracle.tq_encode(z, signs)
    assert znr[0] == 0 and np.all(oracle.tq_decode(zk4, zk3, znr, signs) == 0)


def test_tq_rotated_domain_identity():
    """<Pi q, c> * n == <q, n Pi^T c>: the score the GPU computes without inverse-rotating K."""
    from scipy.linalg import hadamard
    rng = np.random.default_rng(9)
    signs = oracle.tq_signs(5, 0x108).astype(np.float64)
    x = rng.normal(0, 1, (64, 128)).astype(np.float32)
    k4, k3, nr, cu = oracle.tq_encode(x, signs.astype(np.float32))
    khat = oracle.tq_decode(k4, k3, nr, signs.astype(np.float32)).astype(np.float64)
    c4, _ = oracle.codebook(4)
    c3, _ = oracle.codebook(3)
    cvals = np.where(np.arange(128) < 64, c4[np.minimum(cu, 15)], c3[np.minimum(cu, 7)]).astype(np.float64)
    H = hadamard(128).astype(np.float64) / np.sqrt(128)
    q = rng.normal(0, 1, 128)
    qrot = H @ (signs * q)
    s_rot = (cvals @ qrot) * nr.view(np.float16).astype(np.float64)
    s_dir = khat @ q
    assert rel_err(s_rot, s_dir) < 1e-5


def test_tq_attention_close_to_fp16_attention():
    """Quantization error of 3.5-bit KV on attention output stays moderate."""
    rng = np.random.default_rng(10)
    hq, hkv, ctx = 4, 1, 48
    K = rng.normal(0, 1, (ctx, hkv, 128)).astype(np.float32)
    V = rng.normal(0, 1, (ctx, hkv, 128)).astype(np.float32)
    q = rng.normal(0, 0.3, (1, hq, 128)).astype(np.float32)
    ks, vs = oracle.tq_signs(1, 1), oracle.tq_signs(1, 2)
    c4, b4 = oracle.codebook(4)
    c3, b3 = oracle.codebook(3)
    max_blocks = 3
    bt = np.array([[2, 0, 1]], np.int32)
    nv = max_blocks * hkv * 16
    kc4, kc3, kn = np.zeros((nv, 32), np.uint8), np.zeros((nv, 24), np.uint8), np.zeros(nv, np.uint16)
    vc4, vc3, vn = np.zeros_like(kc4), np.zeros_like(kc3), np.zeros_like(kn)
    for p in range(ctx):
        L.nxo_tq_append(np.ascontiguousarray(K[p]), np.ascontiguousarray(V[p]), hkv, ks, vs, b4, b3,
                        kc4, kc3, kn, vc4, vc3, vn, bt, max_blocks, 0, p)
    out = np.empty_like(q)
    L.nxo_attn_decode_paged_tq(q, kc4, kc3, kn, vc4, vc3, vn, ks, vs, c4, c3, bt, max_blocks,
                               np.array([ctx], np.int32), 1, hq, hkv, out)
    want = _attn_fp64(q[0].astype(np.float64), K.astype(np.float64), V.astype(np.float64), hq, hkv, 128)
    assert rel_err(out[0], want) < 0.25


def _tq_decode_fp64(k4, k3, nr, signs):
    """Independent float64 decode: unpack LSB-first with numpy, codebook
    values, scipy's Hadamard matrix, x = n * D * H c / sqrt(128)."""
    from scipy.linalg import hadamard
    c4, _ = oracle.codebook(4)
    c3, _ = oracle.codebook(3)
    b4 = np.unpackbits(k4, axis=1, bitorder="little").reshape(-1, 64, 4)
    q4 = b4[..., 0] | (b4[..., 1] << 1) | (b4[..., 2] << 2) | (b4[..., 3] << 3)
    b3 = np.unpackbits(k3, axis=1, bitorder="little").reshape(-1, 64, 3)
    q3 = b3[..., 0] | (b3[..., 1] << 1) | (b3[..., 2] << 2)
    cv = np.concatenate([c4[q4], c3[q3]], axis=1).astype(np.float64)
    H = hadamard(128).astype(np.float64) / np.sqrt(128)
    n = oracle.f16_to_f32(nr).astype(np.float64)
    return (cv @ H) * signs.astype(np.float64) * n[:, None]


def test_tq_paged_attention_vs_fp64_decode():
    """nxo_attn_decode_paged_tq as a whole: two kv heads, two sequences of
    ragged length, a shuffled block table; against float64 attention over
    an independent float64 decode of the stored codes, within 1e-5.  Reading
    V with the K signs (the planted mistake) moves the restatement far past
    the bound."""
    rng = np.random.default_rng(31)
    hq, hkv, B = 8, 2, 2
    lens = [45, 70]
    max_blocks = 5
    bt = rng.permutation(B * max_blocks).astype(np.int32).reshape(B, max_blocks)
    ks, vs = oracle.tq_signs(6, 1), oracle.tq_signs(6, 2)
    c4, b4 = oracle.codebook(4)
    c3, b3 = oracle.codebook(3)
    nv = B * max_blocks * hkv * 16
    kc4, kc3, kn = np.zeros((nv, 32), np.uint8), np.zeros((nv, 24), np.uint8), np.zeros(nv, np.uint16)
    vc4, vc3, vn = np.zeros_like(kc4), np.zeros_like(kc3), np.zeros_like(kn)
    Ks = [rng.normal(0, 1, (n, hkv, 128)).astype(np.float32) for n in lens]
    Vs = [rng.normal(0, 1, (n, hkv, 128)).astype(np.float32) for n in lens]
    for b in range(B):
        for p in range(lens[b]):
            L.nxo_tq_append(np.ascontiguousarray(Ks[b][p]), np.ascontiguousarray(Vs[b][p]), hkv, ks, vs, b4, b3,
                            kc4, kc3, kn, vc4, vc3, vn, bt, max_blocks, b, p)
    q = rng.normal(0, 0.5, (B, hq, 128)).astype(np.float32)
    out = np.empty_like(q)
    L.nxo_attn_decode_paged_tq(q, kc4, kc3, kn, vc4, vc3, vn, ks, vs, c4, c3, bt, max_blocks,
                               np.array(lens, np.int32), B, hq, hkv, out)

    def want_for(vsign):
        res = []
        for b in range(B):
            idx = np.array([[(bt[b, p // 16] * hkv + h) * 16 + p % 16 for h in range(hkv)] for p in range(lens[b])])
            K = _tq_decode_fp64(kc4[idx.ravel()], kc3[idx.ravel()], kn[idx.ravel()], ks).reshape(lens[b], hkv, 128)
            V = _tq_decode_fp64(vc4[idx.ravel()], vc3[idx.ravel()], vn[idx.ravel()], vsign).reshape(lens[b], hkv, 128)
            res.append(_attn_fp64(q[b].astype(np.float64), K, V, hq, hkv, 128))
        return np.stack(res)

    want = want_for(vs)
    assert rel_err(out, want) < 1e-5
    assert rel_err(want_for(ks), want) > 1e-2


def test_tiered_cold_boundary():
    """Attention over ctx positions reads as compressed the pages wholly
    before the window of the H positions preceding the current one:
    cold = 16 floor((ctx - 1 - H) / 16), 0 while ctx <= H + 16."""
    for ctx, H, want in [(1, 16, 0), (16, 16, 0), (32, 16, 0), (33, 16, 16), (48, 16, 16), (49, 16, 32),
                         (300, 64, 224), (4096, 4096, 0), (32768, 4096, 28656), (32769, 4096, 28672)]:
        assert L.nxo_tiered_cold(ctx, H) == want, (ctx, H)


@pytest.mark.parametrize("ctx,H", [(100, 32), (41, 16), (20, 48), (16, 16)])
def test_tiered_attention_vs_fp64(ctx, H):
    """Tiered pages against an independent float64 restatement: positions
    before cold read as the TurboQuant round trip of their fp16 values,
    the rest as fp16, one softmax over all.  A cold boundary one page off
    (the planted mistake below) moves the result well past the bound."""
    rng = np.random.default_rng(ctx + H)
    hq, hkv, B = 4, 2, 2
    K = rng.normal(0, 1, (B, ctx, hkv, 128)).astype(np.float32)
    V = rng.normal(0, 1, (B, ctx, hkv, 128)).astype(np.float32)
    q = rng.normal(0, 0.4, (B, hq, 128)).astype(np.float32)
    ks, vs = oracle.tq_signs(3, 1), oracle.tq_signs(3, 2)
    c4, b4 = oracle.codebook(4)
    c3, b3 = oracle.codebook(3)
    max_blocks = (ctx + 15) // 16 + 1
    bt = rng.permutation(B * max_blocks).astype(np.int32).reshape(B, max_blocks)
    nv = B * max_blocks * hkv * 16
    kp, vp = np.zeros(nv * 128, np.uint16), np.zeros(nv * 128, np.uint16)
    kc4, kc3, kn = np.zeros((nv, 32), np.uint8), np.zeros((nv, 24), np.uint8), np.zeros(nv, np.uint16)
    vc4, vc3, vn = np.zeros_like(kc4), np.zeros_like(kc3), np.zeros_like(kn)
    for b in range(B):
        for p in range(ctx):
            L.nxo_tiered_append(np.ascontiguousarray(K[b, p]), np.ascontiguousarray(V[b, p]), hkv, ks, vs, b4,
                                b3, kp, vp, kc4, kc3, kn, vc4, vc3, vn, bt, max_blocks, b, p)
    out = np.empty_like(q)
    L.nxo_attn_decode_tiered(q, kp, vp, kc4, kc3, kn, vc4, vc3, vn, ks, vs, c4, c3, bt, max_blocks,
                             np.full(B, ctx, np.int32), H, B, hq, hkv, out)

    def want_for(cold):
        Kf = K.astype(np.float16).astype(np.float64)
        Vf = V.astype(np.float16).astype(np.float64)
        for b in range(B):
            for h in range(hkv):
                if cold:
                    rk = oracle.tq_decode(*oracle.tq_encode(K[b, :cold, h].astype(np.float16).astype(np.float32), ks)[:3], ks)
                    rv = oracle.tq_decode(*oracle.tq_encode(V[b, :cold, h].astype(np.float16).astype(np.float32), vs)[:3], vs)
                    Kf[b, :cold, h], Vf[b, :cold, h] = rk, rv
        return np.stack([_attn_fp64(q[b].astype(np.float64), Kf[b], Vf[b], hq, hkv, 128) for b in range(B)])

    cold = max(0, (ctx - 1 - H) // 16 * 16)
    want = want_for(cold)
    e = rel_err(out, want)
    assert e < 1e-5, e
    if cold + 16 <= ctx:
        assert rel_err(want_for(cold + 16), want) > 1e-3


# ------------------------------------------------------------ Cool tier --
def _unpack3_lsb(cc):
    """[n][48] bytes -> [n][128] 3-bit codes, LSB-first (numpy's bit order)."""
    bits = np.unpackbits(cc, axis=1, bitorder="little").reshape(cc.shape[0], 128, 3)
    return (bits[:, :, 0] | (bits[:, :, 1] << 1) | (bits[:, :, 2] << 2)).astype(np.uint8)


def _rotated(x, signs):
    from scipy.linalg import hadamard
    H = hadamard(128).astype(np.float64) / np.sqrt(128)
    x = x.astype(np.float64)
    n = np.linalg.norm(x, axis=1, keepdims=True)
    return (H @ (signs.astype(np.float64) * x / n).T).T, n[:, 0]


def test_cool_codes_vs_hadamard_fp64():
    """Cool codes: every coordinate of y = H D x / (|x| sqrt(128)) coded by
    the 8-level boundaries (first j with y < b_j), packed 3 bits LSB-first
    in 48 bytes; norm fp16(|x|).  Checked against an fp64 restatement with
    scipy's Hadamard matrix and numpy's bit unpacking; codes may differ only
    where y lies within 1e-5 of a boundary."""
    rng = np.random.default_rng(21)
    x = rng.normal(0, 1, (300, 128)).astype(np.float32)
    x[:, [3, 77]] *= 10.0
    signs = oracle.tq_signs(7, 0x208)
    cc, nr = oracle.cool_encode(x, signs)
    y, n = _rotated(x, signs)
    _, b3 = oracle.codebook(3)
    want = np.searchsorted(b3.astype(np.float64), y, side="right").astype(np.uint8)
    got = _unpack3_lsb(cc)
    near = np.min(np.abs(y[..., None] - b3.astype(np.float64)), axis=-1) < 1e-5
    assert np.array_equal(got[~near], want[~near])
    assert (got == want).mean() > 0.999
    assert np.array_equal(nr, oracle.f16_bits(n.astype(np.float32)))
    # the first 64 coordinates fill bytes 0..23 exactly (two 24-byte halves)
    lo = np.unpackbits(cc[:, :24], axis=1, bitorder="little").reshape(-1, 64, 3)
    assert np.array_equal(lo[:, :, 0] | (lo[:, :, 1] << 1) | (lo[:, :, 2] << 2), got[:, :64])


def test_cool_roundtrip_distortion():
    """3-bit codes on every coordinate: the Gaussian 8-level Lloyd-Max
    distortion 0.03454 per unit variance (the 3.5-bit form sits at 0.022)."""
    rng = np.random.default_rng(22)
    x = rng.normal(0, 1, (2000, 128)).astype(np.float32)
    signs = oracle.tq_signs(7, 0x209)
    cc, nr = oracle.cool_encode(x, signs)
    xh = oracle.cool_decode(cc, nr, signs)
    err = np.sum((xh - x) ** 2, 1) / np.sum(x**2, 1)
    assert 0.030 < err.mean() < 0.039
    z = np.zeros((1, 128), np.float32)
    zc, zn = oracle.cool_encode(z, signs)
    assert zn[0] == 0 and np.all(oracle.cool_decode(zc, zn, signs) == 0)


def test_tq_to_cool_is_nearest_code_of_warm_values():
    """Warm -> Cool decodes the 3.5-bit vector and encodes it Cool.  The
    rotation is orthonormal, so in exact arithmetic the Cool coordinates are
    the Warm codebook values over their norm, c / |c|: the Cool codes equal
    the 8-level codes of c / |c| (away from boundaries), and the Cool norm is
    the Warm norm times |c|."""
    rng = np.random.default_rng(23)
    x = rng.normal(0, 1, (400, 128)).astype(np.float32)
    signs = oracle.tq_signs(7, 0x20A)
    k4, k3, nr, cu = oracle.tq_encode(x, signs)
    cc, cn = oracle.tq_to_cool(k4, k3, nr, signs)
    c4, _ = oracle.codebook(4)
    c3, b3 = oracle.codebook(3)
    cv = np.where(np.arange(128) < 64, c4[np.minimum(cu, 15)], c3[np.minimum(cu, 7)]).astype(np.float64)
    cnorm = np.linalg.norm(cv, axis=1)
    y = cv / cnorm[:, None]
    want = np.searchsorted(b3.astype(np.float64), y, side="right").astype(np.uint8)
    got = _unpack3_lsb(cc)
    near = np.min(np.abs(y[..., None] - b3.astype(np.float64)), axis=-1) < 1e-5
    assert np.array_equal(got[~near], want[~near])
    wn = oracle.f16_to_f32(nr).astype(np.float64) * cnorm * np.sqrt(128) * 0.08838834764831845
    assert np.allclose(oracle.f16_to_f32(cn), wn, rtol=2e-3)


def test_tiered_cool_boundary():
    """cool = 16 floor((ctx - 1 - H - W) / 16) clamped at 0; no Cool tier
    when W is 0."""
    for ctx, H, W, want in [(1, 16, 16, 0), (48, 16, 16, 0), (49, 16, 16, 16), (300, 64, 32, 192),
                            (32768, 4096, 4096, 24560), (32769, 4096, 4096, 24576), (5000, 16, 0, 0)]:
        assert L.nxo_tiered_cool(ctx, H, W) == want, (ctx, H, W)
        assert L.nxo_tiered_cool(ctx, H, W) <= L.nxo_tiered_cold(ctx, H)


@pytest.mark.parametrize("ctx,H,W", [(130, 32, 16), (90, 16, 48), (40, 16, 16), (70, 48, 32)])
def test_tiered_cool_attention_vs_fp64(ctx, H, W):
    """Three tiers against an independent float64 restatement: positions
    before cool read as the Cool round trip of the Warm round trip of their
    fp16 values, [cool, cold) as the Warm round trip, the rest fp16, one
    softmax over all.  Moving the Cool boundary by one page (the planted
    mistake) moves the result past the bound."""
    rng = np.random.default_rng(ctx * 3 + H + W)
    hq, hkv, B = 4, 2, 2
    K = rng.normal(0, 1, (B, ctx, hkv, 128)).astype(np.float32)
    V = rng.normal(0, 1, (B, ctx, hkv, 128)).astype(np.float32)
    q = rng.normal(0, 0.4, (B, hq, 128)).astype(np.float32)
    ks, vs = oracle.tq_signs(4, 1), oracle.tq_signs(4, 2)
    c4, b4 = oracle.codebook(4)
    c3, b3 = oracle.codebook(3)
    max_blocks = (ctx + 15) // 16 + 1
    bt = rng.permutation(B * max_blocks).astype(np.int32).reshape(B, max_blocks)
    nv = B * max_blocks * hkv * 16
    kp, vp = np.zeros(nv * 128, np.uint16), np.zeros(nv * 128, np.uint16)
    kc4, kc3, kn = np.zeros((nv, 32), np.uint8), np.zeros((nv, 24), np.uint8), np.zeros(nv, np.uint16)
    vc4, vc3, vn = np.zeros_like(kc4), np.zeros_like(kc3), np.zeros_like(kn)
    kcc, kcn = np.zeros((nv, 48), np.uint8), np.zeros(nv, np.uint16)
    vcc, vcn = np.zeros_like(kcc), np.zeros_like(kcn)
    for b in range(B):
        for p in range(ctx):
            L.nxo_tiered_append(np.ascontiguousarray(K[b, p]), np.ascontiguousarray(V[b, p]), hkv, ks, vs, b4,
                                b3, kp, vp, kc4, kc3, kn, vc4, vc3, vn, bt, max_blocks, b, p)
            L.nxo_tiered_append_cool(hkv, ks, vs, c4, c3, b3, kc4, kc3, kn, vc4, vc3, vn, kcc, kcn, vcc, vcn, bt,
                                     max_blocks, b, p)
    out = np.empty_like(q)
    L.nxo_attn_decode_tiered_cool(q, kp, vp, kc4, kc3, kn, vc4, vc3, vn, kcc, kcn, vcc, vcn, ks, vs, c4, c3, bt,
                                  max_blocks, np.full(B, ctx, np.int32), H, W, B, hq, hkv, out)

    def want_for(cool, cold):
        Kf = K.astype(np.float16).astype(np.float64)
        Vf = V.astype(np.float16).astype(np.float64)
        for b in range(B):
            for h in range(hkv):
                for X, Xf, s in ((K, Kf, ks), (V, Vf, vs)):
                    if not cold:
                        continue
                    warm = oracle.tq_encode(X[b, :cold, h].astype(np.float16).astype(np.float32), s)[:3]
                    Xf[b, :cold, h] = oracle.tq_decode(*warm, s)
                    if cool:
                        cc, cn = oracle.tq_to_cool(warm[0][:cool], warm[1][:cool], warm[2][:cool], s)
                        Xf[b, :cool, h] = oracle.cool_decode(cc, cn, s)
        return np.stack([_attn_fp64(q[b].astype(np.float64), Kf[b], Vf[b], hq, hkv, 128) for b in range(B)])

    cold = max(0, (ctx - 1 - H) // 16 * 16)
    cool = max(0, (ctx - 1 - H - W) // 16 * 16)
    assert cool == L.nxo_tiered_cool(ctx, H, W) and cold == L.nxo_tiered_cold(ctx, H)
    want = want_for(cool, cold)
    e = rel_err(out, want)
    assert e < 1e-5, e
    if cool + 16 <= cold:
        assert rel_err(want_for(cool + 16, cold), want) > 1e-3


def test_tiered_evict_boundary():
    """evict = 16 floor((ctx - 1 - H - W - C) / 16) clamped at 0; nothing is
    evicted without a Warm range or with C = 0."""
    for ctx, H, W, C, want in [(49, 16, 16, 16, 0), (65, 16, 16, 16, 16), (300, 64, 32, 64, 128),
                               (32769, 4096, 4096, 8192, 16384), (5000, 16, 0, 16, 0), (5000, 16, 16, 0, 0)]:
        assert L.nxo_tiered_evict(ctx, H, W, C) == want, (ctx, H, W, C)
        assert L.nxo_tiered_evict(ctx, H, W, C) <= L.nxo_tiered_cool(ctx, H, W)


@pytest.mark.parametrize("ctx,H,W,C", [(130, 16, 16, 32), (100, 32, 16, 16)])
def test_tiered_evict_attention_vs_fp64(ctx, H, W, C):
    """Evicted positions read as zero vectors (get_vectors zero-fills a
    page it does not find): against an fp64 restatement in which positions
    before evict have zero K and V -- they still take softmax weight
    exp(0 - max) each.  Dropping them from the softmax instead (the planted
    mistake) moves the result past the bound."""
    rng = np.random.default_rng(ctx + 7 * H + W + C)
    hq, hkv, B = 4, 1, 1
    K = rng.normal(0, 1, (B, ctx, hkv, 128)).astype(np.float32)
    V = rng.normal(0, 1, (B, ctx, hkv, 128)).astype(np.float32)
    q = rng.normal(0, 0.4, (B, hq, 128)).astype(np.float32)
    ks, vs = oracle.tq_signs(5, 1), oracle.tq_signs(5, 2)
    c4, b4 = oracle.codebook(4)
    c3, b3 = oracle.codebook(3)
    max_blocks = (ctx + 15) // 16 + 1
    bt = np.arange(max_blocks, dtype=np.int32).reshape(1, max_blocks)
    nv = max_blocks * hkv * 16
    kp, vp = np.zeros(nv * 128, np.uint16), np.zeros(nv * 128, np.uint16)
    kc4, kc3, kn = np.zeros((nv, 32), np.uint8), np.zeros((nv, 24), np.uint8), np.zeros(nv, np.uint16)
    vc4, vc3, vn = np.zeros_like(kc4), np.zeros_like(kc3), np.zeros_like(kn)
    kcc, kcn = np.zeros((nv, 48), np.uint8), np.zeros(nv, np.uint16)
    vcc, vcn = np.zeros_like(kcc), np.zeros_like(kcn)
    for p in range(ctx):
        L.nxo_tiered_append(np.ascontiguousarray(K[0, p]), np.ascontiguousarray(V[0, p]), hkv, ks, vs, b4, b3, kp,
                            vp, kc4, kc3, kn, vc4, vc3, vn, bt, max_blocks, 0, p)
        L.nxo_tiered_append_cool(hkv, ks, vs, c4, c3, b3, kc4, kc3, kn, vc4, vc3, vn, kcc, kcn, vcc, vcn, bt,
                                 max_blocks, 0, p)
    out = np.empty_like(q)
    L.nxo_attn_decode_tiered_evict(q, kp, vp, kc4, kc3, kn, vc4, vc3, vn, kcc, kcn, vcc, vcn, ks, vs, c4, c3, bt,
                                   max_blocks, np.full(B, ctx, np.int32), H, W, C, B, hq, hkv, out)
    ev = L.nxo_tiered_evict(ctx, H, W, C)
    cool, cold = L.nxo_tiered_cool(ctx, H, W), L.nxo_tiered_cold(ctx, H)
    assert 0 < ev < cool < cold
    Kf = K[0].astype(np.float16).astype(np.float64)
    Vf = V[0].astype(np.float16).astype(np.float64)
    for X, Xf, s in ((K[0], Kf, ks), (V[0], Vf, vs)):
        warm = oracle.tq_encode(X[:cold, 0].astype(np.float16).astype(np.float32), s)[:3]
        Xf[:cold, 0] = oracle.tq_decode(*warm, s)
        cc, cn = oracle.tq_to_cool(warm[0][:cool], warm[1][:cool], warm[2][:cool], s)
        Xf[:cool, 0] = oracle.cool_decode(cc, cn, s)
        Xf[:ev] = 0.0
    want = _attn_fp64(q[0].astype(np.float64), Kf, Vf, hq, hkv, 128)
    assert rel_err(out[0], want) < 1e-5
    dropped = _attn_fp64(q[0].astype(np.float64), Kf[ev:], Vf[ev:], hq, hkv, 128)
    assert rel_err(dropped, want) > 1e-3


# -------------------------------------------------------------------- MoE --
def test_moe_route_golden():
    g = gold("moe_route.npz")
    k = int(g["k"])
    for i in range(g["logits"].shape[0]):
        ids = np.empty(k, np.int32)
        w = np.empty(k, np.float32)
        L.nxo_moe_route(np.ascontiguousarray(g["logits"][i]), g["logits"].shape[1], k, ids, w)
        assert np.array_equal(ids, g["ids"][i])
        assert np.allclose(w, g["weights"][i], rtol=1e-6, atol=0)


@pytest.mark.parametrize("E,k", [(64, 10), (256, 16), (160, 7)])
def test_moe_route_wide(E, k):
    """Routing over up to 256 experts and top-16 (the reference's default
    is top-10, hybrid_model.cpp:1648): against the reference MoERouter built
    from its sources (identity gate, so the logits are the hidden state) and
    against a float64 softmax with the k largest by value (ties by id)."""
    rng = np.random.default_rng(E + k)
    R = oracle.ref()
    for rep in range(6):
        lg = (rng.standard_normal(E) * (0.5 + rep)).astype(np.float32)
        ids = np.empty(k, np.int32)
        w = np.empty(k, np.float32)
        L.nxo_moe_route(lg, E, k, ids, w)
        p = np.exp(lg.astype(np.float64) - lg.max())
        p /= p.sum()
        order = np.lexsort((np.arange(E), -p))[:k]
        assert np.array_equal(ids, order)
        assert np.allclose(w, p[order] / p[order].sum(), rtol=2e-6, atol=0)
        if R is not None:
            rid = np.empty(k, np.int32)
            rw = np.empty(k, np.float32)
            gate = np.eye(E, dtype=np.float32)
            assert R.ref_moe_route(E, k, E, gate, lg, rid, rw) == k
            assert np.array_equal(ids, rid)
            assert np.allclose(w, rw, rtol=1e-6, atol=0)


def test_moe_route_ties_pick_lower_id():
    ids = np.empty(2, np.int32)
    w = np.empty(2, np.float32)
    L.nxo_moe_route(np.array([0.5, 1.0, 1.0, 1.0], np.float32), 4, 2, ids, w)
    assert list(ids) == [1, 2] and np.allclose(w, 0.5)


# ------------------------------------------------------------------ model --
TINY = dict(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=688, vocab=4096,
            n_experts=0, top_k=0, max_seq=128, batch=1, kv_kind=0, rope_theta=10000.0, eps=1e-5,
            seed=0x5EED)


def _deq(tid, N, K, sigma=0.02, seed=0x5EED):
    c, s = oracle.gen_quant_rows(0, N, K, seed, tid, sigma)
    return oracle.dequantize(c, s, N, K).astype(np.float64)


@pytest.mark.parametrize("sigma", [0.0, 0.1])
def test_tiny_model_step_vs_fp64_composition(sigma):
    """One forward step of the oracle model against an fp64 composition of
    independently pinned pieces (dequant, fp64 matmul, closed-form norm /
    RoPE / softmax / SwiGLU) in the reference layer order.  With sigma > 0
    the three kinds of RMSNorm weights differ (1 + N(0, sigma) per tensor),
    so applying one in the wrong place fails."""
    m = oracle.Model(**dict(TINY, norm_sigma=sigma))
    toks = [17, 999, 4000]
    logits = [m.forward(np.array([t], np.int32))[0] for t in toks]
    d, hq, hkv, hd, F, V = 256, 4, 2, 64, 688, 4096
    emb = oracle.gen_normal(V * d, 0x5EED, 1, 0.02).reshape(V, d).astype(np.float16).astype(np.float64)
    lid = lambda Li, kind: 0x100 * (Li + 1) + kind
    W = [{k: _deq(lid(Li, i), n, kk) for k, i, n, kk in
          (("q", 0, hq * hd, d), ("k", 1, hkv * hd, d), ("v", 2, hkv * hd, d), ("o", 3, d, hq * hd),
           ("g", 4, F, d), ("u", 5, F, d), ("dn", 6, d, F))} for Li in range(2)]
    lm = _deq(2, V, d)
    f16r = lambda a: np.asarray(a, np.float32).astype(np.float16).astype(np.float64)
    nw = lambda tid: (1.0 + oracle.gen_normal(d, 0x5EED, tid, sigma).astype(np.float64)) if sigma else 1.0
    norm = lambda h, w: f16r(h / np.sqrt(np.mean(h**2) + 1e-5) * w)
    ang = lambda p: p * 10000.0 ** (-(2.0 * np.arange(hd // 2)) / hd)

    def rope(x, p, heads):
        z = x.reshape(heads, hd // 2, 2)
        zc = (z[..., 0] + 1j * z[..., 1]) * np.exp(1j * ang(p))
        return np.stack([zc.real, zc.imag], -1).reshape(-1)

    cache = [([], []) for _ in range(2)]
    for p, t in enumerate(toks):
        h = emb[t].copy()
        for Li in range(2):
            w = W[Li]
            xn = norm(h, nw(lid(Li, 10)))
            q, k, v = rope(w["q"] @ xn, p, hq), rope(w["k"] @ xn, p, hkv), w["v"] @ xn
            cache[Li][0].append(f16r(k).reshape(hkv, hd))
            cache[Li][1].append(f16r(v).reshape(hkv, hd))
            att = _attn_fp64(q.reshape(hq, hd), np.array(cache[Li][0]), np.array(cache[Li][1]), hq, hkv, hd)
            h = h + w["o"] @ f16r(att.reshape(-1))
            xn = norm(h, nw(lid(Li, 11)))
            g, u = w["g"] @ xn, w["u"] @ xn
            h = h + w["dn"] @ f16r(g / (1 + np.exp(-g)) * u)
        want = lm @ norm(h, nw(3))
        # non-unit norm weights move more fp16 rounding boundaries of the GEMV
        # inputs (2e-4 here); a norm weight in the wrong place gives 0.1-0.26
        assert rel_err(logits[p], want) < (1e-4 if sigma == 0 else 1e-3)
    m.close()


@pytest.mark.parametrize("sigma", [0.0, 0.1])
def test_tiny_moe_step_vs_fp64_composition(sigma):
    """MoE FFN of the oracle model (hybrid_model.cpp:1656-1711 order: router
    logits, softmax, top-k, renormalize, weighted sum of expert SwiGLUs)
    against an fp64 composition, two steps on one sequence; with sigma > 0
    the router and experts read the ffn-normed input."""
    cfg = dict(TINY, n_experts=4, top_k=2, seed=0x0E0E, norm_sigma=sigma)
    m = oracle.Model(**cfg)
    toks = [5, 3000]
    logits = [m.forward(np.array([t], np.int32))[0] for t in toks]
    m.close()
    seed, d, hq, hkv, hd, F, V, E = 0x0E0E, 256, 4, 2, 64, 688, 4096, 4
    emb = oracle.gen_normal(V * d, seed, 1, 0.02).reshape(V, d).astype(np.float16).astype(np.float64)
    lid = lambda Li, kind: 0x100 * (Li + 1) + kind
    eid = lambda Li, e, w: 0x01000000 + 0x1000 * Li + 4 * e + w
    W = []
    for Li in range(2):
        w = {k: _deq(lid(Li, i), n, kk, seed=seed) for k, i, n, kk in
             (("q", 0, hq * hd, d), ("k", 1, hkv * hd, d), ("v", 2, hkv * hd, d), ("o", 3, d, hq * hd))}
        w["r"] = _deq(lid(Li, 7), E, d, sigma=1 / np.sqrt(d), seed=seed)
        w["e"] = [(_deq(eid(Li, e, 0), F, d, seed=seed), _deq(eid(Li, e, 1), F, d, seed=seed),
                   _deq(eid(Li, e, 2), d, F, seed=seed)) for e in range(E)]
        W.append(w)
    lm = _deq(2, V, d, seed=seed)
    f16r = lambda a: np.asarray(a, np.float32).astype(np.float16).astype(np.float64)
    nw = lambda tid: (1.0 + oracle.gen_normal(d, seed, tid, sigma).astype(np.float64)) if sigma else 1.0
    norm = lambda h, w: f16r(h / np.sqrt(np.mean(h**2) + 1e-5) * w)
    ang = lambda p: p * 10000.0 ** (-(2.0 * np.arange(hd // 2)) / hd)

    def rope(x, p, heads):
        z = x.reshape(heads, hd // 2, 2)
        zc = (z[..., 0] + 1j * z[..., 1]) * np.exp(1j * ang(p))
        return np.stack([zc.real, zc.imag], -1).reshape(-1)

    cache = [([], []) for _ in range(2)]
    for p, t in enumerate(toks):
        h = emb[t].copy()
        for Li in range(2):
            w = W[Li]
            xn = norm(h, nw(lid(Li, 10)))
            q, k, v = rope(w["q"] @ xn, p, hq), rope(w["k"] @ xn, p, hkv), w["v"] @ xn
            cache[Li][0].append(f16r(k).reshape(hkv, hd))
            cache[Li][1].append(f16r(v).reshape(hkv, hd))
            att = _attn_fp64(q.reshape(hq, hd), np.array(cache[Li][0]), np.array(cache[Li][1]), hq, hkv, hd)
            h = h + w["o"] @ f16r(att.reshape(-1))
            xn = norm(h, nw(lid(Li, 11)))
            lg = w["r"] @ xn
            pr = np.exp(lg - lg.max())
            pr /= pr.sum()
            top = np.argsort(-pr, kind="stable")[:2]
            wts = pr[top] / pr[top].sum()
            out = np.zeros(d)
            for e, we in zip(top, wts):
                g1, u1, d1 = w["e"][e]
                g, u = g1 @ xn, u1 @ xn
                out += we * (d1 @ f16r(g / (1 + np.exp(-g)) * u))
            h = h + out
        want = lm @ norm(h, nw(3))
        # fp16-rounded activations can land on the other side of a rounding
        # boundary in fp32 vs fp64 (one fp16 ulp is 4.9e-4 relative)
        assert rel_err(logits[p], want) < (5e-4 if sigma == 0 else 1e-3)

    p = oracle.prompt_tokens(0x5EED, 1, 16, 4096)
    a = oracle.Model(**TINY)
    b = oracle.Model(**TINY)
    ta, ma = a.generate(p, 8)
    tb, _ = b.generate(p, 8)
    assert np.array_equal(ta, tb)
    assert np.all(ma >= 0)
