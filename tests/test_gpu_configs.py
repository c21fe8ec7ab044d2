"""Parity at the benchmark workloads' own shapes, on the GPU, against the
oracle on identical seeded inputs:

- the Llama-3.1-8B shape at 32768 positions of TurboQuant pages (one layer,
  plus lm_head): the split plan there gives more than 16 pages per split, so
  the pipelined TurboQuant attention runs; the same with tiered pages (4096
  fp16 positions, older ones TurboQuant), whose split plan pipelines both
  tiers and whose decode compresses a page on the device;
- the Mixtral-8x7B shape (d 4096, 8 experts of 14336, top-2): RMSNorm +
  router + routing in one launch, the routed gate/up and down GEMVs at batch
  1 and 8, and the standalone expert FFN entry point at full size;
- the 8B shape at batch 8: a full layer plus lm_head against the oracle, and
  the 32-layer decode's determinism and range.

Every decode is teacher-forced: the GPU model and the oracle consume the
oracle's greedy tokens, and at every step the logits must agree within
1e-3 (pages the decode itself compresses: TQ_TOL) and the greedy token must
be the oracle's wherever the oracle's top-two margin is not a numerical
tie.  TurboQuant codes of the pages compressed during the decode must be
bit-exact."""
import numpy as np
import pytest

import nexus_amd
import oracle
from conftest import check_forced, f16, forced_logits, rel_err
from test_gpu_kernels import _tq_pools, up
from test_gpu_model import LLAMA8B, TIE_MARGIN
from test_gpu_tiered import TQ_TIE, TQ_TOL

pytestmark = pytest.mark.gpu
L = oracle.lib

MIXTRAL = dict(n_layers=32, d_model=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=14336, vocab=32000,
               n_experts=8, top_k=2, max_seq=4096 + 256, batch=1, kv_kind=0, rope_theta=1e6, eps=1e-5,
               seed=0x3117)


def _start_tokens(cfg):
    return np.array([L.nxo_rand_u64(cfg["seed"], 5, b) % cfg["vocab"] for b in range(cfg["batch"])], np.int32)


def _filled_parity(ctx, cfg, ctx_len, steps, n_outlier=0, tol=1e-3, tie=TIE_MARGIN, check_pages=None):
    """Fill ctx_len positions on both sides and run `steps` teacher-forced
    decode steps (check_forced); check_pages(gm, om) runs before close."""
    label = f"ctx {ctx_len} batch {cfg['batch']} kv_kind {cfg['kv_kind']} seed {cfg['seed']:#x}"
    print(f"[case] {cfg} ctx {ctx_len} steps {steps}", flush=True)
    gm = nexus_amd.Model(ctx, **cfg)
    gm.fill_context(ctx_len, n_outlier)
    start = gm.pending()
    om = oracle.Model(**cfg)
    om.fill_context(ctx_len, n_outlier)
    assert np.array_equal(start, _start_tokens(cfg))
    glog, olog = forced_logits(gm, om, start, steps)
    if check_pages is not None:
        check_pages(gm, om)
    gm.close()
    om.close()
    check_forced(glog, olog, tol, tie, label)


# ------------------------------------------------- 8B @ 32K TurboQuant pages --
@pytest.mark.parametrize("lens", [[32768], [4096] * 8])
def test_tq_attention_parity_pipelined(ctx, lens):
    """(32, 8, 128) heads: 32768 positions at batch 1 (32 splits of 65
    pages) and 4096 at batch 8 (4 splits of 65 pages) -- the pipelined
    TurboQuant attention that the 32K decode runs."""
    hq, hkv = 32, 8
    rng = np.random.default_rng(0x32 + len(lens))
    B = len(lens)
    ks, vs = oracle.tq_signs(3, 11), oracle.tq_signs(3, 12)
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
        assert rel_err(got[b], want[b]) < 1e-3
    for bb in bufs + [ob]:
        ctx.free(bb)


def test_8b_turboquant_32k_one_layer(ctx):
    """One 8B-shaped layer plus lm_head over 32768 TurboQuant positions
    (4 outlier channels per head x10), 64 teacher-forced decode steps (the
    steps of the 32K workload), each appending its position to the pages."""
    cfg = dict(LLAMA8B, n_layers=1, kv_kind=1, max_seq=32768 + 256, seed=0x32C4)
    _filled_parity(ctx, cfg, 32768, 64, n_outlier=4, tol=TQ_TOL, tie=TQ_TIE)


def test_8b_tiered_32k_one_layer(ctx):
    """One 8B-shaped layer at 32760 positions with tiered pages (last 4096
    fp16): both tiers' split loops are pipelined; at the 8th step position
    32767 completes page (32767 - 4096 + 1) / 16 - 1 = 1791 outside the
    window and the device compresses it, bit-exact with the oracle."""
    cfg = dict(LLAMA8B, n_layers=1, kv_kind=2, hot_window=4096, max_seq=32768 + 256, seed=0x71E8)
    ctx_len, steps = 32760, 10

    def pages(gm, om):
        for p in range(1791 * 16, 1792 * 16):
            for kv in range(2):
                form, g = gm.kv_read(0, 0, p, kv)
                assert form == 1, (p, kv)
                assert np.array_equal(g, om.kv_read(0, 0, p, kv, 1)), (p, kv)

    _filled_parity(ctx, cfg, ctx_len, steps, n_outlier=4, tol=TQ_TOL, tie=TQ_TIE, check_pages=pages)


def test_tiered_pipelined_batch8(ctx):
    """Batch 8, 8 kv heads, 4608 positions of capacity and a 512-position
    window: the split plan gives 86 TurboQuant pages and 34 fp16 pages per
    split, so both pipelined loops run; 20 steps from 4000 filled positions,
    crossing one compression per sequence (at the 16th step)."""
    cfg = dict(LLAMA8B, n_layers=2, d_model=512, n_heads=16, n_kv_heads=8, ffn=688, vocab=4096, batch=8,
               max_seq=4608, kv_kind=2, hot_window=512, seed=0x7A88)

    def pages(gm, om):
        # the fill compresses pages 0..217; position 4015 completes page
        # (4015 - 512 + 1) / 16 - 1 = 218 outside the window
        for b in (0, 7):
            for p in range(218 * 16, 219 * 16, 5):
                for kv in range(2):
                    form, g = gm.kv_read(1, b, p, kv)
                    assert form == 1 and np.array_equal(g, om.kv_read(1, b, p, kv, 1)), (b, p, kv)

    _filled_parity(ctx, cfg, 4000, 20, n_outlier=4, tol=TQ_TOL, tie=TQ_TIE, check_pages=pages)


def test_8b_three_tier_32k_one_layer(ctx):
    """One 8B-shaped layer at 32760 positions with three tiers (last 4096
    fp16, the 4096 before them TurboQuant, older pages Cool): all three
    split loops are pipelined; at the 8th step position 32767 completes
    page 1791 outside the window and page (32767 - 8192 + 1) / 16 - 1 = 1535
    outside the Warm range, and the device re-encodes page 1535 Cool,
    bit-exact with the oracle."""
    cfg = dict(LLAMA8B, n_layers=1, kv_kind=2, hot_window=4096, warm_window=4096, max_seq=32768 + 256,
               seed=0x3C8E)
    ctx_len, steps = 32760, 10

    def pages(gm, om):
        for p in list(range(1535 * 16, 1536 * 16)) + [0, 12345, 24559]:
            for kv in range(2):
                form, g = gm.kv_read(0, 0, p, kv)
                assert form == 2, (p, kv)
                assert np.array_equal(g, om.kv_read(0, 0, p, kv, 2)), (p, kv)
        for p in (1791 * 16, 1791 * 16 + 15, 24576, 28671):
            form, g = gm.kv_read(0, 0, p, 0)
            assert form == 1 and np.array_equal(g, om.kv_read(0, 0, p, 0, 1)), p

    _filled_parity(ctx, cfg, ctx_len, steps, n_outlier=4, tol=TQ_TOL, tie=TQ_TIE, check_pages=pages)


def test_8b_evicting_tiers_32k_one_layer(ctx):
    """One 8B-shaped layer at 32760 positions: last 4096 fp16, 4096
    TurboQuant, 8192 Cool in a ring of 513 pages, older pages evicted (16368
    positions read as zero keys and values).  At the 8th step page 1535
    moves to the Cool ring (bit-exact) and page 1023 is evicted."""
    cfg = dict(LLAMA8B, n_layers=1, kv_kind=2, hot_window=4096, warm_window=4096, cool_window=8192,
               max_seq=32768 + 256, seed=0xE78E)
    ctx_len, steps = 32760, 10

    def pages(gm, om):
        for p in (0, 9999, 1023 * 16, 1023 * 16 + 15):
            form, g = gm.kv_read(0, 0, p, 0)
            assert form == 3 and g.size == 0, p
        for p in list(range(1535 * 16, 1536 * 16)) + [1024 * 16, 20000]:
            for kv in range(2):
                form, g = gm.kv_read(0, 0, p, kv)
                assert form == 2 and np.array_equal(g, om.kv_read(0, 0, p, kv, 2)), (p, kv)

    _filled_parity(ctx, cfg, ctx_len, steps, n_outlier=4, tol=TQ_TOL, tie=TQ_TIE, check_pages=pages)


def test_three_tier_pipelined_batch8(ctx):
    """Batch 8, 8 kv heads, 4608 positions of capacity, a 512-position
    window and a 512-position Warm range: the split plan pipelines the Cool,
    TurboQuant and fp16 loops; 20 steps from 4000 filled positions cross one
    compression of each kind per sequence (at the 16th step)."""
    cfg = dict(LLAMA8B, n_layers=2, d_model=512, n_heads=16, n_kv_heads=8, ffn=688, vocab=4096, batch=8,
               max_seq=4608, kv_kind=2, hot_window=512, warm_window=512, seed=0x3CB8)

    def pages(gm, om):
        # position 4015 completes page 218 outside the window and page
        # (4015 - 1024 + 1) / 16 - 1 = 186 outside the Warm range
        for b in (0, 7):
            for p in range(186 * 16, 187 * 16, 5):
                for kv in range(2):
                    form, g = gm.kv_read(1, b, p, kv)
                    assert form == 2 and np.array_equal(g, om.kv_read(1, b, p, kv, 2)), (b, p, kv)
            for p in range(218 * 16, 219 * 16, 5):
                form, g = gm.kv_read(1, b, p, 1)
                assert form == 1 and np.array_equal(g, om.kv_read(1, b, p, 1, 1)), (b, p)

    _filled_parity(ctx, cfg, 4000, 20, n_outlier=4, tol=TQ_TOL, tie=TQ_TIE, check_pages=pages)


# ------------------------------------------------------------ Mixtral shape --
@pytest.mark.parametrize("batch", [1, 8])
def test_mixtral_one_layer_parity(ctx, batch):
    """One Mixtral-shaped layer (d 4096, 8 experts of 14336, top-2, vocab
    32000) at 512 positions: routing launch, routed gate/up + SwiGLU and down
    GEMVs and the combine at full size, three steps."""
    cfg = dict(MIXTRAL, n_layers=1, max_seq=1024, batch=batch, seed=0x3117 + batch)
    _filled_parity(ctx, cfg, 512, 3)


def test_moe_expert_ffn_mixtral_shape(ctx):
    """nx_moe_expert_ffn at d 4096, F 14336, E 8, top-2, batch 8 (every
    expert active): each token's output against the oracle's expert GEMVs."""
    d, F, E, k, B = 4096, 14336, 8, 2, 8
    Gd, Gf = d // 32, F // 32
    w13 = np.empty((E, 2 * F, Gd * 16), np.uint8)
    s13 = np.empty((E, 2 * F, Gd), np.uint16)
    w2 = np.empty((E, d, Gf * 16), np.uint8)
    s2 = np.empty((E, d, Gf), np.uint16)
    for e in range(E):
        cg, sg = oracle.gen_quant_rows(0, F, d, 0x6E, 3 * e, 0.02)
        cu, su = oracle.gen_quant_rows(0, F, d, 0x6E, 3 * e + 1, 0.02)
        w13[e, 0::2], s13[e, 0::2], w13[e, 1::2], s13[e, 1::2] = cg, sg, cu, su
        w2[e], s2[e] = oracle.gen_quant_rows(0, d, F, 0x6E, 3 * e + 2, 0.02)
    rng = np.random.default_rng(12)
    x = rng.normal(0, 1, (B, d)).astype(np.float16)
    ids = np.array([[b, (b + 3) % E] for b in range(B)], np.int32)
    wts = rng.uniform(0.1, 0.9, (B, k)).astype(np.float32)
    bufs = [up(ctx, a) for a in (x.view(np.uint16), w13, s13, w2, s2, ids, wts)]
    ob = ctx.alloc(B * d * 4)
    ctx.check(ctx.L.nx_moe_expert_ffn(ctx.h, *bufs, ob, d, F, E, k, B, 0), "moe_ffn")
    got = ctx.download(ob, (B, d), np.float32)
    for bb in bufs + [ob]:
        ctx.free(bb)
    for b in range(B):
        acc = np.zeros(d, np.float32)
        xf = x[b].astype(np.float32)
        for j in range(k):
            e = ids[b, j]
            gu = oracle.gemv(w13[e], s13[e], xf, 2 * F, d)[0]
            a = np.empty(F, np.float32)
            L.nxo_swiglu(np.ascontiguousarray(gu[0::2]), np.ascontiguousarray(gu[1::2]), F, a)
            a = a.astype(np.float16).astype(np.float32)
            acc += wts[b, j] * oracle.gemv(w2[e], s2[e], a, d, F)[0]
        assert rel_err(got[b], acc) < 1e-3, b


# ---------------------------------------------------------- 8B at batch 8 --
def test_8b_one_layer_batch8_parity(ctx):
    """A full 8B layer plus lm_head at batch 8 (matrix-core GEMVs with the
    RMSNorm staging over K 4096, RoPE + page writes, SwiGLU, the staged down
    projection over K 14336, logits + argmax) against the oracle."""
    cfg = dict(LLAMA8B, n_layers=1, max_seq=1024, batch=8, seed=0x8B08)
    _filled_parity(ctx, cfg, 512, 3)


def test_8b_decode_properties_batch8(ctx):
    """The 32-layer 8B shape at batch 8 over 4096 positions: deterministic
    across two models, tokens in range, finite logits, and the step's
    algorithmic bytes match the closed form."""
    cfg = dict(LLAMA8B, batch=8)
    runs = []
    for _ in range(2):
        gm = nexus_amd.Model(ctx, **cfg)
        gm.fill_context(4096, 0)
        if not runs:
            # weights once + fp16 KV of 4096 positions x 32 layers per sequence
            assert abs(gm.step_bytes() - (4221370368 + 8 * 536870912)) < 1e7
        toks = gm.decode(4)
        lg = gm.logits()
        assert toks.min() >= 0 and toks.max() < cfg["vocab"]
        assert np.all(np.isfinite(lg))
        runs.append((toks, lg))
        gm.close()
    assert np.array_equal(runs[0][0], runs[1][0])
    assert np.array_equal(runs[0][1], runs[1][1])


@pytest.mark.parametrize("batch", [1, 8])
def test_mixtral_decode_properties(ctx, batch):
    """The 32-layer Mixtral shape (8 experts of 14336, top-2, all resident)
    over 4096 positions: deterministic across two models, tokens in range,
    finite logits, and the step's algorithmic bytes between the closed forms
    for top-2 and for every expert active in each layer."""
    cfg = dict(MIXTRAL, batch=batch)
    d, F, E, V, qkv = 4096, 14336, 8, 32000, 4096 + 2 * 1024
    qb = lambda n, k: n * ((k + 31) // 32) * 18  # int4-g32 codes + fp16 scales
    shared = qb(V, d) + 32 * (qb(qkv, d) + qb(d, 4096) + qb(E, d))
    expert = qb(2 * F, d) + qb(d, F)
    kv = batch * 32 * 4096 * 2 * 8 * 128 * 2
    runs = []
    for _ in range(2):
        print(f"[case] mixtral 32 layers batch {batch} ctx 4096", flush=True)
        gm = nexus_amd.Model(ctx, **cfg)
        gm.fill_context(4096, 0)
        toks = gm.decode(4)
        lg = gm.logits()
        nb = gm.step_bytes()
        assert shared + 32 * 2 * expert + kv - 1e7 <= nb <= shared + 32 * E * expert + kv + 1e8, nb
        assert toks.min() >= 0 and toks.max() < V
        assert np.all(np.isfinite(lg))
        runs.append((toks, lg))
        gm.close()
    assert np.array_equal(runs[0][0], runs[1][0])
    assert np.array_equal(runs[0][1], runs[1][1])


@pytest.mark.parametrize("batch,kv_kind", [(1, 0), (8, 0), (1, 1)])
def test_8b_one_layer_qk_norm(ctx, batch, kv_kind):
    """One 8B-shaped layer with per-head Q/K RMSNorm (the attn_q_norm /
    attn_k_norm of Qwen3- and Gemma-style models, hybrid_model.cpp:1325-1349,
    weights 1 + N(0, 0.1)) at 512 positions: the batch-1 streaming and
    batch-8 matrix-core QKV GEMVs write the projection alone, the Q/K norm
    launch normalizes, rotates and writes the pages (TurboQuant pages: the
    attention launch appends), four teacher-forced steps."""
    cfg = dict(LLAMA8B, n_layers=1, max_seq=1024, batch=batch, kv_kind=kv_kind, qk_norm=1, norm_sigma=0.1,
               seed=0x9C8B + batch + 16 * kv_kind)
    _filled_parity(ctx, cfg, 512, 4, n_outlier=4 if kv_kind else 0, tol=TQ_TOL if kv_kind else 1e-3,
                   tie=TQ_TIE if kv_kind else TIE_MARGIN)
