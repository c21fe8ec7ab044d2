"""Tiered pages on the GPU (kv_kind 2): the last hot_window positions in
fp16, older pages compressed to TurboQuant on the device as they leave the
window (the Hot -> Warm step of PagedKVCache::compress_tier,
kv/paged_attention.cpp:244-291, run per page), attention over both tiers
in one softmax (the mixed-tier gather of get_vectors, :161-230).  With a
warm_window, pages that also leave the Warm range are re-encoded Cool
(3-bit codes on every coordinate; the Warm -> Cool step of compress_tier)
and attention reads three tiers.  Checked against the oracle's
restatement: greedy tokens, teacher-forced logits of every step, and the
stored bytes of every compressed page bit-exact."""
import numpy as np
import pytest

import nexus_amd
import oracle
from conftest import TQ_DECODE_TIE, TQ_DECODE_TOL, TQ_TIE, TQ_TOL, check_forced, forced_logits, rel_err
from test_gpu_model import TINY, assert_greedy_parity, run_both, run_forced, top2_margin

pytestmark = pytest.mark.gpu

TQ_TINY = dict(TINY, n_heads=4, n_kv_heads=2, head_dim=128, d_model=512)





@pytest.mark.parametrize("batch,H", [(1, 16), (2, 48)])
def test_tiered_greedy_parity(ctx, batch, H):
    """A 12-token prompt and 100 greedy tokens: pages leave the window and
    are compressed every 16 steps from position H + 15 on."""
    cfg = dict(TQ_TINY, batch=batch, kv_kind=2, hot_window=H, seed=0x7E1 + H)
    got, want, margins = run_both(ctx, cfg, P=12, n_new=100)
    assert_greedy_parity(got, want, margins, tie=TQ_DECODE_TIE)
    run_forced(ctx, cfg, 12, 100, tol=TQ_DECODE_TOL, tie=TQ_DECODE_TIE)


def test_tiered_filled_context_and_compressor(ctx):
    """A 300-position context with a 64-position window (pages 0..13
    compressed by the fill, 14..18 in the window), then 40 decode steps, in
    which pages 14, 15 and 16 leave the window and the device compressor
    encodes them.  Every stored position of the fill is bit-exact against
    the oracle (codes before the window, fp16 in it), so are the pages the
    compressor wrote, and the decode gives the oracle's tokens."""
    cfg = dict(TQ_TINY, batch=2, max_seq=512, kv_kind=2, hot_window=64, seed=0x71E2)
    ctx_len, steps = 300, 40
    gm = nexus_amd.Model(ctx, **cfg)
    gm.fill_context(ctx_len, 4)
    om = oracle.Model(**cfg)
    om.fill_context(ctx_len, 4)

    def check(positions, form_want):
        for L in range(cfg["n_layers"]):
            for b in range(2):
                for kv in range(2):
                    for p in positions:
                        form, got = gm.kv_read(L, b, p, kv)
                        assert form == form_want, (L, b, p, kv)
                        want = om.kv_read(L, b, p, kv, form)
                        assert np.array_equal(got, want), (L, b, p, kv, form)

    check(list(range(0, 224, 7)) + [223], 1)
    check(range(224, 300), 0)
    start = gm.pending()
    glog, olog = forced_logits(gm, om, start, steps)
    check(range(224, 272), 1)  # compressed on the device during the decode
    check(range(272, 300), 0)
    gm.close()
    om.close()
    check_forced(glog, olog, TQ_TOL, TQ_TIE, f"seed {cfg['seed']:#x}")


@pytest.mark.parametrize("hq,hkv,H,ctx_len", [(8, 2, 128, 700), (8, 1, 32, 1000), (4, 4, 256, 260)])
def test_tiered_filled_context_group_sizes(ctx, hq, hkv, H, ctx_len):
    """Query groups of 4 and 8 heads, a single kv head, windows of 32 to 256
    positions and a context just past the first compressed page: 20 decode
    steps from a filled context give the oracle's tokens (and logits within
    1e-3 when the tokens agree); the compressed pages stay bit-exact."""
    cfg = dict(TINY, n_heads=hq, n_kv_heads=hkv, head_dim=128, d_model=hq * 128, max_seq=1024 + 64, batch=1,
               kv_kind=2, hot_window=H, seed=0x6000 + hq * 16 + hkv + H)
    steps = 20
    gm = nexus_amd.Model(ctx, **cfg)
    gm.fill_context(ctx_len, 4)
    om = oracle.Model(**cfg)
    om.fill_context(ctx_len, 4)
    start = gm.pending()
    glog, olog = forced_logits(gm, om, start, steps)
    cold = 16 * max(0, (ctx_len - H) // 16)
    for p in list(range(0, cold, 37)) + ([cold - 1] if cold else []):
        for kv in range(2):
            form, g = gm.kv_read(cfg["n_layers"] - 1, 0, p, kv)
            assert form == 1 and np.array_equal(g, om.kv_read(cfg["n_layers"] - 1, 0, p, kv, 1)), (p, kv)
    gm.close()
    om.close()
    check_forced(glog, olog, TQ_TOL, TQ_TIE, f"seed {cfg['seed']:#x}")


def test_tiered_window_covering_context_matches_fp16_pages(ctx):
    """A window larger than the context keeps every position in fp16: the
    tiered path (an empty compressed part, the fp16 kernel's record and the
    merge) gives the fp16-page model's logits within 1e-3 and its tokens."""
    base = dict(TQ_TINY, batch=2, max_seq=512, seed=0xF16)
    ctx_len, steps = 200, 12
    out = {}
    for kind, extra in ((0, {}), (2, {"hot_window": 480})):
        m = nexus_amd.Model(ctx, **dict(base, kv_kind=kind, **extra))
        m.fill_context(ctx_len, 0)
        toks = m.decode(steps)
        out[kind] = (toks, m.logits())
        m.close()
    assert np.array_equal(out[0][0], out[2][0])
    assert rel_err(out[2][1], out[0][1]) < 1e-3


def test_tiered_config_rejected(ctx):
    for H in (0, 24, 128):
        with pytest.raises(RuntimeError):
            nexus_amd.Model(ctx, **dict(TQ_TINY, kv_kind=2, hot_window=H))
    with pytest.raises(RuntimeError):
        nexus_amd.Model(ctx, **dict(TINY, kv_kind=2, hot_window=32))  # head_dim 64


# ------------------------------------------------------------- three tiers --
@pytest.mark.parametrize("batch,H,W,pool", [(1, 16, 16, 0), (2, 32, 48, 0), (2, 16, 16, 15)])
def test_three_tier_greedy_parity(ctx, batch, H, W, pool):
    """A 12-token prompt and 100 greedy tokens: pages leave the fp16 window
    from position H + 15 on and the Warm range from H + W + 15 on, both
    compressions on the device in the attention launch.  pool > 0: the Cool
    table draws from a shared pool of that many pages (two sequences of 7
    pages each)."""
    cfg = dict(TQ_TINY, batch=batch, kv_kind=2, hot_window=H, warm_window=W, seed=0x3C1 + H + W + pool,
               kv_blocks=pool)
    got, want, margins = run_both(ctx, cfg, P=12, n_new=100)
    assert_greedy_parity(got, want, margins, tie=TQ_DECODE_TIE)
    run_forced(ctx, cfg, 12, 100, tol=TQ_DECODE_TOL, tie=TQ_DECODE_TIE)


def _check_forms(gm, om, n_layers, batch, ranges):
    for L in range(n_layers):
        for b in range(batch):
            for kv in range(2):
                for positions, form_want in ranges:
                    for p in positions:
                        form, got = gm.kv_read(L, b, p, kv)
                        assert form == form_want, (L, b, p, kv, form)
                        want = om.kv_read(L, b, p, kv, form)
                        assert np.array_equal(got, want), (L, b, p, kv, form)


def test_three_tier_filled_context_and_compressors(ctx):
    """300 filled positions with a 64-position window and a 32-position Warm
    range: the fill writes pages 0..11 Cool, 12..13 TurboQuant, 14..18
    fp16.  In 40 decode steps pages 14, 15, 16 leave the window and pages
    12, 13, 14 leave the Warm range (page 14 both: the Warm codes the
    device wrote are re-encoded 32 steps later).  Every Cool, TurboQuant and
    fp16 position is bit-exact against the oracle, before and after."""
    cfg = dict(TQ_TINY, batch=2, max_seq=512, kv_kind=2, hot_window=64, warm_window=32, seed=0x3C2)
    ctx_len, steps = 300, 40
    gm = nexus_amd.Model(ctx, **cfg)
    gm.fill_context(ctx_len, 4)
    om = oracle.Model(**cfg)
    om.fill_context(ctx_len, 4)
    n_layers = cfg["n_layers"]
    _check_forms(gm, om, n_layers, 2, [(list(range(0, 192, 5)) + [191], 2), (range(192, 224, 3), 1),
                                       (range(224, 300, 4), 0)])
    start = gm.pending()
    glog, olog = forced_logits(gm, om, start, steps)
    _check_forms(gm, om, n_layers, 2, [(range(192, 240), 2), (range(240, 272), 1), (range(272, 300), 0)])
    gm.close()
    om.close()
    check_forced(glog, olog, TQ_TOL, TQ_TIE, f"seed {cfg['seed']:#x}")


@pytest.mark.parametrize("hq,hkv,H,W,ctx_len", [(8, 2, 128, 64, 700), (8, 1, 32, 32, 1000), (4, 4, 256, 16, 400)])
def test_three_tier_group_sizes(ctx, hq, hkv, H, W, ctx_len):
    """Query groups of 2 to 8 heads, a single kv head, several window and
    Warm sizes: 20 decode steps from a filled context give the oracle's
    tokens (logits within 1e-3 when the tokens agree); Cool pages stay
    bit-exact."""
    cfg = dict(TINY, n_heads=hq, n_kv_heads=hkv, head_dim=128, d_model=hq * 128, max_seq=1024 + 64, batch=1,
               kv_kind=2, hot_window=H, warm_window=W, seed=0x6100 + hq * 16 + hkv + H + W)
    steps = 20
    gm = nexus_amd.Model(ctx, **cfg)
    gm.fill_context(ctx_len, 4)
    om = oracle.Model(**cfg)
    om.fill_context(ctx_len, 4)
    start = gm.pending()
    glog, olog = forced_logits(gm, om, start, steps)
    cool = 16 * max(0, (ctx_len + steps - H - W) // 16)
    for p in list(range(0, cool, 37)) + ([cool - 1] if cool else []):
        for kv in range(2):
            form, g = gm.kv_read(cfg["n_layers"] - 1, 0, p, kv)
            assert form == 2 and np.array_equal(g, om.kv_read(cfg["n_layers"] - 1, 0, p, kv, 2)), (p, kv)
    gm.close()
    om.close()
    check_forced(glog, olog, TQ_TOL, TQ_TIE, f"seed {cfg['seed']:#x}")


def test_three_tier_empty_cool_range_matches_two_tiers(ctx):
    """A Warm range that covers the whole compressed part (no page ever
    reaches Cool): the three-tier launch (an empty Cool range, its extra
    records and compressor blocks) gives the two-tier model's tokens and
    logits within 1e-3."""
    base = dict(TQ_TINY, batch=2, max_seq=512, kv_kind=2, hot_window=32, seed=0x3C3)
    ctx_len, steps = 200, 12
    out = {}
    for W in (0, 448):
        m = nexus_amd.Model(ctx, **dict(base, warm_window=W))
        m.fill_context(ctx_len, 4)
        toks = m.decode(steps)
        out[W] = (toks, m.logits())
        form, _ = m.kv_read(0, 0, 0, 0)
        assert form == 1
        m.close()
    assert np.array_equal(out[0][0], out[448][0])
    assert rel_err(out[448][1], out[0][1]) < 1e-3


def test_three_tier_config_rejected(ctx):
    for W in (-16, 8, 24):
        with pytest.raises(RuntimeError):
            nexus_amd.Model(ctx, **dict(TQ_TINY, kv_kind=2, hot_window=32, warm_window=W))
    for kind in (0, 1):
        with pytest.raises(RuntimeError):
            nexus_amd.Model(ctx, **dict(TQ_TINY, kv_kind=kind, warm_window=32))


# ----------------------------------------------------------- Cold eviction --
@pytest.mark.parametrize("batch,H,W,C", [(1, 16, 16, 32), (2, 32, 16, 16)])
def test_evicting_tiers_greedy_parity(ctx, batch, H, W, C):
    """A 12-token prompt and 100 greedy tokens with a Cool window: from
    position H + W + C + 15 on, pages leave the Cool range and are evicted
    (read as zero keys and values, as get_vectors gathers a page it no longer
    holds); the Cool pages live in a ring of C / 16 + 1 pages."""
    cfg = dict(TQ_TINY, batch=batch, kv_kind=2, hot_window=H, warm_window=W, cool_window=C,
               seed=0xE71 + H + W + C)
    got, want, margins = run_both(ctx, cfg, P=12, n_new=100)
    assert_greedy_parity(got, want, margins, tie=TQ_DECODE_TIE)
    run_forced(ctx, cfg, 12, 100, tol=TQ_DECODE_TOL, tie=TQ_DECODE_TIE)


def test_evicting_tiers_filled_context(ctx):
    """300 filled positions, window 64, Warm 32, Cool 64: the fill evicts
    pages 0..7 and writes 8..11 Cool (into the ring), 12..13 TurboQuant;
    40 decode steps evict pages 8..10 and move 12..14 to the Cool ring.
    Stored pages stay bit-exact against the oracle, tokens agree."""
    cfg = dict(TQ_TINY, batch=2, max_seq=512, kv_kind=2, hot_window=64, warm_window=32, cool_window=64,
               seed=0xE72)
    ctx_len, steps = 300, 40
    gm = nexus_amd.Model(ctx, **cfg)
    gm.fill_context(ctx_len, 4)
    om = oracle.Model(**cfg)
    om.fill_context(ctx_len, 4)
    n_layers = cfg["n_layers"]

    def evicted(positions):
        for b in range(2):
            for p in positions:
                form, got = gm.kv_read(n_layers - 1, b, p, 0)
                assert form == 3 and got.size == 0, (b, p, form)

    evicted(range(0, 128, 9))
    _check_forms(gm, om, n_layers, 2, [(range(128, 192, 3), 2), (range(192, 224, 3), 1), (range(224, 300, 4), 0)])
    start = gm.pending()
    glog, olog = forced_logits(gm, om, start, steps)
    evicted([0, 127, 128, 175])
    _check_forms(gm, om, n_layers, 2, [(range(176, 240), 2), (range(240, 272), 1), (range(272, 300), 0)])
    gm.close()
    om.close()
    check_forced(glog, olog, TQ_TOL, TQ_TIE, f"seed {cfg['seed']:#x}")


def test_evicting_tiers_config_rejected(ctx):
    for C in (-16, 8):
        with pytest.raises(RuntimeError):
            nexus_amd.Model(ctx, **dict(TQ_TINY, kv_kind=2, hot_window=32, warm_window=16, cool_window=C))
    with pytest.raises(RuntimeError):  # a Cool window needs a Warm range
        nexus_amd.Model(ctx, **dict(TQ_TINY, kv_kind=2, hot_window=32, cool_window=32))
