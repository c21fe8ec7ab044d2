"""The fused attention block (QKV, paged attention and wo of a layer in one
launch, batch 1 over fp16 pages; selected with nx_model_set_fused) against
the separate launches and the oracle, on the GPU.

The two layouts compute the same values except for the attention's split
plan (the order in which split records are merged), so their greedy tokens
must agree and their logits agree to fp32 rounding.  The decodes cross page
boundaries, so the in-launch patch of the position's K/V slot into a page
requested before the slot was written is exercised at every page offset."""
import numpy as np
import pytest

import nexus_amd
import oracle
from conftest import rel_err
from test_gpu_model import LLAMA8B, TINY, assert_greedy_parity, top2_margin

pytestmark = pytest.mark.gpu


def _decode_both_layouts(ctx, cfg, ctx_len, steps):
    out = {}
    for fused in (True, False):
        print(f"[case] fused={fused} {cfg} ctx {ctx_len} steps {steps}", flush=True)
        gm = nexus_amd.Model(ctx, **cfg)
        gm.set_fused(fused)
        gm.fill_context(ctx_len, 0)
        toks = gm.decode(steps)
        out[fused] = (toks, gm.logits())
        gm.close()
    return out


def test_fused_tiny_greedy_parity(ctx):
    """The tiny model through the fused block: prompt of 16 (batched
    prefill), then 64 greedy tokens equal to the oracle's."""
    P, n_new = 16, 64
    prompt = oracle.prompt_tokens(TINY["seed"], 1, P, TINY["vocab"])
    om = oracle.Model(**TINY)
    want, margins = om.generate(prompt, n_new)
    om.close()
    gm = nexus_amd.Model(ctx, **TINY)
    gm.set_fused(True)
    first = gm.prefill(prompt)
    rest = gm.decode(n_new - 1)
    gm.close()
    got = np.concatenate([first[:, None], rest], axis=1)
    assert_greedy_parity(got, want, margins)


def test_fused_tiny_matches_separate_launches(ctx):
    cfg = dict(TINY, max_seq=256, seed=0xF05E)
    out = _decode_both_layouts(ctx, cfg, 100, 40)
    assert np.array_equal(out[True][0], out[False][0])
    assert rel_err(out[True][1], out[False][1]) < 1e-4


def test_fused_8b_two_layers_matches_separate_launches(ctx):
    """Two 8B-shaped layers over 4096 filled positions, 24 steps (positions
    4096..4119: two pages, every slot of the first)."""
    cfg = dict(LLAMA8B, n_layers=2, seed=0xF08B)
    out = _decode_both_layouts(ctx, cfg, 4096, 24)
    assert np.array_equal(out[True][0], out[False][0])
    assert rel_err(out[True][1], out[False][1]) < 1e-4


def test_fused_8b_one_layer_oracle_parity(ctx):
    """One 8B-shaped layer plus lm_head at 4096 filled positions through the
    fused block, three greedy steps against the oracle."""
    cfg = dict(LLAMA8B, n_layers=1, seed=0xF0A1)
    gm = nexus_amd.Model(ctx, **cfg)
    gm.set_fused(True)
    gm.fill_context(4096, 0)
    start = gm.pending()
    got = gm.decode(3)
    glog = gm.logits()
    gm.close()
    om = oracle.Model(**cfg)
    om.fill_context(4096, 0)
    tok, want, margins = start, [], []
    for _ in range(3):
        logits = om.forward(tok)
        tok = logits.argmax(axis=1).astype(np.int32)
        want.append(tok)
        margins.append(top2_margin(logits))
    om.close()
    want = np.stack(want, 1)
    assert_greedy_parity(got, want, np.stack(margins, 1))
    if np.array_equal(got, want):
        assert rel_err(glog, logits) < 1e-3


def test_fused_toggle_restarts_counters(ctx):
    """Switching layouts between decodes keeps the tokens of one layout's
    run (the in-launch counters restart with the step count)."""
    cfg = dict(TINY, max_seq=256, seed=0x70C1)
    gm = nexus_amd.Model(ctx, **cfg)
    gm.set_fused(True)
    gm.fill_context(60, 0)
    a = [gm.decode(5)]
    gm.set_fused(False)
    a.append(gm.decode(5))
    gm.set_fused(True)
    a.append(gm.decode(5))
    gm.close()
    ref = nexus_amd.Model(ctx, **cfg)
    ref.set_fused(False)
    ref.fill_context(60, 0)
    b = ref.decode(15)
    ref.close()
    assert np.array_equal(np.concatenate(a, axis=1), b)


def test_fused_unsupported_is_an_error(ctx):
    gm = nexus_amd.Model(ctx, **dict(TINY, batch=2))
    with pytest.raises(nexus_amd.NxError) as e:
        gm.set_fused(True)
    assert e.value.code == 4
    gm.set_fused(False)
    gm.close()
