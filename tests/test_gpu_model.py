"""End-to-end decode-loop parity on the GPU against the oracle on the same
seeded model, prompt and context: greedy token ids produced by the HIP
runner (one HIP graph per step, token fed back on the device) must equal
the oracle's, and in teacher-forced runs (both sides consume the oracle's
tokens) the logits of every step must agree within 1e-3 (TQ_TOL where the
decode writes TurboQuant pages)."""
import numpy as np
import pytest

import nexus_amd
import oracle
from conftest import TIE_MARGIN, TQ_DECODE_TIE, TQ_DECODE_TOL, TQ_TIE, TQ_TOL, check_forced, forced_logits, rel_err

pytestmark = pytest.mark.gpu

TINY = dict(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=688, vocab=4096,
            n_experts=0, top_k=0, max_seq=128, batch=1, kv_kind=0, rope_theta=10000.0, eps=1e-5,
            seed=0x5EED)


def assert_greedy_parity(got, want, margins, tie=TIE_MARGIN):
    """Token ids must be identical; the only allowed difference is at a step
    whose oracle margin is a numerical tie, after which the sequences
    legitimately diverge."""
    for b in range(want.shape[0]):
        diff = np.nonzero(got[b] != want[b])[0]
        if diff.size:
            i = int(diff[0])
            print(f"[parity] sequence {b}: diverged at token {i} of {want.shape[1]}, oracle margin "
                  f"{margins[b, i]:.3g}", flush=True)
            assert margins[b, i] < tie, (
                f"sequence {b}: token {i} differs ({got[b, i]} vs {want[b, i]}) "
                f"at oracle margin {margins[b, i]:.3g}")
        else:
            print(f"[parity] sequence {b}: {want.shape[1]} tokens identical", flush=True)


def top2_margin(logits):
    """top1 - top2 logit per row."""
    part = np.sort(logits, axis=1)
    return part[:, -1] - part[:, -2]


def run_both(ctx, cfg, P=16, n_new=64):
    prompt = oracle.prompt_tokens(cfg["seed"], cfg["batch"], P, cfg["vocab"])
    om = oracle.Model(**cfg)
    want, margins = om.generate(prompt, n_new)
    om.close()
    gm = nexus_amd.Model(ctx, **cfg)
    first = gm.prefill(prompt)
    rest = gm.decode(n_new - 1)
    got = np.concatenate([first[:, None], rest], axis=1)
    assert gm.position(0) == P + n_new - 2
    gm.close()
    return got, want, margins


def run_forced(ctx, cfg, P, n_new, tol=1e-3, tie=TIE_MARGIN, batched=True):
    """The prompt through both sides (the GPU's prefill: batched or one step
    per token), the prefill's last logits within tol, then n_new
    teacher-forced steps from the oracle's first token (check_forced)."""
    prompt = oracle.prompt_tokens(cfg["seed"], cfg["batch"], P, cfg["vocab"])
    om = oracle.Model(**cfg)
    for t in range(P):
        olast = om.forward(np.ascontiguousarray(prompt[:, t]))
    gm = nexus_amd.Model(ctx, **cfg)
    gm.set_prefill(batched)
    gm.prefill(prompt)
    assert rel_err(gm.logits(), olast) < tol
    glog, olog = forced_logits(gm, om, olast.argmax(axis=1).astype(np.int32), n_new)
    assert gm.position(0) == P + n_new - 1
    gm.close()
    om.close()
    return check_forced(glog, olog, tol, tie, f"prompt {P} + {n_new} forced, seed {cfg['seed']:#x}")


def test_tiny_greedy_parity(ctx):
    """The tiny Llama-style model: 16-token prompt, 64 greedy tokens
    (identical ids), and the same 64 steps teacher-forced (logits)."""
    got, want, margins = run_both(ctx, TINY)
    print("min top1-top2 margin", float(margins.min()))
    assert_greedy_parity(got, want, margins)
    run_forced(ctx, TINY, 16, 64)


def test_tiny_greedy_parity_batch2(ctx):
    cfg = dict(TINY, batch=2, seed=0xBEEF)
    got, want, margins = run_both(ctx, cfg, P=9, n_new=24)
    assert_greedy_parity(got, want, margins)
    run_forced(ctx, cfg, 9, 24)


def test_tiny_moe_greedy_parity(ctx):
    cfg = dict(TINY, n_experts=4, top_k=2, seed=0x0E0E)
    got, want, margins = run_both(ctx, cfg, P=8, n_new=24)
    assert_greedy_parity(got, want, margins)
    run_forced(ctx, cfg, 8, 24)


def test_tiny_moe_greedy_parity_batch3(ctx):
    cfg = dict(TINY, n_experts=8, top_k=2, batch=3, seed=0x0E0F)
    got, want, margins = run_both(ctx, cfg, P=5, n_new=12)
    assert_greedy_parity(got, want, margins)
    run_forced(ctx, cfg, 5, 12)


def test_tiny_turboquant_greedy_parity(ctx):
    cfg = dict(TINY, n_heads=4, n_kv_heads=1, head_dim=128, kv_kind=1, seed=0x7777, d_model=512)
    got, want, margins = run_both(ctx, cfg, P=12, n_new=24)
    assert_greedy_parity(got, want, margins, tie=TQ_DECODE_TIE)
    run_forced(ctx, cfg, 12, 24, tol=TQ_DECODE_TOL, tie=TQ_DECODE_TIE)


@pytest.mark.parametrize("E,k,batch", [(64, 10, 1), (256, 16, 2), (16, 10, 3)])
def test_wide_moe_parity(ctx, E, k, batch):
    """Routing over up to 256 experts with up to 16 per token (the
    reference's default top-10, hybrid_model.cpp:1648; any E, :1647-1711):
    routing in its own launch past 16 experts, the routed GEMVs over up to 32
    active experts, batched prefill routing, greedy tokens and teacher-forced
    logits against the oracle."""
    cfg = dict(TINY, n_experts=E, top_k=k, batch=batch, seed=0xE000 + E + k)
    got, want, margins = run_both(ctx, cfg, P=7, n_new=16)
    assert_greedy_parity(got, want, margins)
    run_forced(ctx, cfg, 7, 16)


@pytest.mark.parametrize("d,F,k", [(8192, 1024, 1), (2048, 7168, 2), (512, 14336, 3)])
def test_moe_batch1_routed_shapes(ctx, d, F, k):
    """Batch-1 routed experts at the widths whose kernels no other test
    reaches: d_model 8192 (the routing gate/up launch with x in LDS), an FFN
    of 7168 and 14336 (the down projection with the combine at 4 and 7
    groups per lane), top-1 (one slot per output row) and top-3 (the
    separate down projection and combine after the routing gate/up launch);
    greedy tokens and teacher-forced logits against the oracle."""
    cfg = dict(TINY, n_layers=1, d_model=d, ffn=F, n_experts=4, top_k=k, vocab=2048, seed=0xB100 + k)
    got, want, margins = run_both(ctx, cfg, P=5, n_new=8)
    assert_greedy_parity(got, want, margins)
    run_forced(ctx, cfg, 5, 8)


@pytest.mark.parametrize("batch,qk", [(1, 0), (3, 1)])
def test_head_dim_256_parity(ctx, batch, qk):
    """256-long heads (the Gemma-style width the reference's Q/K-norm code
    defaults to, hybrid_model.cpp:1328): RoPE, the page layout, the split
    attention and its merge over 256 dimensions, with and without the Q/K
    norm, against the oracle (tokens and teacher-forced logits)."""
    cfg = dict(TINY, n_heads=4, n_kv_heads=2, head_dim=256, d_model=512, batch=batch, qk_norm=qk, norm_sigma=0.1,
               seed=0x2560 + batch)
    got, want, margins = run_both(ctx, cfg, P=9, n_new=20)
    assert_greedy_parity(got, want, margins)
    run_forced(ctx, cfg, 9, 20)


def test_wide_ffn_and_heads_parity(ctx):
    """An FFN of 16384 and 64 query heads of 256 (hq * hd = 16384): the down
    projection and wo take K beyond 14336 (the batch-1 kernel with x in LDS,
    the matrix cores at batch 2), against the oracle."""
    for batch in (1, 2):
        cfg = dict(TINY, d_model=512, n_heads=64, n_kv_heads=8, head_dim=256, ffn=16384, batch=batch,
                   seed=0x7A0B + batch)
        got, want, margins = run_both(ctx, cfg, P=5, n_new=8)
        assert_greedy_parity(got, want, margins)
        run_forced(ctx, cfg, 5, 8)


QK = dict(qk_norm=1, norm_sigma=0.1)


@pytest.mark.parametrize("name,extra,batched", [
    ("dense", {}, True), ("dense-steps", {}, False), ("batch3", {"batch": 3}, True),
    ("moe", {"n_experts": 4, "top_k": 2}, True),
    ("turboquant", {"n_heads": 4, "n_kv_heads": 1, "head_dim": 128, "d_model": 512, "kv_kind": 1}, True),
    ("tiered", {"n_heads": 4, "n_kv_heads": 2, "head_dim": 128, "d_model": 512, "kv_kind": 2, "hot_window": 16},
     True),
    ("tiered-steps", {"n_heads": 4, "n_kv_heads": 2, "head_dim": 128, "d_model": 512, "kv_kind": 2,
                      "hot_window": 16}, False),
    ("hd128-batch8", {"n_heads": 8, "n_kv_heads": 2, "head_dim": 128, "d_model": 512, "batch": 8}, True)])
def test_qk_norm_parity(ctx, name, extra, batched):
    """Per-head Q/K RMSNorm (attn_q_norm / attn_k_norm, hybrid_model.cpp:
    1325-1349) before RoPE, with non-unit weights: the decode step (batch 1
    streaming GEMV, batch 3 and 8 on the matrix cores, MoE, TurboQuant and
    tiered pages) and the prefill (batched GEMM or one step per token) give
    the oracle's tokens and logits."""
    cfg = dict(TINY, seed=0x9C00 + len(name), **QK, **extra)
    tq = cfg["kv_kind"] != 0
    P, n = 11, 24
    got, want, margins = run_both(ctx, cfg, P=P, n_new=n)
    assert_greedy_parity(got, want, margins, tie=TQ_DECODE_TIE if tq else TIE_MARGIN)
    run_forced(ctx, cfg, P, n, tol=TQ_DECODE_TOL if tq else 1e-3, tie=TQ_DECODE_TIE if tq else TIE_MARGIN,
               batched=batched)


def test_qk_norm_changes_the_model(ctx):
    """The same seeded model with and without the Q/K norm decodes different
    logits (the norm is applied, not skipped)."""
    out = []
    for qk in (0, 1):
        gm = nexus_amd.Model(ctx, **dict(TINY, qk_norm=qk, norm_sigma=0.1, seed=0x9C77))
        gm.prefill(oracle.prompt_tokens(0x9C77, 1, 8, TINY["vocab"]))
        out.append(gm.logits())
        gm.close()
    assert rel_err(out[1], out[0]) > 0.05


@pytest.mark.parametrize("kv_kind,n_outlier", [(0, 0), (1, 4)])
def test_filled_context_decode_parity(ctx, kv_kind, n_outlier):
    cfg = dict(TINY, n_kv_heads=2, n_heads=4, head_dim=128, d_model=512, max_seq=512, batch=2,
               kv_kind=kv_kind, seed=0xC0DE)
    ctx_len, steps = 300, 10
    gm = nexus_amd.Model(ctx, **cfg)
    gm.fill_context(ctx_len, n_outlier)
    start = gm.pending()
    got = gm.decode(steps)
    glog = gm.logits()
    gm.close()
    om = oracle.Model(**cfg)
    om.fill_context(ctx_len, n_outlier)
    want_start = np.array([oracle.lib.nxo_rand_u64(cfg["seed"], 5, b) % cfg["vocab"] for b in range(2)], np.int32)
    assert np.array_equal(start, want_start)
    tok = start
    want = []
    margins = []
    for _ in range(steps):
        logits = om.forward(tok)
        tok = logits.argmax(axis=1).astype(np.int32)
        want.append(tok)
        margins.append(top2_margin(logits))
    om.close()
    assert_greedy_parity(got, np.stack(want, 1), np.stack(margins, 1),
                         tie=TQ_TIE if kv_kind else TIE_MARGIN)
    # the same context teacher-forced: every step's logits
    gm = nexus_amd.Model(ctx, **cfg)
    gm.fill_context(ctx_len, n_outlier)
    om = oracle.Model(**cfg)
    om.fill_context(ctx_len, n_outlier)
    glog, olog = forced_logits(gm, om, want_start, steps)
    gm.close()
    om.close()
    check_forced(glog, olog, TQ_TOL if kv_kind else 1e-3, TQ_TIE if kv_kind else TIE_MARGIN,
                 f"filled {ctx_len}, kv_kind {kv_kind}")


LLAMA8B = dict(n_layers=32, d_model=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=14336,
               vocab=128256, n_experts=0, top_k=0, max_seq=4096 + 256, batch=1, kv_kind=0,
               rope_theta=500000.0, eps=1e-5, seed=0x5EED)


def test_8b_one_layer_full_shape_parity(ctx):
    """Full Llama-3-8B layer and lm_head shapes (one layer) at 512 context:
    three greedy steps with the token fed back on the device, then eight
    teacher-forced steps on a second model (logits of every step)."""
    cfg = dict(LLAMA8B, n_layers=1, max_seq=1024)
    gm = nexus_amd.Model(ctx, **cfg)
    gm.fill_context(512, 0)
    got = gm.decode(3)
    gm.close()
    om = oracle.Model(**cfg)
    om.fill_context(512, 0)
    tok = np.array([oracle.lib.nxo_rand_u64(cfg["seed"], 5, 0) % cfg["vocab"]], np.int32)
    start = tok
    want, margins = [], []
    for _ in range(3):
        logits = om.forward(tok)
        tok = logits.argmax(axis=1).astype(np.int32)
        want.append(tok)
        margins.append(top2_margin(logits))
    om.close()
    assert_greedy_parity(got, np.stack(want, 1), np.stack(margins, 1))
    gm = nexus_amd.Model(ctx, **cfg)
    gm.fill_context(512, 0)
    om = oracle.Model(**cfg)
    om.fill_context(512, 0)
    glog, olog = forced_logits(gm, om, start, 8)
    gm.close()
    om.close()
    check_forced(glog, olog, 1e-3, TIE_MARGIN, "8B layer, ctx 512")


def test_8b_decode_properties(ctx):
    """The full 32-layer 8B shape at 4096 context: deterministic, in range,
    and the algorithmic bytes of a step match the closed form."""
    gm = nexus_amd.Model(ctx, **LLAMA8B)
    gm.fill_context(4096, 0)
    bytes_at_4096 = gm.step_bytes()
    # weights 4,221,370,368 B + fp16 KV of 4096 positions x 32 layers
    assert abs(bytes_at_4096 - (4221370368 + 536870912)) < 1e6
    a = gm.decode(6)
    assert a.min() >= 0 and a.max() < LLAMA8B["vocab"]
    assert np.all(np.isfinite(gm.logits()))
    gm.close()
    gm2 = nexus_amd.Model(ctx, **LLAMA8B)
    gm2.fill_context(4096, 0)
    b = gm2.decode(6)
    gm2.close()
    assert np.array_equal(a, b)


def test_capacity_is_an_error(ctx):
    gm = nexus_amd.Model(ctx, **dict(TINY, max_seq=32))
    gm.prefill(np.arange(20, dtype=np.int32)[None, :])
    with pytest.raises(nexus_amd.NxError) as e:
        gm.decode(20)
    assert e.value.code == 7
    gm.close()
