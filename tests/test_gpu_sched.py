"""Sequences joining and leaving a batch (nx_model_admit / nx_model_retire)
and the request scheduler (nx_sched) on the GPU: every sequence's greedy
tokens equal the oracle's for that sequence decoded alone, whatever its
prompt length, the slot it lands in and what the other slots do meanwhile."""
import numpy as np
import pytest

import nexus_amd
import oracle
from test_gpu_model import TINY, assert_greedy_parity

pytestmark = pytest.mark.gpu


def standalone(cfg, prompt, n):
    om = oracle.Model(**dict(cfg, batch=1))
    want, margins = om.generate(np.asarray(prompt, np.int32)[None, :], n)
    om.close()
    return want[0], margins[0]


def prompts(cfg, lens):
    return [oracle.prompt_tokens(cfg["seed"] + 17 * i + 1, 1, n, cfg["vocab"])[0] for i, n in enumerate(lens)]


CFGS = {
    "dense": dict(TINY, batch=3, max_seq=128, seed=0x5C01),
    "dense-steps": dict(TINY, batch=3, max_seq=128, seed=0x5C02),
    "moe": dict(TINY, batch=3, max_seq=128, n_experts=4, top_k=2, seed=0x5C03),
    "turboquant": dict(TINY, batch=3, max_seq=128, n_heads=4, n_kv_heads=1, head_dim=128, d_model=512,
                       kv_kind=1, seed=0x5C04),
    # a shared pool of 4 pages (the three slots would hold 24): C takes A's page
    "dense-pool": dict(TINY, batch=3, max_seq=128, seed=0x5C07, kv_blocks=4),
    "turboquant-pool": dict(TINY, batch=3, max_seq=128, n_heads=4, n_kv_heads=1, head_dim=128, d_model=512,
                            kv_kind=1, seed=0x5C08, kv_blocks=4),
    "tiered-pool": dict(TINY, batch=3, max_seq=128, n_heads=4, n_kv_heads=1, head_dim=128, d_model=512,
                        kv_kind=2, hot_window=16, seed=0x5C09, kv_blocks=4),
}


@pytest.mark.parametrize("kind", sorted(CFGS))
def test_admit_and_retire_mid_decode(ctx, kind):
    """A joins slot 0; after 6 steps B joins slot 1; after 5 more A leaves
    and C joins slot 0; slot 2 stays free throughout.  Dense models prefill
    an admitted prompt as a batched GEMM pass ("dense-steps" turns that off),
    the others one step per prompt token while the other sequences are held."""
    cfg = CFGS[kind]
    print(f"[case] {kind}", flush=True)
    A, B, C = prompts(cfg, [5, 9, 3])
    gm = nexus_amd.Model(ctx, **cfg)
    if kind == "dense-steps":
        gm.set_prefill(False)
    for s in range(3):
        gm.retire(s)
    got = {"A": [gm.admit(0, A)], "B": [], "C": []}
    out = gm.decode(6)
    got["A"] += out[0].tolist()
    assert (out[1] == -1).all() and (out[2] == -1).all()
    got["B"].append(gm.admit(1, B))
    out = gm.decode(5)
    got["A"] += out[0].tolist()
    got["B"] += out[1].tolist()
    gm.retire(0)
    assert not gm.slot_active(0) and gm.slot_active(1)
    got["C"].append(gm.admit(0, C))
    out = gm.decode(7)
    got["B"] += out[1].tolist()
    got["C"] += out[0].tolist()
    assert (out[2] == -1).all()
    if "kv_blocks" in cfg:
        # B holds positions 0..20 (two pages), C 0..9 (one)
        assert gm.kv_pages() == (4, 1)
        gm.retire(0)
        gm.retire(1)
        assert gm.kv_pages() == (4, 4)
    gm.close()
    for name, p in (("A", A), ("B", B), ("C", C)):
        want, margins = standalone(cfg, p, len(got[name]))
        assert_greedy_parity(np.array([got[name]]), want[None, :], margins[None, :])


def test_scheduler_serves_requests_in_two_slots(ctx):
    """Five requests of different prompt lengths and token counts through two
    slots, one of them stopping at a token it emits; each request's tokens
    equal the oracle's for it alone."""
    cfg = dict(TINY, batch=2, max_seq=128, seed=0x5C05)
    lens, counts = [4, 11, 6, 2, 9], [7, 3, 10, 5, 6]
    ps = prompts(cfg, lens)
    wants = [standalone(cfg, p, n) for p, n in zip(ps, counts)]
    stop = int(wants[2][0][2])  # request 2 stops at the third token it emits (first occurrence)
    first = int(np.nonzero(wants[2][0] == stop)[0][0])
    gm = nexus_amd.Model(ctx, **cfg)
    sched = nexus_amd.Scheduler(gm)
    ids = [sched.submit(p, n, stop if i == 2 else -1) for i, (p, n) in enumerate(zip(ps, counts))]
    sched.run()
    for i, rid in enumerate(ids):
        out, done = sched.result(rid)
        assert done
        want, margins = wants[i]
        n = first + 1 if i == 2 else counts[i]
        assert len(out) == n, (i, len(out), n)
        assert_greedy_parity(out[None, :], want[None, :n], margins[None, :n])
    sched.close()
    gm.close()


def test_scheduler_rejects_what_cannot_fit(ctx):
    cfg = dict(TINY, batch=2, max_seq=32, seed=0x5C06)
    gm = nexus_amd.Model(ctx, **cfg)
    sched = nexus_amd.Scheduler(gm)
    with pytest.raises(nexus_amd.NxError) as e:
        sched.submit(np.zeros(20, np.int32), 20)
    assert e.value.code == 7
    with pytest.raises(nexus_amd.NxError):
        sched.submit(np.array([cfg["vocab"]], np.int32), 2)
    sched.close()
    gm.close()


def test_scheduler_waits_for_pool_pages(ctx):
    """A shared pool of 8 pages under three slots: requests are admitted in
    arrival order only while their pages to the last position fit (A 4 + B 2,
    then C 4 waits for A), every request's tokens equal the oracle's for it
    alone, and the pool is whole again at the end."""
    cfg = dict(TINY, batch=3, max_seq=128, seed=0x5C0A, kv_blocks=8)
    lens, counts = [20, 5, 30, 9, 14], [40, 20, 30, 12, 50]  # pages 4, 2, 4, 2, 4
    ps = prompts(cfg, lens)
    wants = [standalone(cfg, p, n) for p, n in zip(ps, counts)]
    gm = nexus_amd.Model(ctx, **cfg)
    sched = nexus_amd.Scheduler(gm)
    ids = [sched.submit(p, n) for p, n in zip(ps, counts)]
    sched.step()
    assert gm.slot_active(0) and gm.slot_active(1) and not gm.slot_active(2)  # C waits for pages
    sched.run()
    for i, rid in enumerate(ids):
        out, done = sched.result(rid)
        assert done and len(out) == counts[i]
        want, margins = wants[i]
        assert_greedy_parity(out[None, :], want[None, :], margins[None, :])
    assert gm.kv_pages() == (8, 8)
    with pytest.raises(nexus_amd.NxError) as e:  # 9 pages: more than the pool
        sched.submit(np.zeros(100, np.int32), 40)
    assert e.value.code == 7
    sched.close()
    gm.close()


def test_pool_exhaustion_fails_before_the_step(ctx):
    """One sequence in a pool of 3 pages: decode to position 47 works and
    matches the oracle; the next step needs a fourth page and fails with
    NX_ERR_CAPACITY without running."""
    cfg = dict(TINY, batch=1, max_seq=128, seed=0x5C0B, kv_blocks=3)
    prompt = prompts(cfg, [10])[0]
    want, margins = standalone(cfg, prompt, 39)
    gm = nexus_amd.Model(ctx, **cfg)
    first = gm.prefill(np.asarray(prompt, np.int32)[None, :])
    got = np.concatenate([first, gm.decode(38)[0]])  # positions 10..47
    assert gm.kv_pages() == (3, 0)
    assert_greedy_parity(got[None, :], want[None, :], margins[None, :])
    with pytest.raises(nexus_amd.NxError) as e:
        gm.decode(1)
    assert e.value.code == 7
    assert gm.position(0) == 47
    gm.close()


def test_scheduler_admission_failure_completes_the_request(ctx):
    """A request whose admission fails leaves the queue as complete with the
    admission's status instead of being dropped: here the pool's pages were
    taken by a sequence admitted into slot 1 directly (not through the
    scheduler), so admitting the request into slot 0 runs out of pages.  The
    step reports NX_ERR_CAPACITY, the request's result carries it, slot 0
    stays free, and the next request is served (tokens equal to the oracle's
    for it alone) once the pages are back."""
    cfg = dict(TINY, batch=2, max_seq=128, seed=0x5C0C, kv_blocks=8)
    p_long, p_req, p_next = prompts(cfg, [90, 40, 12])  # pages 6 (admitted directly), 3 at admission, 1
    gm = nexus_amd.Model(ctx, **cfg)
    sched = nexus_amd.Scheduler(gm)
    gm.admit(1, p_long)
    assert gm.kv_pages() == (8, 2)
    rid = sched.submit(p_req, 20)
    with pytest.raises(nexus_amd.NxError) as e:
        sched.step()
    assert e.value.code == 7
    with pytest.raises(nexus_amd.NxError) as e:
        sched.result(rid)
    assert e.value.code == 7
    assert not gm.slot_active(0)
    gm.retire(1)
    assert gm.kv_pages() == (8, 8)
    rid2 = sched.submit(p_next, 10)
    sched.run()  # the failed request is not tried again
    out, done = sched.result(rid2)
    want, margins = standalone(cfg, p_next, 10)
    assert done and len(out) == 10
    assert_greedy_parity(out[None, :], want[None, :], margins[None, :])
    sched.close()
    gm.close()
