"""nx_attn_decode_paged_f16_noalloc: the fp16 paged attention with its split
records and counters in the library's static device scratch.  Its output
must equal nx_attn_decode_paged_f16's on the same inputs (same kernels, same
split plan: bit for bit) on consecutive calls, the second smaller than the
first (the scratch keeps the first call's contents), inside a captured token
graph replayed with eager work between the replays, and against the oracle
within 1e-3.  A sequence whose block table names a block outside the pool
gets NaN rows and leaves the other sequences' rows intact; shapes whose
split plan needs more scratch than the array holds are refused."""
import numpy as np
import pytest

import oracle
from conftest import f16, rel_err
from test_gpu_kernels import _pools, up

pytestmark = pytest.mark.gpu
L = oracle.lib


def _case(ctx, hq, hkv, hd, lens, seed):
    rng = np.random.default_rng(seed)
    B = len(lens)
    max_blocks, nblk, bt, kp, vp = _pools(rng, B, hkv, hd, lens, seed=seed)
    q = rng.normal(0, 1, (B, hq, hd)).astype(np.float32)
    ln = np.array(lens, np.int32)
    bufs = dict(q=up(ctx, q), kp=up(ctx, kp), vp=up(ctx, vp), bt=up(ctx, bt), ln=up(ctx, ln),
                out=ctx.alloc(B * hq * hd * 2))
    want = np.empty_like(q)
    L.nxo_attn_decode_paged_f16(q, np.ascontiguousarray(kp.reshape(-1)), np.ascontiguousarray(vp.reshape(-1)),
                                bt, max_blocks, ln, B, hq, hkv, hd, want)
    return dict(B=B, hq=hq, hkv=hkv, hd=hd, max_blocks=max_blocks, nblk=nblk, bt=bt, q=q, bufs=bufs, want=want)


def _run(ctx, c, noalloc, capture=False):
    b = c["bufs"]
    fn = ctx.L.nx_attn_decode_paged_f16_noalloc if noalloc else ctx.L.nx_attn_decode_paged_f16
    if capture:
        ctx.check(ctx.L.nx_token_begin(ctx.h), "begin")
    ctx.check(fn(ctx.h, b["q"], b["kp"], b["vp"], b["bt"], b["ln"], b["out"], c["B"], c["hq"], c["hkv"], c["hd"],
                 c["max_blocks"], c["nblk"]), "attn")
    if capture:
        ctx.check(ctx.L.nx_token_end(ctx.h), "end")
    return ctx.download(b["out"], (c["B"], c["hq"], c["hd"]), np.uint16)


def _free(ctx, c):
    for v in c["bufs"].values():
        ctx.free(v)


def test_noalloc_attention_matches_allocating_entry_point(ctx):
    """Two calls in a row, the second with fewer sequences, heads and
    positions: each equals the allocating entry point bit for bit and the
    oracle within 1e-3."""
    big = _case(ctx, 32, 8, 128, [4096, 1000], 21)
    small = _case(ctx, 8, 2, 64, [300], 22)
    for c in (big, small):
        got = _run(ctx, c, True)
        ref = _run(ctx, c, False)
        assert np.array_equal(got, ref)
        for b in range(c["B"]):
            assert rel_err(f16(got[b]), c["want"][b]) < 1e-3
    _free(ctx, big)
    _free(ctx, small)


def test_noalloc_attention_in_a_captured_graph(ctx):
    """Captured into a token graph: each replay, with a new q uploaded and an
    eager call between replays, gives the eager result."""
    c = _case(ctx, 32, 8, 128, [2048, 77, 513], 23)
    rng = np.random.default_rng(24)
    for rep in range(3):
        q = rng.normal(0, 1, c["q"].shape).astype(np.float32)
        ctx.upload(q, c["bufs"]["q"])
        got = _run(ctx, c, True, capture=True)
        eager = _run(ctx, c, True)
        ref = _run(ctx, c, False)
        assert np.array_equal(got, ref), rep
        assert np.array_equal(eager, ref), rep
    _free(ctx, c)


def test_noalloc_attention_bad_table_gives_nan_rows(ctx):
    """A block-table entry of sequence 1 outside the pool (and a context
    length past the table for sequence 2): those sequences' rows are NaN
    (no page outside the pool is read), sequence 0 still equals the oracle."""
    c = _case(ctx, 32, 8, 128, [700, 700, 700], 25)
    bt = c["bt"].copy()
    bt[1, 3] = c["nblk"] + 1000
    ctx.upload(np.ascontiguousarray(bt), c["bufs"]["bt"])
    ctx.upload(np.array([700, 700, c["max_blocks"] * 16 + 1], np.int32), c["bufs"]["ln"])
    got = f16(_run(ctx, c, True))
    assert rel_err(got[0], c["want"][0]) < 1e-3
    assert np.all(np.isnan(got[1])) and np.all(np.isnan(got[2]))
    _free(ctx, c)


def test_noalloc_attention_refuses_beyond_scratch(ctx):
    """33 sequences x 8 kv heads need 264 split counters' worth of scratch
    rows: more than the static array holds, refused before any launch."""
    B, hq, hkv, hd, mb = 33, 32, 8, 64, 2
    nblk = B * mb
    bufs = [ctx.alloc(B * hq * hd * 4), ctx.alloc(nblk * hkv * 16 * hd * 2), ctx.alloc(nblk * hkv * 16 * hd * 2),
            up(ctx, np.zeros((B, mb), np.int32)), up(ctx, np.ones(B, np.int32)), ctx.alloc(B * hq * hd * 2)]
    st = ctx.L.nx_attn_decode_paged_f16_noalloc(ctx.h, *bufs, B, hq, hkv, hd, mb, nblk)
    assert st == 4, st
    for bb in bufs:
        ctx.free(bb)
