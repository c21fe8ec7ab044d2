"""Token sampling (HybridModel::Impl::sample_token, hybrid_model.cpp:2023-2099):
the oracle's MT19937 against numpy's (the generator of std::mt19937), the
oracle sampler against an independent float64 restatement, and the GPU
sampler (nx_sample, and sampling inside the decode graph) against the
oracle wherever the decision is not within rounding of a boundary."""
import numpy as np
import pytest

import nexus_amd
import oracle

L = oracle.lib


def mt_first(seed, n=1):
    out = np.empty(n, np.uint32)
    L.nxo_mt19937(seed, n, out)
    return out


def draw(seed):
    return L.nxo_canonical_f32(int(mt_first(seed)[0]))


def test_mt19937_matches_numpy_and_the_standard():
    """The 10000th output for the default seed 5489 is 4123659995 (required
    of std::mt19937 by the C++ standard); numpy's RandomState is the same
    generator and seeding."""
    assert mt_first(5489, 10000)[-1] == 4123659995
    for seed in (1, 42, 5489, 0xDEADBEEF):
        want = np.random.RandomState(seed).randint(0, 2**32, size=700, dtype=np.uint32)
        assert np.array_equal(mt_first(seed, 700), want)


def test_canonical_draw():
    assert L.nxo_canonical_f32(0) == 0.0
    assert L.nxo_canonical_f32(0xFFFFFFFF) == np.nextafter(np.float32(1), np.float32(0))
    assert L.nxo_canonical_f32(1 << 31) == 0.5


def ref64(logits, T, top_k, top_p, u, with_kept=False):
    """The reference algorithm in float64 with numpy, written independently
    of the oracle: returns (token, margin), margin = the smallest relative
    distance of a decision (top-p crossing, draw) from its boundary (and the
    number of entries kept, with_kept)."""
    l = logits.astype(np.float64)
    p = np.exp((l - l.max()) / T)
    p /= p.sum()
    order = np.lexsort((np.arange(len(p)), -p))  # descending, ties by index
    margin = 1.0
    if 0 < top_k < len(p):
        q = np.zeros_like(p)
        q[order[:top_k]] = p[order[:top_k]]
        p = q
    if top_p < 1:
        order = np.lexsort((np.arange(len(p)), -p))
        cs = np.cumsum(p[order])
        if (cs > top_p).any():  # no element crosses: nothing is cut
            cut = int(np.argmax(cs > top_p))
            q = np.zeros_like(p)
            q[order[:cut + 1]] = p[order[:cut + 1]]
            p = q
        margin = min(margin, np.min(np.abs(cs - top_p)) / top_p)
    s = p.sum()
    r = u * s
    cs = np.cumsum(p)
    tok = int(np.argmax(cs >= r)) if r > 0 else 0
    margin = min(margin, np.min(np.abs(cs[p > 0] - r)) / s) if r > 0 else margin
    if with_kept:
        return tok, margin, int((p > 0).sum())
    return tok, margin


def tol_fp32_sequential(V, kept):
    """How far from a boundary a decision must be for the reference's fp32
    arithmetic (and the oracle's, which restates it) to reach it as float64
    does: the softmax denominator is a sequential sum over V entries, the
    top-p and draw running sums over the kept ones."""
    return max(1e-5, 2.0 * kept * 2.0**-24, 6.0 * np.sqrt(V) * 2.0**-24)


def tol_gpu(kept):
    """The same for the GPU sampler: fixed-order block sums for the
    denominator and the draw, exact fixed-point sums for a top-p cut over
    all candidates, a sequential fp32 sum in sorted order over at most 1024
    candidates otherwise."""
    return max(2e-5, 2.0 * min(kept, 1024) * 2.0**-24)


CASES = [(4096, 0.7, 40, 0.9), (4096, 1.3, 1, 1.0), (32000, 0.7, 40, 0.9), (32000, 1.0, 1024, 0.95),
         (32000, 0.8, 0, 1.0), (4096, 0.5, 7, 0.5),
         # pure nucleus (top_k 0) and top-k above the candidate list, with and without top-p
         (32000, 0.7, 0, 0.9), (4096, 1.0, 0, 0.5), (32000, 0.9, 5000, 1.0), (32000, 0.8, 4000, 0.8)]


@pytest.mark.parametrize("V,T,top_k,top_p", CASES)
def test_oracle_sampler_matches_float64_restatement(V, T, top_k, top_p):
    rng = np.random.default_rng(V + top_k)
    checked = 0
    for rep in range(40):
        logits = (rng.standard_normal(V) * 3).astype(np.float32)
        u = draw(rep + 1)
        want, margin, kept = ref64(logits, T, top_k, top_p, u, with_kept=True)
        got = L.nxo_sample(logits, V, T, top_k, top_p, u)
        if margin > tol_fp32_sequential(V, kept):
            assert got == want, (rep, got, want, margin)
            checked += 1
    # the inputs are seeded, so every case checks a fixed number of its 40
    # draws (19 to 40 of them)
    print(f"oracle == float64 on {checked} of 40 draws")
    assert checked >= 15


def test_oracle_sampler_limits():
    rng = np.random.default_rng(0)
    logits = rng.standard_normal(1000).astype(np.float32)
    am = int(np.argmax(logits))
    assert L.nxo_sample(logits, 1000, 0.0, 40, 0.9, 0.5) == am       # greedy
    assert L.nxo_sample(logits, 1000, 0.7, 1, 1.0, 0.99) == am       # top-1
    assert L.nxo_sample(logits, 1000, 0.7, 40, 1e-6, 0.99) == am     # top-p keeps the first
    assert L.nxo_sample(logits, 1000, 0.7, 0, 1.0, 0.0) == 0         # r = 0 reaches index 0


@pytest.mark.gpu
@pytest.mark.parametrize("V,T,top_k,top_p", CASES + [(128256, 0.7, 40, 0.9), (128256, 0.6, 0, 1.0),
                                                     (128256, 0.7, 0, 0.9), (128256, 0.8, 2000, 0.95)])
def test_gpu_sampler_matches_oracle(ctx, V, T, top_k, top_p):
    """nx_sample on 16 rows per launch, draws from seeded MT19937: the
    float64 restatement's token wherever the decision is farther from a
    boundary than the GPU's rounding reaches, and the oracle's (the
    reference's fp32 arithmetic) wherever it is farther than that one's."""
    rng = np.random.default_rng(V * 3 + top_k)
    B = 16
    checked = checked_o = 0
    for seed in (7, 1234, 99991):
        logits = (rng.standard_normal((B, V)) * 3).astype(np.float32)
        bl, bo = ctx.upload(logits), ctx.alloc(B * 4)
        ctx.sample(bl, bo, V, B, T, top_k, top_p, seed)
        got = ctx.download(bo, (B,), np.int32)
        ctx.free(bl)
        ctx.free(bo)
        u = draw(seed)
        for b in range(B):
            want = L.nxo_sample(np.ascontiguousarray(logits[b]), V, T, top_k, top_p, u)
            w64, margin, kept = ref64(logits[b], T, top_k, top_p, u, with_kept=True)
            if margin > tol_gpu(kept):
                assert got[b] == w64, (seed, b, got[b], w64, margin)
                checked += 1
            if margin > tol_fp32_sequential(V, kept):
                assert got[b] == want, (seed, b, got[b], want, margin)
                checked_o += 1
    # seeded inputs: each case checks a fixed number of its 48 rows against
    # float64 (24 to 48) and against the oracle (6 to 48)
    print(f"GPU == float64 on {checked} of {3 * B} rows, GPU == oracle on {checked_o}")
    assert checked >= 20 and checked_o >= 5


@pytest.mark.gpu
def test_gpu_sampler_wide_top_k_uses_radix_selection(ctx):
    """Flat logits (every entry within exp(-1) of the maximum, 32000 of them):
    no candidate threshold fits the LDS buffer, so the radix selection over
    all probabilities finds the top k; tokens equal the oracle's."""
    V, B = 32000, 8
    rng = np.random.default_rng(5)
    logits = (rng.random((B, V)) * 0.5).astype(np.float32)
    bl, bo = ctx.upload(logits), ctx.alloc(B * 4)
    for k, tp in ((40, 0.9), (1024, 1.0), (3, 0.5), (0, 0.9), (20000, 0.5), (5000, 1.0)):
        ctx.sample(bl, bo, V, B, 0.9, k, tp, 77)
        got = ctx.download(bo, (B,), np.int32)
        u = draw(77)
        for b in range(B):
            want = L.nxo_sample(np.ascontiguousarray(logits[b]), V, 0.9, k, tp, u)
            w64, margin, kept = ref64(logits[b], 0.9, k, tp, u, with_kept=True)
            if margin > tol_gpu(kept):
                assert got[b] == w64, (k, tp, b, got[b], w64)
            if margin > tol_fp32_sequential(V, kept):
                assert got[b] == want, (k, tp, b, got[b], want)
    ctx.free(bl)
    ctx.free(bo)


@pytest.mark.gpu
def test_gpu_sampler_ties_and_edges(ctx):
    """Equal logits (ties at the k-th value keep the lowest indices), a
    one-hot row, and greedy through nx_sample."""
    V = 2048
    logits = np.zeros((3, V), np.float32)
    logits[1, 777] = 50.0
    logits[2] = np.random.default_rng(1).standard_normal(V).astype(np.float32)
    bl, bo = ctx.upload(logits), ctx.alloc(12)
    ctx.sample(bl, bo, V, 3, 1.0, 5, 1.0, 3)
    got = ctx.download(bo, (3,), np.int32)
    u = draw(3)
    for b in range(3):
        assert got[b] == L.nxo_sample(np.ascontiguousarray(logits[b]), V, 1.0, 5, 1.0, u)
    assert got[0] < 5 and got[1] == 777
    ctx.sample(bl, bo, V, 3, 0.0, 5, 1.0, 3)
    assert ctx.download(bo, (3,), np.int32)[2] == int(np.argmax(logits[2]))
    # all equal: top-p 0.5 keeps the 1025 lowest indices (the running sum
    # first exceeds 0.5 at the 1025th), top-k 1500 the 1500 lowest
    for k, tp, keep in ((0, 0.5, 1025), (1500, 1.0, 1500), (1500, 0.25, 513)):
        for seed in (3, 11, 12345):
            ctx.sample(bl, bo, V, 1, 1.0, k, tp, seed)
            got0 = int(ctx.download(bo, (3,), np.int32)[0])
            want0 = L.nxo_sample(np.ascontiguousarray(logits[0]), V, 1.0, k, tp, draw(seed))
            assert got0 == want0 and got0 < keep, (k, tp, seed, got0, want0)
    ctx.free(bl)
    ctx.free(bo)


@pytest.mark.gpu
def test_sampled_decode_matches_oracle(ctx):
    """The tiny model decoding with temperature 0.8, top-k 40, top-p 0.9 and a
    fixed seed (the same draw every step, as in the reference): each step's
    token is the oracle sampler's on the oracle model's logits, until a step
    whose decision lies within 1e-4 of a boundary."""
    from test_gpu_model import TINY
    cfg = dict(TINY, seed=0x5A)
    T, K, Pp, seed = 0.8, 40, 0.9, 424242
    u = draw(seed)
    prompt = oracle.prompt_tokens(cfg["seed"], 1, 8, cfg["vocab"])
    om = oracle.Model(**cfg)
    for i in range(prompt.shape[1]):
        lg = om.forward(np.ascontiguousarray(prompt[:, i]))
    want, margins = [], []
    for _ in range(16):
        tok = L.nxo_sample(np.ascontiguousarray(lg[0]), cfg["vocab"], T, K, Pp, u)
        want.append(tok)
        margins.append(ref64(lg[0], T, K, Pp, u)[1])
        lg = om.forward(np.array([tok], np.int32))
    om.close()
    m = nexus_amd.Model(ctx, **cfg)
    m.set_sampling(T, K, Pp, seed)
    first = m.prefill(prompt)
    got = np.concatenate([first, m.decode(15)[0]])
    m.close()
    for i in range(16):
        if margins[i] < 1e-4:
            break
        assert got[i] == want[i], (i, got[:i + 1], want[:i + 1])


@pytest.mark.gpu
@pytest.mark.parametrize("K,Pp", [(0, 0.9), (2000, 0.95)])
def test_sampled_decode_wide_modes_match_oracle(ctx, K, Pp):
    """Sampling inside the decode graph with pure nucleus sampling and with
    top-k above 1024: each step's token is the oracle sampler's on the oracle
    model's logits, until a step within 1e-4 of a boundary."""
    from test_gpu_model import TINY
    cfg = dict(TINY, seed=0x5B)
    T, seed = 0.9, 31337
    u = draw(seed)
    prompt = oracle.prompt_tokens(cfg["seed"], 1, 8, cfg["vocab"])
    om = oracle.Model(**cfg)
    for i in range(prompt.shape[1]):
        lg = om.forward(np.ascontiguousarray(prompt[:, i]))
    want, margins = [], []
    for _ in range(12):
        tok = L.nxo_sample(np.ascontiguousarray(lg[0]), cfg["vocab"], T, K, Pp, u)
        want.append(tok)
        margins.append(ref64(lg[0], T, K, Pp, u)[1])
        lg = om.forward(np.array([tok], np.int32))
    om.close()
    m = nexus_amd.Model(ctx, **cfg)
    m.set_sampling(T, K, Pp, seed)
    first = m.prefill(prompt)
    got = np.concatenate([first, m.decode(11)[0]])
    m.close()
    for i in range(12):
        if margins[i] < 1e-4:
            break
        assert got[i] == want[i], (i, got[:i + 1], want[:i + 1])
