import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "nexus-inference-engine-_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (runs on the MI355X box)")


@pytest.fixture(scope="session")
def ctx():
    """One nx_ctx for the whole GPU session (tests run in one process)."""
    import nexus_amd
    c = nexus_amd.Context(0)
    print(f"[gpu] device: {c.device_name()}", flush=True)
    yield c
    c.close()


def rel_err(got, ref) -> float:
    """max |got - ref| / max |ref| (the tolerance metric of the parity tests)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    denom = np.max(np.abs(ref))
    if denom == 0:
        return float(np.max(np.abs(got)))
    return float(np.max(np.abs(got - ref)) / denom)


def f16(bits: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(bits, np.uint16).view(np.float16).astype(np.float32)


# Largest oracle top1 - top2 logit margin at which the GPU may pick the other
# token: fp32 summation order and the fp16 rounding of GEMV inputs move the
# logits of these models by ~1e-5..1e-4, so steps with a smaller margin are
# numerical ties.
TIE_MARGIN = 1e-3

# TurboQuant pages (kv_kind 1, and the tiered pages before the fp16 window):
# attention over them is accurate to about 1e-3 (the value codebook enters
# the products as fp16), so logits of decodes over filled contexts, whose
# compressed pages come from identical inputs on both sides (their codes are
# checked bit-exact), agree to TQ_TOL (worst seen 1.2e-3) and greedy tokens
# are compared where the oracle's margin is at least TQ_TIE (twice the worst
# absolute logit error seen, 4.5e-3).
TQ_TOL = 2e-3
TQ_TIE = 1e-2
# Runs whose decode compresses its own positions (prompt-driven runs with
# TurboQuant pages or short fp16 windows): K and V of those positions come
# from GPU and oracle fp32 sums in different orders, so their fp16 values can
# differ in the last bit and a code can land one level apart; such flips add
# up over the run (worst seen 1.0e-2 relative, 1.7e-2 absolute after 100
# steps with a 16-position window).  Misplaced positions or wrong vectors
# move the logits by O(1).
TQ_DECODE_TOL = 2e-2
TQ_DECODE_TIE = 4e-2


def forced_logits(gm, om, start, steps):
    """Teacher forcing: the GPU model gm and the oracle om, in the same state,
    both consume the oracle's greedy tokens for `steps` steps (start first,
    [batch]); returns the GPU and oracle logits [batch][steps][vocab]."""
    tok = np.asarray(start, np.int32)
    fed, olog = [], []
    for _ in range(steps):
        fed.append(tok)
        lg = om.forward(tok)
        olog.append(lg)
        tok = lg.argmax(axis=1).astype(np.int32)
    glog = gm.decode_forced(np.stack(fed, 1))
    return glog, np.stack(olog, 1)


def check_forced(glog, olog, tol, tie, label=""):
    """Every step of every sequence: logits within `tol` (rel_err), and the
    GPU's greedy token equal to the oracle's wherever the oracle's top-two
    margin is at least `tie` (a smaller margin is a numerical tie).  Prints
    the worst relative and absolute logit errors and the smallest margin at
    which the tokens differed."""
    B, S, _ = olog.shape
    worst = worst_abs = 0.0
    checked = 0
    flip = None
    for b in range(B):
        for s in range(S):
            g, o = glog[b, s], olog[b, s]
            e = rel_err(g, o)
            worst = max(worst, e)
            worst_abs = max(worst_abs, float(np.max(np.abs(g.astype(np.float64) - o))))
            assert e < tol, f"{label}: sequence {b} step {s}: logits rel err {e:.3g} >= {tol}"
            top = np.sort(o)[-2:]
            margin = float(top[1] - top[0])
            if int(g.argmax()) != int(o.argmax()):
                flip = margin if flip is None else min(flip, margin)
            if margin >= tie:
                checked += 1
                assert int(g.argmax()) == int(o.argmax()), (
                    f"{label}: sequence {b} step {s}: token {int(g.argmax())} vs {int(o.argmax())} at margin {margin:.3g}")
    print(f"[forced] {label}: {B} x {S} steps, logits rel err <= {worst:.3g} (abs {worst_abs:.3g}), "
          f"tokens equal at {checked} steps with margin >= {tie:g}"
          + (f", a tie flipped at margin {flip:.3g}" if flip is not None else ""), flush=True)
    return worst
