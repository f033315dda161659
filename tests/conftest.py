import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def ctx():
    from common_amd import hardware as hw
    c = hw.HipContext(0)
    yield c
    c.close()


def argmax_decisions(gpu_logits, ref_logits, near_tie=1e-5):
    """Top-1 agreement of every step's logits (prompt steps included, whose inputs vary even when a
    random-weight model's greedy stream repeats one token): every row where the reference's relative
    top-1/top-2 margin is at least `near_tie` must have the same argmax.  Returns (rows compared,
    distinct reference argmaxes among them, smallest margin among them)."""
    g = np.asarray(gpu_logits, dtype=np.float64).reshape(-1, np.shape(ref_logits)[-1])
    r = np.asarray(ref_logits, dtype=np.float64).reshape(g.shape)
    top2 = np.sort(r, axis=1)[:, -2:]
    margin = (top2[:, 1] - top2[:, 0]) / np.maximum(np.abs(top2[:, 1]), 1e-30)
    keep = margin >= near_tie
    ga, ra = g.argmax(axis=1), r.argmax(axis=1)
    bad = np.nonzero(keep & (ga != ra))[0]
    assert bad.size == 0, f"argmax differs at rows {bad[:8].tolist()} (margins {margin[bad[:8]].tolist()})"
    return int(keep.sum()), len(set(ra[keep].tolist())), float(margin[keep].min()) if keep.any() else 0.0


def rel_err(got, ref):
    """max |got - ref| / max |ref| (the north-star tolerance measure)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))
