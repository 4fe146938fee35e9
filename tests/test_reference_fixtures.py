"""The oracle's kept sets against fixtures written by the reference's own sampler.

tests/golden/make_reference_filter.py ran the reference's ``sampler.py`` (loaded by
path in the build container) over every BASELINE configuration and three extra
batches, and stored a compact description of each row's kept set
(tests/golden/kept_summary.py).  Here the canonical C oracle runs the same inputs.

What must hold (engine/batching/sampler.py:187-260):
* greedy tokens are equal;
* every other row's kept set is the reference's, except (a) which members of the
  edge value's tie class survive, which the reference leaves to an unstable sort
  (sampler.py:221), and (b) rows where the reference's fp32 softmax/cumsum moved the
  top-p cut: there the reference's set must be a prefix of the exact order, cut
  within DRIFT_TOL of top_p in exact fp64 mass;
* the number of rows of each kind is exactly what was measured (EXPECTED).
"""

from __future__ import annotations

import os

import numpy as np
import pytest

import oracle as O
from fie_amd import workloads as W
from fie_amd.runtime.sampling import SamplingParams

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
import sys  # noqa: E402

sys.path.insert(0, HERE)
import kept_summary as KS  # noqa: E402


def batch(name, rows=None):
    if name.startswith("C"):
        w = W.make(int(name[1]), rows=rows)
        return w.logits, w.params, w.contexts
    return KS.EXTRA[name](SamplingParams)


@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C4/8", "C5", "Q3ties", "Q2plain", "minp"])
def test_oracle_kept_sets_against_the_reference(name):
    base = name.split("/")[0]
    rows = list(range(0, 1024, 8)) if name == "C4/8" else None
    x, params, ctx = batch(base, rows)
    B, V = x.shape
    res = O.resolve(params, V)
    r = O.canonical_step(x.float().numpy(), res, np.zeros(B), contexts=ctx, want_kept=True)
    working = (r.penalized / res.scale[:, None] + np.float32(0)).astype(np.float32)
    want = KS.load_fixture(base, HERE)
    if rows is not None:
        want = {k: v[rows] for k, v in want.items()}
    n_set, n_ties, drift = KS.check_against_reference(want, r.kept, working, r.tk_key,
                                                      res.top_p, r.tokens, res.min_p)
    print(f"{name}: {B} rows, {n_set} cut by the reference's fp32 rounding "
          f"(largest drift {drift:.2e}), {n_ties} differing only in edge ties")
    assert (n_set, n_ties) == KS.EXPECTED[name]


def test_fixtures_cover_every_row():
    for name, rows in (("C1", 8), ("C2", 64), ("C3", 256), ("C4", 1024), ("C5", 128),
                       ("Q3ties", 48), ("Q2plain", 32), ("minp", 24)):
        f = KS.load_fixture(name, HERE)
        assert f["count"].shape == (rows,)
        assert (f["count"][f["sampled"]] > 0).all()
