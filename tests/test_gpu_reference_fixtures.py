"""The HIP kernels' kept sets and greedy tokens against fixtures written by the
reference's own sampler (tests/golden/make_reference_filter.py), on whole batches:
all five BASELINE configurations at full size (C4's 1024 rows included) and the
tie, plain-sampling and min-p batches of tests/golden/kept_summary.py.

The rules are those of tests/test_reference_fixtures.py (the oracle against the
same fixtures), and the per-batch counts of differing rows must be the same, since
the kernels equal the oracle bit for bit."""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

import oracle as O
from fie_amd import workloads as W
from fie_amd.batching.sampler import resolve_params
from fie_amd.kernel import FusedSampler
from fie_amd.runtime.sampling import SamplingParams

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)
import kept_summary as KS  # noqa: E402


@pytest.fixture(scope="module")
def fs():
    return FusedSampler(DEV)


@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C4", "C5", "Q3ties", "Q2plain", "minp"])
def test_kernel_kept_sets_against_the_reference(fs, name):
    if name.startswith("C"):
        w = W.make(int(name[1]))
        x, params, ctx, uni = w.logits, w.params, w.contexts, w.uniforms
    else:
        x, params, ctx = KS.EXTRA[name](SamplingParams)
        uni = np.zeros(x.shape[0])
    B, V = x.shape
    print(f"  case: {name} rows={B} vocab={V} dtype={x.dtype}", flush=True)
    out, args, _ = fs.step(x.to(DEV), resolve_params(params, V, uni, ctx))
    kept, _ = fs.kept(args, want_probs=False)
    torch.cuda.synchronize()
    kept = kept.cpu().numpy()
    res = O.resolve(params, V)
    pen = x.float().numpy()
    if ctx is not None and res.has_pen.any():
        pen = O.canonical_penalize(pen, res, ctx)
    working = (pen / res.scale[:, None] + np.float32(0)).astype(np.float32)
    want = KS.load_fixture(name, HERE)
    n_set, n_ties, drift = KS.check_against_reference(want, kept, working, out["tk_key"],
                                                      res.top_p, out["tokens"], res.min_p)
    print(f"  {name}: {n_set} rows cut by the reference's fp32 rounding (drift {drift:.2e}), "
          f"{n_ties} differing only in edge ties", flush=True)
    assert (n_set, n_ties) == KS.EXPECTED[name]
