"""Compact descriptions of top-k/top-p/min-p kept sets, and the extra fixture cases.

A kept set over a [rows, vocab] batch is described per row by:

  count        how many tokens survive
  edge_bits    fp32 bits of the smallest surviving working value (the filter edge)
  above_count  survivors whose working value is strictly above the edge
  above_hash   order-independent hash (sum of splitmix64 of token ids, mod 2^64) of
               those survivors
  kept_hash    the same hash over every survivor, edge ties included

The reference sorts with an unstable sort (engine/batching/sampler.py:221), so which
members of the edge value's tie class survive a top-p cut is an artefact of the sort
implementation; how many survive is not (equal values have equal fp32 probabilities,
so every prefix sum is the same whatever their order).  ``count``, ``edge_bits``,
``above_count`` and ``above_hash`` pin everything else bit for bit; ``kept_hash``
tells the tie order apart for reporting.

Used by make_reference_filter.py (which writes the fixtures in the build container)
and by the tests that read them; it imports nothing from the reference.
"""

from __future__ import annotations

import numpy as np
import torch

MASK64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def splitmix64(x: np.ndarray) -> np.ndarray:
    """SplitMix64's output function (Steele, Lea, Flood, OOPSLA 2014) on uint64."""
    with np.errstate(over="ignore"):
        z = np.asarray(x, dtype=np.uint64) + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def summarize(kept: np.ndarray, working: np.ndarray) -> dict[str, np.ndarray]:
    """Describe the kept sets ``kept`` [rows, vocab] (bool) over fp32 ``working``."""
    kept = np.asarray(kept).astype(bool)
    working = np.asarray(working, dtype=np.float32)
    rows, vocab = kept.shape
    h = splitmix64(np.arange(vocab, dtype=np.uint64))
    out = {k: np.zeros(rows, dt) for k, dt in (
        ("count", np.int64), ("edge_bits", np.uint32), ("above_count", np.int64),
        ("above_hash", np.uint64), ("kept_hash", np.uint64))}
    with np.errstate(over="ignore"):
        for r in range(rows):
            k = kept[r]
            n = int(k.sum())
            out["count"][r] = n
            if n == 0:
                continue
            y = working[r]
            edge = np.float32(y[k].min())
            above = k & (y > edge)
            out["edge_bits"][r] = edge.view(np.uint32)
            out["above_count"][r] = int(above.sum())
            out["above_hash"][r] = h[above].sum(dtype=np.uint64)
            out["kept_hash"][r] = h[k].sum(dtype=np.uint64)
    return out


def compare(want: dict, got: dict, rows=None) -> dict[str, list[int]]:
    """Rows (among ``rows``) by how ``got`` differs from ``want``:
    'set'  count, edge, or the survivors above the edge differ;
    'ties' identical except which members of the edge tie class survive."""
    rows = range(len(want["count"])) if rows is None else rows
    res = {"set": [], "ties": []}
    for r in rows:
        same = all(int(want[k][r]) == int(got[k][r])
                   for k in ("count", "edge_bits", "above_count", "above_hash"))
        if not same:
            res["set"].append(int(r))
        elif int(want["kept_hash"][r]) != int(got["kept_hash"][r]):
            res["ties"].append(int(r))
    return res


# ----------------------------------------------------------------- extra cases
def tie_case(params_cls):
    """Q3: 48 rows over V=6000 whose logits sit on a 1/8 grid, so every top-p cut falls
    inside a tie class of tens to hundreds of tokens.  Top-p in {0.5, 0.8, 0.9, 0.95},
    temperature 1.0 (16 rows) and 0.5 (16 rows); 16 more rows add top-k 700."""
    gen = torch.Generator().manual_seed(20261291)
    rows, vocab = 48, 6000
    x = torch.round(torch.randn(rows, vocab, generator=gen) * 8.0) / 8.0
    params = []
    for i in range(rows):
        p = (0.5, 0.8, 0.9, 0.95)[i % 4]
        t = 1.0 if i < 16 else 0.5
        k = 700 if i >= 32 else 0
        params.append(params_cls(temperature=t, top_p=p, top_k=k))
    return x.float(), params, None


def q2_case(params_cls):
    """Q2: 32 rows of peaked logits (the C2 shape at V=151936).  Even rows top-p 0.9 at
    temperature 0.7; odd rows plain sampling at 0.7 (top_p = 1, no top-k), which the
    reference still runs through its `cumulative - probs >= 1.0` test because other
    rows of the batch enable top-p."""
    gen = torch.Generator().manual_seed(20261292)
    rows, vocab = 32, 151936
    ranks = torch.argsort(torch.rand(rows, vocab, generator=gen), dim=1)
    x = -1.1 * torch.log(ranks.float() + 1.0) + 0.5 * torch.randn(rows, vocab, generator=gen)
    params = [params_cls(temperature=0.7, top_p=0.9 if i % 2 == 0 else 1.0)
              for i in range(rows)]
    return x.float(), params, None


def minp_case(params_cls):
    """min-p together with top-k and top-p (the reference's filter order,
    sampler.py:194-228), 24 rows of C1-like N(0, 3^2) logits at V=50000."""
    gen = torch.Generator().manual_seed(20261293)
    rows, vocab = 24, 50000
    x = 3.0 * torch.randn(rows, vocab, generator=gen)
    params = [params_cls(temperature=(0.8, 1.0, 1.5)[i % 3], min_p=(0.01, 0.05, 0.2)[i % 3],
                         top_k=(0, 500)[(i // 3) % 2], top_p=(1.0, 0.9)[(i // 6) % 2])
              for i in range(rows)]
    return x.float(), params, None


EXTRA = {"Q3ties": tie_case, "Q2plain": q2_case, "minp": minp_case}


def explain(want: dict, r: int, y: np.ndarray, survivors: np.ndarray, limit: float,
            got_count: int) -> float:
    """For a row whose kept set differs from the reference's (``compare`` 'set'), check
    that the reference kept a prefix of the exact order (value descending, index
    ascending) over the top-k/min-p ``survivors`` of working row ``y`` (edge ties
    aside), and return how far from ``limit`` the exact fp64 exclusive mass lies at
    every position between the reference's cut and ours: the size of the rounding
    that moved the reference's cut.  Raises AssertionError if the reference's set is
    not such a prefix."""
    y = np.asarray(y, dtype=np.float32)
    idx = np.nonzero(survivors)[0]
    order = idx[np.argsort(-y[idx].astype(np.float64), kind="stable")]
    n_ref = int(want["count"][r])
    assert 0 < n_ref <= order.size, (r, n_ref, order.size)
    prefix = order[:n_ref]
    edge = np.float32(y[prefix[-1]])
    above = prefix[y[prefix] > edge]
    h = splitmix64(above.astype(np.uint64)).sum(dtype=np.uint64) if above.size else np.uint64(0)
    assert int(edge.view(np.uint32)) == int(want["edge_bits"][r]), (r, "edge")
    assert above.size == int(want["above_count"][r]), (r, "above count")
    assert int(h) == int(want["above_hash"][r]), (r, "above set")
    z = y[order].astype(np.float64)
    p = np.exp(z - z.max())
    p /= p.sum()
    excl = np.cumsum(p) - p
    lo, hi = sorted((n_ref, int(got_count)))
    return float(np.abs(excl[lo:hi] - limit).max()) if hi > lo else 0.0


# How each batch's kept sets differ from the reference's (rows of compare()'s 'set'
# and 'ties' classes), measured with the reference's own sampler.py on the CPU.  The
# C4 figures are for its rows 0, 8, 16, ... (128 rows) when ``rows`` selects them.
DRIFT_TOL = 1e-4
EXPECTED = {"C1": (0, 0), "C2": (0, 0), "C3": (6, 1), "C4": (539, 482), "C4/8": (69, 59),
            "C5": (0, 31), "Q3ties": (0, 48), "Q2plain": (16, 0), "minp": (0, 0)}


def load_fixture(name: str, here: str) -> dict:
    import os

    with np.load(os.path.join(here, f"reference_kept_{name}.npz")) as f:
        return {k: f[k] for k in f.files}


def check_against_reference(want: dict, kept, working, tk_key, top_p, tokens,
                            min_p=None) -> tuple[int, int, float]:
    """Compare one batch's kept sets and greedy tokens with a reference fixture.

    Greedy tokens must be equal.  Every sampled row must either match exactly, or
    differ only in which edge ties survive, or be a row whose reference set is a
    prefix of the exact order cut within DRIFT_TOL of top_p (``explain``).  Returns
    (set rows, tie rows, largest drift)."""
    sampled = want["sampled"].astype(bool)
    g = ~sampled
    assert np.array_equal(np.asarray(tokens)[g], want["greedy_token"][g]), "greedy tokens"
    got = summarize(kept, working)
    c = compare(want, got, np.nonzero(sampled)[0])
    worst = 0.0
    for r in c["set"]:
        assert min_p is None or float(min_p[r]) == 0.0, (r, "min-p row differs")
        key = np.asarray(working[r], np.float32) + np.float32(0.0)
        b = key.view(np.uint32)
        fk = np.where(b & np.uint32(0x80000000), ~b, b | np.uint32(0x80000000)).astype(np.uint32)
        d = explain(want, r, working[r], fk >= np.uint32(tk_key[r]), float(top_p[r]),
                    int(got["count"][r]))
        assert d <= DRIFT_TOL, (r, d)
        worst = max(worst, d)
    return len(c["set"]), len(c["ties"]), worst
