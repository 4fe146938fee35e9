"""Pins of the CPU oracle (oracle/canonical.c) -- CPU only, no GPU.

The oracle is what the HIP sampler is checked against bit for bit, so it is pinned
here by things other than its own formulas:

* the reference's own known-answer tests (tests/batching/test_sampler.py:23-184 of
  full-inference-engine), restated on the oracle with a grid of uniforms in place of
  the reference's torch.multinomial stream;
* an independent exact-integer restatement of the canonical rules in Python for tiny
  vocabularies, over random parameters, penalties and ties;
* mathematics: the kept sets against a brute-force sort, the top-p cut against the
  textbook fp64 nucleus, probabilities and logprobs against fp64 softmax, the draw
  against its inverse-CDF frequencies, the canonical exponential against math.exp;
* the torch restatement of the reference (oracle.torch_reference_step, which runs the
  reference's own op sequence on CPU tensors): penalties bit for bit, and top-k /
  top-p / min-p kept sets equal except inside a stated fp32 ambiguity margin.
"""

from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest
import torch

import oracle as O
from fie_amd import workloads as W
from fie_amd.runtime.sampling import GREEDY, SamplingParams

TILE = 2048


# Absolute floor of probability comparisons: rule R1's weight quantisation.
PROB_ATOL = 2.0 ** -40

def step(logits, params, uniforms=None, contexts=None, **kw):
    x = np.asarray(logits, dtype=np.float32)
    if x.ndim == 1:
        x = x[None, :]
    B, V = x.shape
    u = np.zeros(B) if uniforms is None else np.asarray(uniforms, dtype=np.float64)
    return O.canonical_step(x, O.resolve(params, V), u, contexts=contexts, **kw)


def drawn_set(logits, p, n=400):
    """Tokens drawn over a grid of n uniforms (the reference draws 200-300 times)."""
    x = np.asarray(logits, dtype=np.float32)[None, :]
    grid = (np.arange(n) + 0.5) / n
    r = step(np.repeat(x, n, axis=0), [p] * n, grid)
    return set(int(t) for t in r.tokens)


# ------------------------------------------------------------------ reference KATs
def _randn(rows, vocab, seed=0):
    return torch.randn(rows, vocab, generator=torch.Generator().manual_seed(seed)).numpy()


def test_kat_all_greedy_batch_is_exactly_argmax():            # test_sampler.py:23-27
    x = _randn(4, 50)
    assert step(x, [GREEDY] * 4).tokens.tolist() == x.argmax(axis=1).tolist()


def test_kat_zero_temperature_is_greedy_whatever_else_is_set():   # :30-34
    x = _randn(2, 32)
    p = [SamplingParams(temperature=0.0, top_p=0.1, top_k=3, seed=5)] * 2
    assert step(x, p, [0.3, 0.9]).tokens.tolist() == x.argmax(axis=1).tolist()


def test_kat_top_k_one_is_greedy():                              # :37-40
    x = _randn(3, 40)
    p = [SamplingParams(temperature=1.0, top_k=1)] * 3
    assert step(x, p, [0.1, 0.5, 0.9]).tokens.tolist() == x.argmax(axis=1).tolist()


def test_kat_top_k_restricts_choices_to_the_k_best():           # :43-50
    x = _randn(1, 100)[0]
    allowed = set(np.argsort(-x)[:5].tolist())
    drawn = drawn_set(x, SamplingParams(temperature=1.5, top_k=5))
    assert drawn <= allowed and len(drawn) > 1


def test_kat_top_p_keeps_the_smallest_prefix_reaching_the_mass():  # :53-60
    x = np.log(np.array([0.5, 0.25, 0.15, 0.10], dtype=np.float32))
    assert drawn_set(x, SamplingParams(temperature=1.0, top_p=0.7)) == {0, 1}


def test_kat_top_p_always_keeps_the_most_likely_token():         # :63-67
    x = np.log(np.array([0.9, 0.05, 0.05], dtype=np.float32))
    assert drawn_set(x, SamplingParams(temperature=1.0, top_p=0.3)) == {0}


def test_kat_min_p_drops_tokens_far_below_the_mode():             # :70-75
    x = np.log(np.array([0.6, 0.3, 0.09, 0.01], dtype=np.float32))
    assert drawn_set(x, SamplingParams(temperature=1.0, min_p=0.2)) == {0, 1}


def test_kat_mixed_batch_greedy_rows_are_unaffected():            # :88-94
    x = _randn(4, 80, seed=11)
    p = [GREEDY, SamplingParams(temperature=1.2, top_p=0.9), GREEDY,
         SamplingParams(temperature=0.8, top_k=10, seed=99)]
    t = step(x, p, [0.2, 0.4, 0.6, 0.8]).tokens
    assert t[0] == x[0].argmax() and t[2] == x[2].argmax()


def test_kat_repetition_penalty_pushes_seen_tokens_down():        # :97-103
    x = np.array([[2.0, 1.9, 0.0]], dtype=np.float32)
    assert step(x, [GREEDY], contexts=[[0]]).tokens.tolist() == [0]
    assert step(x, [SamplingParams(repetition_penalty=1.5)], contexts=[[0]]).tokens.tolist() == [1]


def test_kat_repetition_penalty_moves_negative_logits_down_too():  # :106-110
    x = np.array([[-1.0, -1.1]], dtype=np.float32)
    assert step(x, [SamplingParams(repetition_penalty=2.0)], contexts=[[0]]).tokens.tolist() == [1]


def test_kat_frequency_penalty_scales_with_occurrences():           # :113-118
    x = np.array([[3.0, 2.0, 1.0]], dtype=np.float32)
    p = [SamplingParams(frequency_penalty=0.6)]
    assert step(x, p, contexts=[[0]]).tokens.tolist() == [0]
    assert step(x, p, contexts=[[0, 0]]).tokens.tolist() == [1]


def test_kat_presence_penalty_applies_once_per_token():            # :121-125
    x = np.array([[3.0, 2.5, 1.0]], dtype=np.float32)
    p = [SamplingParams(presence_penalty=0.75)]
    assert step(x, p, contexts=[[0, 0, 0]]).tokens.tolist() == [1]


def test_kat_penalties_are_per_row():                               # :128-132
    x = np.array([[2.0, 1.9, 0.0], [2.0, 1.9, 0.0]], dtype=np.float32)
    p = [SamplingParams(repetition_penalty=1.5), GREEDY]
    assert step(x, p, contexts=[[0], [0]]).tokens.tolist() == [1, 0]


def test_kat_logprobs_report_chosen_token_first():                  # :135-142
    x = np.log(np.array([0.7, 0.2, 0.1], dtype=np.float32))
    r = step(x, [SamplingParams(logprobs=2)])
    assert r.tokens[0] == 0
    assert math.isclose(float(r.chosen_lp[0]), math.log(0.7), abs_tol=1e-5)
    assert r.top_ids[0, :2].tolist() == [0, 1]
    assert (r.top_lp[0, :2] <= 0).all()


def test_kat_logprobs_follow_temperature():                          # :145-152
    x = np.log(np.array([0.7, 0.2, 0.1], dtype=np.float32))
    hot = float(step(x, [SamplingParams(temperature=2.0, logprobs=1, seed=3)], [0.0]).chosen_lp[0])
    cold = float(step(x, [SamplingParams(logprobs=1)]).chosen_lp[0])
    assert hot > math.log(0.7) - 1e-6 or hot < cold


# ------------------------------------------------------------------ exact restatement
def _key(v: np.float32) -> int:
    b = int(np.float32(v).view(np.uint32))
    return (~b & 0xFFFFFFFF) if b & 0x80000000 else (b | 0x80000000)


def _fixed40(e: np.float32) -> int:
    return math.floor(Fraction(float(e)) * (1 << 40))


def _tile(i: int) -> int:
    return 0 if i == 0 else 1 + i // TILE


def exact_row(y: np.ndarray, k: int, p: float, mp: float, u: float):
    """Rules R1-R5 in Python integers for one row of scaled logits y (fp32).
    Returns (token, kept mask, kept mass)."""
    V = y.shape[0]
    tiles = {}
    for i in range(V):
        t = _tile(i)
        tiles[t] = max(tiles.get(t, 0), _key(y[i]))
    kf = lambda kk: np.uint32(kk & 0x7FFFFFFF if kk & 0x80000000 else ~kk & 0xFFFFFFFF).view(np.float32)
    mt = {t: kf(kk) for t, kk in tiles.items()}
    M = max(mt.values(), key=_key)
    C = {t: _fixed40(O.cexp(np.float32(mt[t] - M))) for t in mt}
    w = [_fixed40(O.cexp(np.float32(y[i] - mt[_tile(i)]))) * C[_tile(i)] for i in range(V)]
    order = sorted(range(V), key=lambda i: (-_key(y[i]), i))
    surv = [True] * V
    if k > 0:
        tk = _key(y[order[k - 1]])
        surv = [_key(y[i]) >= tk for i in range(V)]
    if mp > 0:
        L = O.minp_bound(mp)
        surv = [s and not (np.float32(y[i] - M) < L) for i, s in enumerate(surv)]
    S = sum(w[i] for i in range(V) if surv[i])
    if p < 1.0:
        thr = math.ceil(Fraction(float(np.float32(p))) * S)
        excl, stop = 0, False
        for i in order:
            if not surv[i]:
                continue
            if stop or excl >= thr:
                stop = True
                surv[i] = False
                continue
            excl += w[i]
    T = sum(w[i] for i in range(V) if surv[i])
    t = math.floor(Fraction(u) * T)
    incl = 0
    tok = order[0]
    for i in order:
        if surv[i]:
            incl += w[i]
            if incl > t:
                tok = i
                break
    return tok, np.array(surv, dtype=np.uint8), T


@pytest.mark.parametrize("seed", range(12))
def test_oracle_matches_exact_integer_restatement(seed):
    rng = np.random.default_rng(seed)
    V = int(rng.integers(2, 13))
    B = 4
    x = rng.normal(0, 2, (B, V)).astype(np.float32)
    if seed % 3 == 0:
        x = np.round(x)                     # ties
    params = []
    for r in range(B):
        params.append(SamplingParams(temperature=float(rng.choice([0.5, 1.0, 1.7])),
                                     top_k=int(rng.integers(0, V + 2)),
                                     top_p=float(rng.choice([1.0, 0.3, 0.8, 0.95])),
                                     min_p=float(rng.choice([0.0, 0.0, 0.1, 0.5]))))
    params[0] = SamplingParams(temperature=1.0, top_k=2) if V > 2 else params[0]
    u = rng.random(B)
    res = step(x, params, u, want_kept=True)
    rs = O.resolve(params, V)
    for r in range(B):
        if rs.greedy[r]:
            assert res.tokens[r] == int(np.argmax(x[r]))
            continue
        y = (x[r] / rs.scale[r]).astype(np.float32) + np.float32(0)
        tok, kept, T = exact_row(y, int(rs.top_k[r]), float(rs.top_p[r]), float(rs.min_p[r]), float(u[r]))
        assert res.tokens[r] == tok
        np.testing.assert_array_equal(res.kept[r], kept)
        assert int(res.kept_mass[r, 0]) | (int(res.kept_mass[r, 1]) << 64) == T


# ------------------------------------------------------------------ mathematics
def test_cexp_within_two_ulp_of_exp():
    d = np.concatenate([-np.logspace(-8, math.log10(79.9), 20000), [-0.0, 0.0, -1e-30]]).astype(np.float32)
    got = O.cexp(d).astype(np.float64)
    ref = np.exp(d.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(got - ref) / ulp) <= 2.0


def test_cexp_special_values():
    got = O.cexp(np.array([0.0, -0.0, 5.0, -80.0, -80.5, -np.inf, np.nan], dtype=np.float32))
    assert got[:3].tolist() == [1.0, 1.0, 1.0] and got[3:].tolist() == [0.0, 0.0, 0.0, 0.0]


def test_minp_bound_brackets_the_exponential():
    for mp in (1e-6, 0.01, 0.05, 0.2, 0.5, 0.99, 1.0):
        L = O.minp_bound(mp)
        assert O.cexp(np.array([L], np.float32))[0] >= np.float32(mp)
        assert abs(L - math.log(mp)) <= 1e-6 * max(1.0, abs(math.log(mp)))


@pytest.mark.parametrize("s", [0.7, 1.3, 1.999999, 0.05, float(np.float32(np.nextafter(np.float32(2), np.float32(0))))])
def test_markstein_divide_equals_ieee_divide(s):
    # every fp16 and bf16 value and 200k random fp32 values in the guarded range
    assert O.markstein_mismatches(s, 200_000, 7) == 0


def test_top_k_set_is_the_k_best_values_with_ties():
    rng = np.random.default_rng(3)
    x = np.round(rng.normal(0, 2, (6, 500))).astype(np.float32)   # heavy ties
    ks = [1, 3, 10, 50, 499, 7]
    p = [SamplingParams(temperature=1.0, top_k=k) for k in ks]
    r = step(x, p, rng.random(6), want_kept=True)
    for i, k in enumerate(ks):
        if k == 1:
            continue
        kth = np.sort(x[i])[::-1][k - 1]
        np.testing.assert_array_equal(r.kept[i], (x[i] >= kth).astype(np.uint8))


def _nucleus64(y, p):
    """Textbook nucleus in fp64: stable descending order, drop where the exclusive
    cumulative probability reaches p.  Also returns the ambiguity of the boundary."""
    e = np.exp(y.astype(np.float64) - y.max())
    prob = e / e.sum()
    order = np.argsort(-y, kind="stable")
    excl = np.concatenate([[0.0], np.cumsum(prob[order])[:-1]])
    keep = np.zeros(y.shape[0], dtype=np.uint8)
    keep[order[excl < p]] = 1
    margin = np.min(np.abs(excl - p))
    return keep, margin


def test_top_p_set_is_the_fp64_nucleus():
    rng = np.random.default_rng(4)
    x = rng.normal(0, 1.5, (24, 3000)).astype(np.float32)
    ps = [0.1, 0.5, 0.9, 0.95, 0.99, 0.999] * 4
    params = [SamplingParams(temperature=1.0, top_p=q) for q in ps]
    r = step(x, params, rng.random(24), want_kept=True)
    checked = 0
    for i, q in enumerate(ps):
        keep, margin = _nucleus64(x[i], float(np.float32(q)))
        if margin < 1e-6:
            continue
        checked += 1
        np.testing.assert_array_equal(r.kept[i], keep)
    assert checked >= 20


def test_probabilities_and_logprobs_match_fp64_softmax():
    rng = np.random.default_rng(5)
    x = rng.normal(0, 3, (6, 2000)).astype(np.float32)
    params = [SamplingParams(temperature=t, top_k=k, logprobs=5)
              for t, k in ((1.0, 0), (0.7, 100), (1.3, 500), (0.5, 0), (1.9, 20), (1.0, 1000))]
    r = step(x, params, rng.random(6), want_kept=True)
    rs = O.resolve(params, 2000)
    for i in range(6):
        y = (x[i] / rs.scale[i]).astype(np.float64)
        kept = r.kept[i].astype(bool)
        e = np.exp(y - y.max()) * kept
        want = e / e.sum()
        # 1e-5 relative, with an absolute floor of 2^-40: a probability is
        # W_i C_t / T with W_i = floor(cexp(.) 2^40), so the floor moves it by less
        # than C_t / T <= 2^-40 (rule R1's quantisation, not a precision loss of
        # the larger probabilities)
        np.testing.assert_allclose(r.probs[i][kept], want[kept], rtol=1e-5, atol=PROB_ATOL)
        lsm = y - y.max() - math.log(np.exp(y - y.max()).sum())
        assert abs(float(r.chosen_lp[i]) - lsm[r.tokens[i]]) <= 1e-5 * max(1, abs(lsm[r.tokens[i]]))
        np.testing.assert_allclose(r.top_lp[i, :5], lsm[r.top_ids[i, :5]], rtol=1e-5, atol=1e-6)


def test_draw_frequencies_follow_the_kept_distribution():
    x = np.log(np.array([0.4, 0.3, 0.2, 0.05, 0.05], dtype=np.float32))
    n = 20000
    grid = (np.arange(n) + 0.5) / n
    r = step(np.repeat(x[None], n, axis=0), [SamplingParams(temperature=1.0)] * n, grid)
    freq = np.bincount(r.tokens, minlength=5) / n
    np.testing.assert_allclose(freq, [0.4, 0.3, 0.2, 0.05, 0.05], atol=2.0 / n + 1e-6)


def test_argmax_ties_take_the_first_index():
    x = np.zeros((3, 5000), dtype=np.float32)
    x[0, [7, 4000]] = 3.0
    x[1, 4999] = 1.0
    x[2] = -np.inf
    x[2, 2500] = -1.0
    r = step(x, [GREEDY] * 3)
    assert r.tokens.tolist() == [7, 4999, 2500]


# ------------------------------------------------------------------ vs the torch restatement
def test_penalties_bit_exact_with_the_reference_op_sequence():
    """canonical_penalize vs the reference's gather/where/scatter on CPU tensors (Q1
    included): C3 and C5 rows, plus invalid ids before and after token 0."""
    for cfg, rows in ((3, list(range(0, 256, 16))), (5, list(range(0, 128, 16)))):
        w = W.make(cfg, rows=rows)
        got = O.canonical_penalize(w.logits.float().numpy(), O.resolve(w.params, w.logits.shape[1]),
                                   w.contexts)
        want = O._torch_penalties(w.logits.float(), w.params, w.contexts).numpy()
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    V = 50
    x = torch.linspace(-3, 3, 4 * V).reshape(4, V)
    p = [SamplingParams(repetition_penalty=1.7, frequency_penalty=0.3)] * 4
    ctx = [[0, 3, 3, V + 2], [V + 2, 0, 3], [0], [5, 6, 7, 0]]
    got = O.canonical_penalize(x.numpy(), O.resolve(p, V), ctx)
    want = O._torch_penalties(x, p, ctx).numpy()
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("config", [1, 2, 3, 4, 5])
def test_kept_sets_match_the_reference_op_sequence(config):
    """Kept sets of the canonical rules vs the reference's own fp32 filter (torch
    CPU, sampler.py:187-229), on 8 rows of each configuration.  Every token where
    the two disagree must sit at the top-p boundary, and the disagreement must be
    a rounding of one side: either the reference's fp32 exclusive cumulative
    (softmax then cumsum over the sorted row, as sampler.py:221-226 computes it)
    and the exact fp64 one fall on opposite sides of top_p, or the exact value is
    within 2e-6 of top_p (the canonical integer weights' own rounding)."""
    B = {1: 8, 2: 64, 3: 256, 4: 1024, 5: 128}[config]
    rows = list(range(0, B, max(1, B // 8)))[:8]
    w = W.make(config, rows=rows)
    V = w.logits.shape[1]
    ref = O.canonical_step(w.logits.float().numpy(), O.resolve(w.params, V), w.uniforms,
                           contexts=w.contexts, want_kept=True)
    _, filtered, working = O.torch_reference_step(w.logits, w.params, w.contexts, w.uniforms)
    kept_ref = torch.isfinite(filtered).numpy().astype(np.uint8)
    ambiguous = by_reference = 0
    for i, p in enumerate(w.params):
        if p.greedy:
            continue
        diff = np.nonzero(kept_ref[i] != ref.kept[i])[0]
        if diff.size == 0:
            continue
        limit = float(np.float32(p.top_p))
        y = working[i].numpy()
        surv = O.fkey(y) >= ref.tk_key[i]
        pre = torch.from_numpy(np.where(surv, y, -np.inf).astype(np.float32))
        # exact: fp64 over the stable order; the reference: its fp32 op sequence
        prob = torch.softmax(pre.double(), 0).numpy()
        order = np.argsort(-y, kind="stable")
        excl = np.concatenate([[0.0], np.cumsum(prob[order])[:-1]])
        pos = {int(t): j for j, t in enumerate(order)}
        ordered, rorder = pre.sort(descending=True)
        sm = ordered.softmax(0)
        excl32 = (sm.cumsum(0) - sm).numpy()
        rpos = {int(t): j for j, t in enumerate(rorder.numpy())}
        for t in diff:
            e64 = excl[pos[int(t)]]
            e32 = float(excl32[rpos[int(t)]])
            flipped = (e64 >= limit) != (e32 >= limit)
            assert flipped or abs(e64 - limit) < 2e-6, (i, int(t), e64, e32)
            by_reference += int(flipped)
        ambiguous += diff.size
    print(f"C{config}: {ambiguous} boundary tokens over {len(rows)} rows, "
          f"{by_reference} of them from the reference's fp32 cumsum")
    assert ambiguous - by_reference <= 64


def test_token0_quirk_matches_the_reference_scatter():
    vocab = 1000
    x = torch.full((4, vocab), -3.0)
    x[:, 0], x[:, 1] = 5.0, 4.9
    p = [SamplingParams(repetition_penalty=2.0)] * 4
    ctx = [[0, 7, 8, 9], [0], [7, 0, 8, vocab + 1], [vocab + 1, 0, 7, 8]]
    got = step(x.numpy(), p, np.zeros(4), contexts=ctx).tokens
    want, _, _ = O.torch_reference_step(x, p, ctx, np.zeros(4))
    assert got.tolist() == want.tolist() == [1, 0, 0, 1]
