"""Parity of the HIP sampler with the canonical C oracle, on an MI355X.

Every comparison is bit-exact for integer and index outputs (tokens, top-k key,
top-p cut, kept mask, row maximum, kept and whole-row masses); normalised
probabilities are checked to 1e-5 relative (the north-star tolerance for fp32).
The workloads are the five BASELINE configurations (fie_amd/workloads.py): row
subsets spanning every parameter class at full vocabulary, and whole batches.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from fie_amd import _lib
from fie_amd import workloads as W
from fie_amd.batching.sampler import SEEDED_STREAM, SHARED_STREAM, BatchedSampler, resolve_params
from fie_amd.kernel import FusedSampler
from fie_amd.runtime.sampling import SamplingParams

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
PROB_RTOL = 1e-5
PROB_ATOL = 2.0 ** -40   # rule R1's weight quantisation: |dp| < C_t / T <= 2^-40


@pytest.fixture(scope="module")
def fs():
    return FusedSampler(DEV)


def _needs_mass(params):
    return np.array([(p.logprobs is not None) or (not p.greedy and not (0 < p.top_k))
                     for p in params])


def run_both(fs, logits, params, uniforms, contexts=None, kept=True):
    V = logits.shape[1]
    print(f"  case: rows={logits.shape[0]} vocab={V} dtype={logits.dtype}", flush=True)
    hp = resolve_params(params, V, uniforms, contexts)
    out, args, _ = fs.step(logits.to(DEV), hp)
    ref = O.canonical_step(logits.float().cpu().numpy(), O.resolve(params, V), uniforms,
                           contexts=contexts, want_kept=kept)
    gk = gp = None
    if kept:
        gk, gp = fs.kept(args)
        torch.cuda.synchronize()
        gk, gp = gk.cpu().numpy(), gp.cpu().numpy()
    return out, ref, gk, gp


def check(out, ref, params, gk=None, gp=None, lp=False):
    np.testing.assert_array_equal(out["tokens"], ref.tokens, err_msg="tokens")
    np.testing.assert_array_equal(out["row_max"].view(np.uint32), ref.row_max.view(np.uint32),
                                  err_msg="row max")
    np.testing.assert_array_equal(out["tk_key"], ref.tk_key, err_msg="top-k threshold key")
    np.testing.assert_array_equal(out["cut_comp"], ref.cut_comp, err_msg="top-p cut")
    np.testing.assert_array_equal(out["kept_mass"], ref.kept_mass, err_msg="kept mass")
    m = _needs_mass(params)
    np.testing.assert_array_equal(out["row_mass"][m], ref.row_mass[m], err_msg="row mass")
    if gk is not None:
        np.testing.assert_array_equal(gk, ref.kept, err_msg="kept set")
        np.testing.assert_allclose(gp, ref.probs, rtol=PROB_RTOL, atol=PROB_ATOL, err_msg="probs")
    if lp:
        want = np.array([p.logprobs is not None for p in params])
        np.testing.assert_allclose(out["chosen_lp"][want], ref.chosen_lp[want], rtol=1e-6, atol=1e-6)
        np.testing.assert_array_equal(out["top_ids"][want], ref.top_ids[want])
        np.testing.assert_allclose(out["top_lp"][want], ref.top_lp[want], rtol=1e-6, atol=1e-6)


SUBSETS = {
    1: list(range(8)),
    2: list(range(12)),
    3: [0, 1, 2, 3, 64, 65, 66, 67, 128, 129, 130, 131, 192, 193, 194, 195],
    4: list(range(8)),
    5: list(range(16)),
}


@pytest.mark.parametrize("config", [1, 2, 3, 4, 5])
def test_config_subset_bit_exact(fs, config):
    w = W.make(config, rows=SUBSETS[config])
    out, ref, gk, gp = run_both(fs, w.logits, w.params, w.uniforms, w.contexts)
    check(out, ref, w.params, gk, gp)


@pytest.mark.parametrize("config", [1, 2, 3, 5])
def test_config_full_batch_bit_exact(fs, config):
    w = W.make(config)
    out, ref, _, _ = run_both(fs, w.logits, w.params, w.uniforms, w.contexts, kept=False)
    check(out, ref, w.params)


def test_c4_full_batch_properties(fs):
    """C4 at full size (1024 rows): every token inside its own kept set, kept masses
    positive, and a 64-row sample bit-exact against the oracle."""
    w = W.make(4)
    hp = resolve_params(w.params, w.logits.shape[1], w.uniforms, None)
    out, args, _ = fs.step(w.logits.to(DEV), hp)
    kept, _ = fs.kept(args, want_probs=False)
    tok = torch.as_tensor(out["tokens"], device=DEV)
    assert bool(kept.gather(1, tok.unsqueeze(1)).all())
    assert (out["kept_mass"][:, 0] | out["kept_mass"][:, 1]).all()
    rows = list(range(0, 1024, 16))
    ref = O.canonical_step(w.logits[rows].float().cpu().numpy(), O.resolve(
        [w.params[r] for r in rows], w.logits.shape[1]), w.uniforms[rows])
    np.testing.assert_array_equal(out["tokens"][rows], ref.tokens)
    np.testing.assert_array_equal(out["cut_comp"][rows], ref.cut_comp)


def test_finish_register_variants_agree(fs):
    """A batch with more rows than the GPU has CUs takes the 128-register k_finish; C3's
    256 rows take the wide one.  The same rows in both (C3 plus every fourth row again,
    320 in all) give identical tokens, cuts, thresholds and kept masses."""
    w = W.make(3)
    V = w.logits.shape[1]
    extra = list(range(0, 256, 4))
    idx = list(range(256)) + extra
    print(f"  case: C3 rows 0..255 + {len(extra)} repeats, vocab={V}", flush=True)
    big, _, _ = fs.step(w.logits[idx].to(DEV), resolve_params(
        [w.params[i] for i in idx], V, w.uniforms[idx], [w.contexts[i] for i in idx]))
    small, _, _ = fs.step(w.logits.to(DEV), resolve_params(w.params, V, w.uniforms, w.contexts))
    for key in ("tokens", "cut_comp", "tk_key", "kept_mass"):
        np.testing.assert_array_equal(big[key][:256], small[key], err_msg=key)
        np.testing.assert_array_equal(big[key][256:], small[key][extra], err_msg=key)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_argmax_first_index_on_ties(fs, dtype):
    g = torch.Generator().manual_seed(7)
    x = torch.randn(37, 151936, generator=g).to(dtype)
    x[3, 100] = x[3, 90000] = 50.0          # tie: the first index wins
    x[5, :] = 1.0                            # all equal
    x[6, 151935] = 60.0                      # last index
    x[7, 0] = 70.0                           # first index
    got = fs.argmax(x.to(DEV)).cpu().numpy()
    want = np.argmax(x.float().numpy(), axis=1)
    np.testing.assert_array_equal(got, want)


def _mixed_params(rows, vocab, rng, with_lp=True):
    ps = []
    for i in range(rows):
        kind = i % 8
        lp = int(rng.integers(0, 21)) if with_lp and i % 3 == 0 else None
        if kind == 0:
            ps.append(SamplingParams(logprobs=lp))
        elif kind == 1:
            ps.append(SamplingParams(temperature=0.8, top_k=int(rng.integers(2, 60)), logprobs=lp,
                                     repetition_penalty=1.3, presence_penalty=0.2))
        elif kind == 2:
            ps.append(SamplingParams(temperature=1.3, top_p=float(rng.uniform(0.3, 0.99)),
                                     frequency_penalty=0.4, logprobs=lp))
        elif kind == 3:
            ps.append(SamplingParams(temperature=0.5, top_k=int(rng.integers(2, 200)),
                                     top_p=0.9, logprobs=lp))
        elif kind == 4:
            ps.append(SamplingParams(temperature=1.0, min_p=float(rng.uniform(0.01, 0.3)),
                                     logprobs=lp, repetition_penalty=0.8))
        elif kind == 5:
            ps.append(SamplingParams(temperature=2.0, logprobs=lp))
        elif kind == 6:
            ps.append(SamplingParams(temperature=0.7, top_k=vocab + 5, top_p=0.5,
                                     presence_penalty=-1.0, logprobs=lp))
        else:
            ps.append(SamplingParams(temperature=1.1, top_k=1, repetition_penalty=1.5))
    return ps


@pytest.mark.parametrize("vocab", [1, 7, 100, 8191, 8192, 8193, 20001])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_edge_shapes(fs, vocab, dtype):
    rng = np.random.default_rng(vocab * 7 + int(dtype == torch.float16))
    rows = 9
    x = torch.from_numpy(rng.normal(0, 2.0, (rows, vocab)).astype(np.float32)).to(dtype)
    params = _mixed_params(rows, vocab, rng)
    ctx = [list(rng.integers(0, vocab + 3, size=int(rng.integers(0, 40)))) + ([0] if r % 2 else [])
           for r in range(rows)]
    out, ref, gk, gp = run_both(fs, x, params, rng.random(rows), ctx)
    check(out, ref, params, gk, gp, lp=True)


def test_unaligned_rows_take_the_scalar_path(fs):
    rng = np.random.default_rng(11)
    rows, vocab = 6, 30001
    big = torch.from_numpy(rng.normal(0, 1.5, (rows, vocab + 1)).astype(np.float32)).half()
    x = big[:, :vocab]                                   # row stride vocab + 1
    assert x.stride(0) == vocab + 1
    params = _mixed_params(rows, vocab, rng)
    out, ref, gk, gp = run_both(fs, x, params, rng.random(rows), None)
    check(out, ref, params, gk, gp, lp=True)


def test_exact_path_rows(fs):
    """Rows whose answer lies outside the streamed candidates: a wide top-k, a deep
    nucleus on flat logits, plain temperature sampling and min-p on flat logits."""
    rng = np.random.default_rng(5)
    rows, vocab = 8, 151936
    x = torch.from_numpy(rng.normal(0, 0.2, (rows, vocab)).astype(np.float32)).to(torch.bfloat16)
    params = [SamplingParams(temperature=1.0, top_k=5000),
              SamplingParams(temperature=1.0, top_p=0.99),
              SamplingParams(temperature=1.0),
              SamplingParams(temperature=1.0, min_p=0.5, logprobs=20),
              SamplingParams(temperature=0.9, top_k=3000, top_p=0.97, logprobs=3),
              SamplingParams(temperature=1.7, top_p=0.999),
              SamplingParams(logprobs=5),
              SamplingParams(temperature=1.0, top_k=100000, top_p=0.5)]
    out, ref, gk, gp = run_both(fs, x, params, rng.random(rows), None)
    assert (out["status"] & _lib.FIE_ROW_EXACT_PATH).any()
    check(out, ref, params, gk, gp, lp=True)


def test_queued_full_row_path_matches_in_place(fs):
    """Rows outside the candidates go through the full-row path inside k_finish when a
    batch fits the CUs, and through k_deep's queue when it does not: the eight rows
    above, alone and repeated 33 times (264 rows), give identical outputs."""
    rng = np.random.default_rng(5)
    rows, vocab = 8, 151936
    x = torch.from_numpy(rng.normal(0, 0.2, (rows, vocab)).astype(np.float32)).to(torch.bfloat16)
    params = [SamplingParams(temperature=1.0, top_k=5000),
              SamplingParams(temperature=1.0, top_p=0.99),
              SamplingParams(temperature=1.0),
              SamplingParams(temperature=1.0, min_p=0.5, logprobs=20),
              SamplingParams(temperature=0.9, top_k=3000, top_p=0.97, logprobs=3),
              SamplingParams(temperature=1.7, top_p=0.999),
              SamplingParams(logprobs=5),
              SamplingParams(temperature=1.0, top_k=100000, top_p=0.5)]
    u = rng.random(rows)
    rep = 33
    print(f"  case: 8 full-row rows alone and x{rep}, vocab={vocab}", flush=True)
    one, _, _ = fs.step(x.to(DEV), resolve_params(params, vocab, u, None))
    many, _, _ = fs.step(x.repeat(rep, 1).to(DEV), resolve_params(params * rep, vocab, np.tile(u, rep), None))
    assert (many["status"] & _lib.FIE_ROW_EXACT_PATH).any()
    for key in ("status", "tokens", "tk_key", "cut_comp", "kept_mass", "row_mass"):
        want = np.concatenate([one[key]] * rep)
        np.testing.assert_array_equal(many[key], want, err_msg=key)
    lp_rows = [i for i, p in enumerate(params) if p.logprobs is not None]   # others write no logprobs
    for key in ("chosen_lp", "top_ids", "top_lp"):
        for r in range(rep):
            np.testing.assert_array_equal(many[key][[r * rows + i for i in lp_rows]], one[key][lp_rows], err_msg=key)


def test_ties_and_constant_rows(fs):
    rows, vocab = 6, 40000
    x = torch.zeros(rows, vocab)
    x[1] = torch.arange(vocab) % 3            # three values, huge tie classes
    x[2, 500:600] = 4.0
    x[3] = -1.0
    x[4, ::2] = 2.0
    x[5] = float("-inf")
    x[5, 777] = 1.0
    params = [SamplingParams(temperature=1.0, top_p=0.5), SamplingParams(temperature=1.0, top_k=10),
              SamplingParams(temperature=0.5, top_k=50, top_p=0.3, logprobs=20),
              SamplingParams(temperature=1.0, top_p=0.01, logprobs=4),
              SamplingParams(temperature=1.0, top_k=7, top_p=0.9),
              SamplingParams(temperature=1.0, top_p=0.9, logprobs=2)]
    out, ref, gk, gp = run_both(fs, x, params, np.linspace(0.01, 0.99, rows), None)
    check(out, ref, params, gk, gp, lp=True)


def test_long_history_counts_in_32_bits(fs):
    rng = np.random.default_rng(3)
    rows, vocab = 3, 50000
    x = torch.from_numpy(rng.normal(0, 2.0, (rows, vocab)).astype(np.float32))
    ctx = [[5] * 70000 + [0] * 3, list(rng.integers(0, vocab, 100)), [1, 2, 3]]
    params = [SamplingParams(temperature=1.0, top_k=20, frequency_penalty=0.001),
              SamplingParams(frequency_penalty=0.5, presence_penalty=0.1),
              SamplingParams(temperature=0.9, top_p=0.8, repetition_penalty=1.9)]
    out, ref, gk, gp = run_both(fs, x, params, rng.random(rows), ctx)
    check(out, ref, params, gk, gp)


def test_token0_penalty_quirk(fs):
    """Q1: a penalised token 0 keeps its penalty only in the batch's widest row, and
    an id >= vocab first seen after it undoes it (sampler.py:148,156-157,174-175)."""
    vocab = 1000
    x = torch.full((4, vocab), -3.0)
    x[:, 0] = 5.0
    x[:, 1] = 4.9
    p = SamplingParams(repetition_penalty=2.0)
    ctx = [[0, 7, 8, 9],          # widest row: token 0 penalised -> token 1 wins
           [0],                   # narrower row: pad writes undo it -> token 0 wins
           [7, 0, 8, vocab + 1],  # widest, but an invalid id after token 0 undoes it
           [vocab + 1, 0, 7, 8]]  # widest, invalid id before token 0: penalty holds
    out, ref, gk, gp = run_both(fs, x, [p] * 4, np.zeros(4), ctx)
    check(out, ref, [p] * 4, gk, gp)
    assert out["tokens"].tolist() == [1, 0, 0, 1]


def test_repeated_launch_with_same_args(fs):
    """The same argument block launched twice gives the same tokens (no state carried
    between calls)."""
    w = W.make(3, rows=SUBSETS[3])
    hp = resolve_params(w.params, w.logits.shape[1], w.uniforms, w.contexts)
    out, args, buf = fs.step(w.logits.to(DEV), hp)
    first = out["tokens"].copy()
    fs.launch(args)
    buf.download(torch.cuda.current_stream())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(buf.outputs()["tokens"], first)
    ref = O.canonical_step(w.logits.float().numpy(), O.resolve(w.params, w.logits.shape[1]),
                           w.uniforms, contexts=w.contexts)
    np.testing.assert_array_equal(first, ref.tokens)


def test_batched_sampler_end_to_end_logprobs(fs):
    rng = np.random.default_rng(9)
    rows, vocab = 10, 151936
    x = torch.from_numpy(rng.normal(0, 3.0, (rows, vocab)).astype(np.float32)).half().to(DEV)
    params = [SamplingParams(temperature=0.8, top_p=0.9, logprobs=5, seed=100 + r,
                             presence_penalty=0.5) for r in range(rows)]
    ctx = [list(rng.integers(0, vocab, 50)) for _ in range(rows)]
    s = BatchedSampler(DEV)
    res = s.sample(x, params, ctx, request_ids=[f"r{r}" for r in range(rows)])
    assert len(res.token_ids) == rows and set(res.logprobs) == set(range(rows))
    work = O.canonical_penalize(x.float().cpu().numpy(), O.resolve(params, vocab), ctx) / np.float32(0.8)
    for r in range(rows):
        lsm = O.log_softmax_ref(work[r])
        entries = res.logprobs[r]
        assert entries[0][0] == res.token_ids[r]
        for tok, val in entries:
            assert abs(val - lsm[tok]) <= 1e-5 * max(1.0, abs(lsm[tok])), (r, tok, val, lsm[tok])
        alts = [t for t, _ in entries[1:]]
        best = [int(i) for i in np.argsort(-lsm, kind="stable")[:5] if int(i) != res.token_ids[r]]
        assert alts == best[:len(alts)]


def test_batched_sampler_greedy_fast_path(fs):
    x = torch.randn(33, 151936).half().to(DEV)
    res = BatchedSampler(DEV).sample(x, [SamplingParams()] * 33)
    assert res.token_ids == x.float().argmax(dim=-1).tolist()
    assert res.logprobs == {}


def test_seeded_rows_are_batch_independent(fs):
    x = torch.randn(3, 5000).to(DEV)
    p = [SamplingParams(temperature=1.0, seed=1234)] * 3
    alone = BatchedSampler(DEV).sample(x[:1], p[:1]).token_ids[0]
    with_others = BatchedSampler(DEV).sample(x, p).token_ids[0]
    assert alone == with_others


def _philox_uniform(key0, key1, counter):
    """numpy's Philox4x64-10 generator at the kernel's block (numpy advances its
    counter before a block, hence counter - 1)."""
    g = np.random.Generator(np.random.Philox(key=int(key0) | (int(key1) << 64), counter=int(counter) - 1))
    return g.random()


def test_device_uniforms_match_numpys_philox(fs):
    rng = np.random.default_rng(17)
    keys = rng.integers(0, 2**63, size=(300, 3), dtype=np.uint64)
    keys[:, 2] = rng.integers(1, 2**40, size=300, dtype=np.uint64)
    keys[0] = (0, 0, 1)
    keys[1] = (2**64 - 1, 2**64 - 1, 2**64 - 1)
    got = fs.uniforms(torch.from_numpy(keys.view(np.int64)).to(DEV)).cpu().numpy()
    want = np.array([_philox_uniform(*k) for k in keys])
    np.testing.assert_array_equal(got, want)


def test_batched_sampler_draws_on_device_like_the_oracle(fs):
    """BatchedSampler's rows draw on the device from (seed or shared key, stream,
    counter); the oracle, given the same uniforms from numpy's Philox, picks the
    same tokens, over two steps (the counters advance)."""
    rng = np.random.default_rng(23)
    rows, vocab = 12, 30000
    x = torch.from_numpy(rng.normal(0, 1.5, (rows, vocab)).astype(np.float32)).to(DEV)
    params = [SamplingParams(temperature=1.0, top_p=0.95, seed=(77 if r % 3 == 0 else None))
              for r in range(rows)]
    ids = [f"q{r}" for r in range(rows)]
    s = BatchedSampler(DEV, generator_seed=4242)
    shared = 0
    for step in (1, 2):
        res = s.sample(x, params, None, ids)
        u = []
        for r, p in enumerate(params):
            if p.seed is None:
                shared += 1
                u.append(_philox_uniform(4242, SHARED_STREAM, shared))
            else:
                u.append(_philox_uniform(p.seed, SEEDED_STREAM, step))
        ref = O.canonical_step(x.cpu().numpy(), O.resolve(params, vocab), np.array(u))
        assert res.token_ids == ref.tokens.tolist(), step


def test_device_resident_history_over_decode_steps(fs):
    """BatchedSampler keeps penalty contexts on the device and uploads only the
    appended tokens: over several decode steps (one token per row, a rebuilt
    context, ids >= vocab and token 0 for the token-0 rule) its tokens equal the
    oracle's on the full contexts packed afresh."""
    rng = np.random.default_rng(31)
    rows, vocab = 9, 20000
    x = torch.from_numpy(rng.normal(0, 2.0, (rows, vocab)).astype(np.float32)).half().to(DEV)
    params = [SamplingParams(temperature=0.9, top_k=(0, 40)[r % 2], top_p=(1.0, 0.9)[r % 3 == 0],
                             repetition_penalty=1.3, frequency_penalty=0.2, presence_penalty=0.1,
                             seed=500 + r) for r in range(rows)]
    ctx = [list(rng.integers(0, vocab, size=int(rng.integers(5, 300)))) for _ in range(rows)]
    ctx[2] += [0, vocab + 5]
    ctx[4] = [vocab + 1, 0] + ctx[4]
    ids = [f"d{r}" for r in range(rows)]
    s = BatchedSampler(DEV)
    for step in range(1, 6):
        if step == 3:
            ctx[6] = ctx[6][:10]                                          # rebuilt, shorter
        res = s.sample(x, params, ctx, ids)
        u = [_philox_uniform(p.seed, SEEDED_STREAM, step) for p in params]
        ref = O.canonical_step(x.float().cpu().numpy(), O.resolve(params, vocab), np.array(u),
                               contexts=ctx)
        assert res.token_ids == ref.tokens.tolist(), step
        for c, t in zip(ctx, res.token_ids):
            c.append(t)


def test_cut_and_draw_beyond_the_first_sorted_prefix(fs):
    """Power-law rows whose top-p cut or plain draw lies hundreds of candidates
    deep, yet inside the complete region: the sorted prefix must reach it, equal
    the oracle, and need no full-row path."""
    rng = np.random.default_rng(41)
    rows, vocab = 8, 151936
    ranks = np.argsort(rng.random((rows, vocab)), axis=1)
    expo = np.array([1.7, 1.75, 1.65, 1.7, 1.7, 1.8, 1.7, 1.72])[:, None]
    x = torch.from_numpy((-expo * np.log(ranks + 1.0)).astype(np.float32))
    params = [SamplingParams(temperature=1.0, top_p=0.99)] * 4 + [SamplingParams(temperature=1.0)] * 4
    u = np.array([0.3, 0.9, 0.5, 0.99, 0.99, 0.995, 0.98, 0.97])
    out, ref, gk, gp = run_both(fs, x, params, u)
    check(out, ref, params, gk, gp)
    assert (out["status"] & 1).sum() == 0, out["status"]


def test_c_abi_direct_calls_and_errors(fs):
    lib = _lib.load()
    ws = fs.ensure_workspace(4, 1000)
    a = _lib.SamplerArgs()
    assert lib.fie_sampler_sample(ctypes.byref(a), ctypes.byref(ws), None) == _lib.FIE_E_ARG
    x = torch.randn(4, 1000, device=DEV)
    out = torch.empty(4, dtype=torch.int64, device=DEV)
    rc = lib.fie_sampler_argmax(x.data_ptr(), _lib.FIE_F32, 4, 1000, 1000, out.data_ptr(),
                                ctypes.byref(ws), None)
    assert rc == _lib.FIE_OK
    torch.cuda.synchronize()
    assert out.tolist() == x.argmax(-1).tolist()
    small = _lib.Workspace(ws.ptr, 16, 4, 1000)
    rc = lib.fie_sampler_argmax(x.data_ptr(), _lib.FIE_F32, 4, 1000, 1000, out.data_ptr(),
                                ctypes.byref(small), None)
    assert rc == _lib.FIE_E_WORKSPACE
    rc = lib.fie_sampler_argmax(x.data_ptr(), 7, 4, 1000, 1000, out.data_ptr(), ctypes.byref(ws), None)
    assert rc == _lib.FIE_E_ARG


def test_cexp_matches_oracle(fs):
    d = torch.linspace(-90.0, 0.0, 200001)
    got = fs.cexp(d.to(DEV)).cpu().numpy()
    want = O.cexp(d.numpy()[::97])
    np.testing.assert_array_equal(got[::97].view(np.uint32), want.view(np.uint32))


# ---------------------------------------------------------------- fused lm_head (f3)
def _lmhead_case(rows, vocab, H, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    hidden = torch.randn(rows, H, generator=g).to(dtype)
    weight = (torch.randn(vocab, H, generator=g) * (2.5 / H ** 0.5)).to(dtype)
    rng = np.random.default_rng(seed)
    params = _mixed_params(rows, vocab, rng)
    ctx = [list(rng.integers(0, vocab + 3, size=int(rng.integers(0, 300)))) + ([0] if r % 2 else [])
           for r in range(rows)]
    return hidden, weight, params, ctx, rng.random(rows)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,vocab,H", [(5, 5000, 128), (70, 20001, 512), (64, 8192, 256),
                                          (130, 151936, 1024)])
def test_lmhead_fused_matches_the_two_step_path(fs, dtype, rows, vocab, H):
    """fie_sampler_lmhead_sample: its logits are hidden @ weight.T to within one
    rounding of the model dtype (the fp32 sum's order differs from a library GEMM's),
    and every sampler output equals fie_sampler_sample's on those same logits, bit
    for bit: the fused epilogue computes the partials k_scan would have."""
    hidden, weight, params, ctx, u = _lmhead_case(rows, vocab, H, dtype, rows * 31 + H)
    hp = resolve_params(params, vocab, u, ctx)
    out, _, _, logits = fs.lmhead_step(hidden.to(DEV), weight.to(DEV), hp)
    ref = hidden.to(DEV).float() @ weight.to(DEV).float().T
    # the fused value is the fp32 reference rounded to the dtype, or a neighbour of it
    # (one ulp: the two fp32 sums may round to either side of a midpoint)
    got = logits.view(torch.int16).int()
    want = ref.to(dtype).view(torch.int16).int()
    # or, where the sum cancels, within the fp32 accumulation error of either order
    mag = hidden.to(DEV).float().abs() @ weight.to(DEV).float().abs().T
    near = ((got - want).abs() <= 1) | ((logits.float() - ref).abs() <= 32 * 2.0 ** -24 * mag)
    assert bool(near.all()), int((~near).sum())
    two, _, _ = fs.step(logits, hp)
    for name in ("tokens", "status", "tk_key", "cut_comp", "row_max", "kept_mass", "row_mass",
                 "chosen_lp", "top_ids", "top_lp"):
        np.testing.assert_array_equal(out[name], two[name], err_msg=name)


def test_lmhead_rejects_what_it_cannot_run(fs):
    hidden = torch.zeros(4, 100, dtype=torch.bfloat16, device=DEV)
    weight = torch.zeros(300, 100, dtype=torch.bfloat16, device=DEV)
    hp = resolve_params([SamplingParams()] * 4, 300, np.zeros(4), None)
    with pytest.raises(RuntimeError, match="multiple of 128"):
        fs.lmhead_step(hidden, weight, hp)
    with pytest.raises(ValueError):
        fs.lmhead_step(hidden.float(), weight.float(), hp)


def test_lmhead_long_history_counts(fs):
    """The fused kernel's long-history variant (a row's history over 65535 ids: u32
    penalty counts) matches the two-step path bit for bit."""
    rows, vocab, H = 6, 9000, 256
    hidden, weight, params, _, u = _lmhead_case(rows, vocab, H, torch.bfloat16, 77)
    rng = np.random.default_rng(77)
    params = [SamplingParams(temperature=0.9, top_p=0.8, repetition_penalty=1.3, frequency_penalty=0.01)] * rows
    ctx = [list(rng.integers(0, 40, size=70_000)) if r == 2 else list(rng.integers(0, vocab, size=50))
           for r in range(rows)]
    hp = resolve_params(params, vocab, u, ctx)
    assert hp.max_row_hist > 65535
    out, _, _, logits = fs.lmhead_step(hidden.to(DEV), weight.to(DEV), hp)
    two, _, _ = fs.step(logits, hp)
    for name in ("tokens", "status", "cut_comp", "row_max", "kept_mass", "row_mass"):
        np.testing.assert_array_equal(out[name], two[name], err_msg=name)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_queued_full_row_rows_match_the_oracle(fs, dtype):
    """More rows than CUs, many of them deep (flat logits): top-p and plain rows, with
    and without penalties, are queued by k_finish and settled by k_deep's full-row
    passes; tokens, cuts, thresholds and kept masses equal the oracle's."""
    rng = np.random.default_rng(77 + int(dtype == torch.bfloat16))
    rows, vocab = 300, 50000
    x = torch.from_numpy(rng.normal(0, 0.3, (rows, vocab)).astype(np.float32)).to(dtype)
    pen = dict(repetition_penalty=1.2, frequency_penalty=0.3, presence_penalty=0.1)
    params = []
    for r in range(rows):
        kind = r % 6
        if kind == 0:
            params.append(SamplingParams(temperature=1.0, top_p=0.95))
        elif kind == 1:
            params.append(SamplingParams(temperature=0.8, top_p=0.9, **pen))
        elif kind == 2:
            params.append(SamplingParams(temperature=1.0))
        elif kind == 3:
            params.append(SamplingParams(temperature=1.3, **pen))
        elif kind == 4:
            params.append(SamplingParams(temperature=1.0, top_p=0.5, top_k=3000))   # not split: top-k
        else:
            params.append(SamplingParams(**pen))                                    # greedy
    ctx = [list(rng.integers(0, vocab, size=int(rng.integers(0, 3000)))) for _ in range(rows)]
    out, ref, _, _ = run_both(fs, x, params, rng.random(rows), ctx, kept=False)
    check(out, ref, params)
    assert ((out["status"] & 1) != 0).sum() >= rows // 2, "the flat rows should take the full-row path"


def _helper_rows(rng, rows, vocab, dtype, sigma=3.0):
    x = torch.from_numpy(rng.normal(0, sigma, (rows, vocab)).astype(np.float32)).to(dtype)
    params = [SamplingParams(temperature=1.0),
              SamplingParams(temperature=1.0, top_p=0.9),
              SamplingParams(temperature=0.8, top_p=0.99, repetition_penalty=1.3,
                             frequency_penalty=0.2, presence_penalty=0.1),
              SamplingParams(temperature=1.0, min_p=0.001),
              SamplingParams(temperature=1.0, top_k=5000, top_p=0.95),
              SamplingParams(),
              SamplingParams(temperature=1.0, top_k=40),
              SamplingParams(temperature=1.2, logprobs=4)][:rows]
    ctx = [rng.integers(0, vocab, 3000).tolist() for _ in range(rows)]
    ctx[2] += list(range(8192, 9000)) * 2          # a span bucket that overflows
    return x, params, ctx


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_span_helpers_settle_small_batches(fs, dtype):
    """Batches of at most 16 rows run k_finish with a helper workgroup per span of
    each sampled row; the full-row rows (deep draws, deep nuclei, low min-p) are
    settled from the helpers' histograms and bucketed composites.  Bit-exact with the
    oracle, twice in a row (the arrival counters reset themselves), and equal to the
    same rows batched past the helper limit."""
    rng = np.random.default_rng(11)
    vocab = 151936
    x, params, ctx = _helper_rows(rng, 8, vocab, dtype)
    u = np.array([0.97, 0.5, 0.93, 0.99, 0.9, 0.0, 0.3, 0.95])
    out, ref, gk, gp = run_both(fs, x, params, u, ctx)
    assert (out["status"] & _lib.FIE_ROW_EXACT_PATH).sum() >= 3
    check(out, ref, params, gk, gp, lp=True)
    again, _, _ = fs.step(x.to(DEV), resolve_params(params, vocab, u, ctx))
    for key in ("status", "tokens", "cut_comp", "kept_mass", "row_mass", "tk_key"):
        np.testing.assert_array_equal(again[key], out[key], err_msg=key)
    rep = 3                                                   # 24 rows: no helpers
    print(f"  case: the same rows x{rep} (past the helper limit)", flush=True)
    many, _, _ = fs.step(x.repeat(rep, 1).to(DEV), resolve_params(params * rep, vocab, np.tile(u, rep), ctx * rep))
    for key in ("status", "tokens", "cut_comp", "kept_mass", "row_mass", "tk_key"):
        np.testing.assert_array_equal(many[key], np.concatenate([out[key]] * rep), err_msg=key)


def test_span_helpers_lone_rows_and_odd_shapes(fs):
    """One deep row alone; an unaligned row stride (scalar loads); a vocabulary that
    ends inside a span; token 0 as the row maximum (the helpers' maximum leaves it
    out, so the row is re-read instead)."""
    rng = np.random.default_rng(12)
    x = torch.from_numpy(rng.normal(0, 3.0, (1, 151936)).astype(np.float32))
    p = [SamplingParams(temperature=1.0, top_p=0.95)]
    out, ref, gk, gp = run_both(fs, x, p, np.array([0.98]))
    assert out["status"][0] & _lib.FIE_ROW_EXACT_PATH
    check(out, ref, p, gk, gp)
    for vocab in (20001, 8193):
        y = torch.from_numpy(rng.normal(0, 2.0, (5, vocab)).astype(np.float32)).to(torch.float16)
        params = [SamplingParams(temperature=1.0, top_p=0.99)] * 4 + [SamplingParams(temperature=1.0)]
        out, ref, gk, gp = run_both(fs, y, params, rng.random(5))
        check(out, ref, params, gk, gp)
    wide = torch.from_numpy(rng.normal(0, 3.0, (3, 151936 + 3)).astype(np.float32)).to(DEV)
    y = wide[:, :151936]                                     # rows 151939 elements apart
    assert y.stride(0) == 151939
    params = [SamplingParams(temperature=1.0, top_p=0.97)] * 3
    out, ref, _, _ = run_both(fs, y, params, np.array([0.99, 0.7, 0.95]), kept=False)
    check(out, ref, params)
    z = torch.from_numpy(rng.normal(0, 1.0, (2, 151936)).astype(np.float32))
    z[:, 0] = 6.0                                             # token 0 is the maximum
    params = [SamplingParams(temperature=1.0, top_p=0.999), SamplingParams(temperature=1.0)]
    out, ref, gk, gp = run_both(fs, z, params, np.array([0.999, 0.999]))
    assert (out["status"] & _lib.FIE_ROW_EXACT_PATH).all()
    check(out, ref, params, gk, gp)


def test_span_helpers_flat_rows_repeated(fs):
    """Twelve flat bf16 rows (top-p, min-p, a wide top-k, both, plain draws) run with
    span helpers five times over: every call bit-exact with the oracle, whichever of
    a row's workgroups arrives last."""
    rng = np.random.default_rng(5)
    x = torch.from_numpy(rng.normal(0, 0.3, (12, 151936)).astype(np.float32)).to(torch.bfloat16)
    params = [SamplingParams(temperature=1.0, top_p=0.95), SamplingParams(temperature=1.0, min_p=0.05),
              SamplingParams(temperature=1.0, top_k=2000),
              SamplingParams(temperature=0.9, top_k=3000, top_p=0.97),
              SamplingParams(temperature=1.0)] * 2 + [SamplingParams(), SamplingParams(temperature=1.0, top_p=0.5)]
    u = rng.random(12)
    V = x.shape[1]
    print(f"  case: 12 flat bf16 rows x5, vocab={V}", flush=True)
    ref = O.canonical_step(x.float().numpy(), O.resolve(params, V), u, want_kept=False)
    hp = resolve_params(params, V, u, None)
    xd = x.to(DEV)
    for _ in range(5):
        out, _, _ = fs.step(xd, hp)
        assert (out["status"] & _lib.FIE_ROW_EXACT_PATH).sum() >= 4
        check(out, ref, params)
