"""CPU tests of the host side: the parameter type, history packing, per-request
uniforms, logprob assembly, and the C-ABI's exports and argument errors (no
kernel runs; the library loads without a GPU).

The reference behaviour restated here is engine/runtime/sampling.py:19-97 and
engine/batching/sampler.py:32-117,262-291 (read, not run).
"""

import ctypes
import os
import re

import numpy as np
import pytest

from fie_amd import _lib
from fie_amd.batching.sampler import (SEEDED_STREAM, SHARED_STREAM, BatchedSampler, SampleResult,
                                      pack_history, resolve_params)
from fie_amd.kernel import FLAG_GREEDY, FLAG_PENALTY
from fie_amd.runtime.sampling import GREEDY, SamplingParams

HEADER = os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "include", "fie_sampler.h")


# ---------------------------------------------------------------- SamplingParams
def test_defaults_are_plain_greedy():
    p = SamplingParams()
    assert (p.temperature, p.top_p, p.top_k, p.min_p) == (0.0, 1.0, 0, 0.0)
    assert (p.repetition_penalty, p.presence_penalty, p.frequency_penalty) == (1.0, 0.0, 0.0)
    assert p.greedy and not p.has_penalties and p.deterministic and p.can_reuse_cached_prediction
    assert GREEDY == p
    assert SamplingParams(stop_token_ids=[3, 3, 5]).stop_token_ids == frozenset({3, 5})


@pytest.mark.parametrize("kwargs, message", [
    (dict(temperature=-0.1), "temperature must be in [0, 2]"),
    (dict(temperature=2.5), "temperature must be in [0, 2]"),
    (dict(top_p=0.0), "top_p must be in (0, 1]"),
    (dict(top_p=1.5), "top_p must be in (0, 1]"),
    (dict(top_k=-1), "top_k must be non-negative (0 disables it)"),
    (dict(min_p=1.5), "min_p must be in [0, 1]"),
    (dict(repetition_penalty=0.0), "repetition_penalty must be in (0, 2]"),
    (dict(repetition_penalty=2.5), "repetition_penalty must be in (0, 2]"),
    (dict(presence_penalty=-3.0), "presence_penalty must be in [-2, 2]"),
    (dict(frequency_penalty=2.5), "frequency_penalty must be in [-2, 2]"),
    (dict(logprobs=21), "logprobs must be in [0, 20]"),
    (dict(seed=-1), "seed must be a non-negative 63-bit integer"),
    (dict(seed=2**63), "seed must be a non-negative 63-bit integer"),
])
def test_validation_matches_the_reference_messages(kwargs, message):
    """sampling.py:50-69: the same ranges, each failure a ValueError with its text."""
    with pytest.raises(ValueError) as e:
        SamplingParams(**kwargs)
    assert str(e.value) == message


def test_predicates():
    """sampling.py:71-94."""
    assert SamplingParams(temperature=0.8, top_k=1).greedy
    assert not SamplingParams(temperature=0.8).greedy
    assert SamplingParams(temperature=0.8, seed=3).deterministic
    assert not SamplingParams(temperature=0.8).deterministic
    assert SamplingParams(presence_penalty=0.1).has_penalties
    assert not SamplingParams(presence_penalty=0.1).can_reuse_cached_prediction
    assert not SamplingParams(logprobs=2).can_reuse_cached_prediction


# ---------------------------------------------------------------- host packing
def _naive_pack(contexts, include, vocab):
    """The history CSR and the Q1 flags by direct definition: first occurrences in
    order, ids >= vocab counted distinct, bit 30 when one first occurs after 0."""
    offs, ids, invalid = [0], [], []
    for c, inc in zip(contexts, include):
        c = list(c) if inc else []
        ids.extend(c)
        offs.append(len(ids))
        big_first = {}
        for pos, t in enumerate(c):
            if t >= vocab and t not in big_first:
                big_first[t] = pos
        v = len(big_first)
        if 0 in c and any(pos > c.index(0) for pos in big_first.values()):
            v |= 1 << 30
        invalid.append(v)
    return np.array(offs), np.array(ids, dtype=np.int32), np.array(invalid, dtype=np.int32)


def test_pack_history_matches_its_definition():
    rng = np.random.default_rng(3)
    vocab = 50
    for _ in range(40):
        rows = int(rng.integers(1, 7))
        contexts = [list(rng.integers(0, vocab + 4, size=int(rng.integers(0, 12)))) for _ in range(rows)]
        include = rng.random(rows) < 0.7
        offs, ids, invalid, longest = pack_history(contexts, include, vocab)
        w_offs, w_ids, w_inv = _naive_pack(contexts, include, vocab)
        np.testing.assert_array_equal(offs, w_offs)
        np.testing.assert_array_equal(ids, w_ids)
        np.testing.assert_array_equal(invalid if invalid is not None else np.zeros(rows, np.int32), w_inv)
        assert longest == max(np.diff(w_offs))


def test_pack_history_rejects_negative_ids():
    with pytest.raises(ValueError):
        pack_history([[1, -2]], np.array([True]), 10)


def test_resolve_params_follows_the_reference_row_rules():
    """sampler.py:109,182-192: greedy rows are unscaled and unfiltered; top_k >= vocab,
    top_p == 1 and min_p == 0 are off; penalties apply only with contexts."""
    vocab = 100
    params = [SamplingParams(),
              SamplingParams(temperature=0.5, top_k=150, top_p=0.9, min_p=0.1),
              SamplingParams(temperature=0.7, top_k=1, top_p=0.5),
              SamplingParams(temperature=1.2, repetition_penalty=1.3, logprobs=3)]
    hp = resolve_params(params, vocab, np.zeros(4), [[1, 2], [3], [4], [5, 5, 7]])
    np.testing.assert_array_equal(hp.scale, np.float32([1.0, 0.5, 1.0, 1.2]))
    np.testing.assert_array_equal(hp.top_k, [0, 0, 0, 0])
    np.testing.assert_array_equal(hp.top_p, np.float32([1.0, 0.9, 1.0, 1.0]))
    np.testing.assert_array_equal(hp.min_p, np.float32([0.0, 0.1, 0.0, 0.0]))
    np.testing.assert_array_equal(hp.flags, [FLAG_GREEDY, 0, FLAG_GREEDY, FLAG_PENALTY])
    np.testing.assert_array_equal(hp.logprobs, [-1, -1, -1, 3])
    assert hp.apply_penalties
    np.testing.assert_array_equal(hp.hist_off, [0, 0, 0, 0, 3])    # only the penalised row
    np.testing.assert_array_equal(hp.hist_ids, [5, 5, 7])
    assert not resolve_params(params, vocab, np.zeros(4), None).apply_penalties


def test_device_history_tracks_appends_rebuilds_and_growth():
    """DeviceHistory's bookkeeping on a CPU array, the appends written as the
    kernel writes them: after every update each penalised row's [start, end) range
    holds exactly its context, only appended tokens are written, and the token-0
    flags equal pack_history's."""
    import torch
    from fie_amd.batching.history import DeviceHistory

    vocab = 40
    h = DeviceHistory(torch.device("cpu"), capacity=300)
    rng = np.random.default_rng(8)
    ctx = {f"r{i}": list(rng.integers(0, vocab, size=int(rng.integers(1, 30)))) for i in range(5)}
    for step in range(60):
        ids = list(ctx)
        for rid in ids:
            ctx[rid].append(int(rng.integers(0, vocab + 3)))           # decode: one token
        if step % 17 == 5:
            ctx["r1"] = ctx["r1"][:3] + [7, 7]                         # rebuilt shorter
        if step % 23 == 11:
            h.forget(["r2"])
            ctx["r9"] = list(rng.integers(0, vocab, size=400))         # forces growth
        ids = list(ctx)
        include = np.array([rid != "r3" for rid in ids])
        contexts = [ctx[rid] for rid in ids]
        starts, ends, invalid, longest, dst, src = h.update(contexts, include, ids, vocab)
        h.ids[torch.from_numpy(dst)] = torch.from_numpy(src)            # what k_history_write does
        for r, rid in enumerate(ids):
            got = h.ids[starts[r]:ends[r]].numpy()
            if include[r]:
                np.testing.assert_array_equal(got, np.array(ctx[rid], dtype=np.int32))
            else:
                assert starts[r] == ends[r] == 0
        _, _, want_inv, want_long = pack_history(contexts, include, vocab)
        np.testing.assert_array_equal(invalid if invalid is not None else 0,
                                      want_inv if want_inv is not None else 0)
        assert longest == want_long
        if step > 0 and step % 17 != 5 and step % 23 != 11:
            assert dst.size == sum(include)                            # only the appends moved


def test_device_history_duplicate_rows_and_rejected_ids():
    """A request twice in one batch takes the row-by-row update: each of its rows reads
    the request's whole context.  An id outside [0, 2**31) raises before any slot moves:
    the next valid update appends exactly as if the failed one never happened."""
    import torch
    from fie_amd.batching.history import DeviceHistory

    vocab = 50
    h = DeviceHistory(torch.device("cpu"), capacity=64)
    a_ctx, b_ctx = [1, 2, 3], [4, 0, 60]
    starts, ends, invalid, _, dst, src = h.update([a_ctx, b_ctx, a_ctx], np.ones(3, bool), ["a", "b", "a"], vocab)
    h.ids[torch.from_numpy(dst)] = torch.from_numpy(src)
    for r, ctx in enumerate([a_ctx, b_ctx, a_ctx]):
        np.testing.assert_array_equal(h.ids[starts[r]:ends[r]].numpy(), np.array(ctx, dtype=np.int32))
    assert invalid is not None and invalid[1] == 1 | (1 << 30) and invalid[0] == invalid[2] == 0
    before = {rid: (s.start, s.length, tuple(s.tail)) for rid, s in h.slots.items()}
    with pytest.raises(ValueError):
        h.update([a_ctx + [5], b_ctx + [-1]], np.ones(2, bool), ["a", "b"], vocab)
    assert {rid: (s.start, s.length, tuple(s.tail)) for rid, s in h.slots.items()} == before
    starts, ends, _, _, dst, src = h.update([a_ctx + [5], b_ctx + [6]], np.ones(2, bool), ["a", "b"], vocab)
    assert dst.size == 2
    h.ids[torch.from_numpy(dst)] = torch.from_numpy(src)
    np.testing.assert_array_equal(h.ids[starts[1]:ends[1]].numpy(), np.array(b_ctx + [6], dtype=np.int32))


def _check_ranges(h, contexts, include, starts, ends, dst, src):
    """Apply the appends as k_history_write does, then every included row's range
    must hold exactly its context."""
    import torch
    h.ids[torch.from_numpy(dst)] = torch.from_numpy(src)
    for r, ctx in enumerate(contexts):
        if include[r]:
            np.testing.assert_array_equal(h.ids[starts[r]:ends[r]].numpy(), np.array(ctx, dtype=np.int32))


def test_device_history_compaction_inside_one_batch():
    """A batch whose later rows need fresh space after most stored contexts were
    forgotten: the array is compacted (slots move) before any row's range or write
    position is recorded, so every row, the earlier ones included, reads exactly its
    context and each appended token lands inside its row's range."""
    import torch
    from fie_amd.batching.history import DeviceHistory

    vocab = 100
    h = DeviceHistory(torch.device("cpu"), capacity=1024)
    first = {"x1": [1] * 10, "x2": [2] * 10, "x3": [3] * 10, "a": [4, 5, 6]}
    ids = list(first)
    ctxs = [first[k] for k in ids]
    inc = np.ones(len(ids), bool)
    starts, ends, _, _, dst, src = h.update(ctxs, inc, ids, vocab)
    _check_ranges(h, ctxs, inc, starts, ends, dst, src)
    assert h.slots["a"].start == 768                     # behind three 256-int slots
    h.forget(["x1", "x2", "x3"])
    # 'a' appends one token (recorded first), 'b' is new and does not fit: compaction
    ctxs = [[4, 5, 6, 7], list(range(300))]
    ids = ["a", "b"]
    inc = np.ones(2, bool)
    starts, ends, _, _, dst, src = h.update(ctxs, inc, ids, vocab)
    assert h.slots["a"].start == 0                       # 'a' moved down
    assert starts[0] == h.slots["a"].start and ends[0] == starts[0] + 4
    assert starts[0] <= dst[0] < ends[0]
    _check_ranges(h, ctxs, inc, starts, ends, dst, src)


def test_device_history_detects_a_changed_prefix():
    """A stored context is reused only when the new one extends it: a context of
    the same request id that keeps the stored last token but differs earlier (a
    reused id), or that rolls back and regrows, is stored afresh."""
    import torch
    from fie_amd.batching.history import DeviceHistory

    vocab = 50
    h = DeviceHistory(torch.device("cpu"), capacity=4096)
    inc = np.ones(1, bool)
    for old, new in (([1, 2, 3], [9, 9, 3, 4]),                       # differs before the last token
                     (list(range(40)), list(range(30)) + [7] * 9 + [39, 40]),   # rollback, regrown
                     (list(range(40)), [5] + list(range(1, 41)))):     # the first token changed
        h.forget(["q"])
        starts, ends, _, _, dst, src = h.update([old], inc, ["q"], vocab)
        _check_ranges(h, [old], inc, starts, ends, dst, src)
        starts, ends, _, _, dst, src = h.update([new], inc, ["q"], vocab)
        assert dst.size == len(new)                                    # stored afresh
        _check_ranges(h, [new], inc, starts, ends, dst, src)


def test_device_history_rowwise_replacement_keeps_earlier_rows():
    """One request twice in a batch with a context the second row does not extend:
    the first row's range stays readable (its slot is not reused in the step)."""
    import torch
    from fie_amd.batching.history import DeviceHistory

    vocab = 50
    h = DeviceHistory(torch.device("cpu"), capacity=300)
    ctxs = [[1, 2, 3, 4], [7, 8], [1, 2, 3, 4, 5]]
    inc = np.ones(3, bool)
    starts, ends, _, _, dst, src = h.update(ctxs, inc, ["a", "a", "b"], vocab)
    _check_ranges(h, ctxs, inc, starts, ends, dst, src)


# ---------------------------------------------------------------- the adapter's calls
class _NoKernels(BatchedSampler):
    """BatchedSampler with its host state only (the constructor's device setup is
    skipped): exercises validation, draw keys and logprob assembly on the CPU."""

    def __init__(self, generator_seed=None, max_generators=1024):
        from collections import OrderedDict
        self._shared_key = generator_seed if generator_seed is not None else 12345
        self._shared_draws = 0
        self._seeded = OrderedDict()
        self._max_generators = max_generators
        import torch
        from fie_amd.batching.history import DeviceHistory
        self._history = DeviceHistory(torch.device("cpu"), capacity=16)


def test_sample_validation_errors():
    """sampler.py:89-97."""
    import torch
    s = _NoKernels()
    x = torch.zeros(2, 5)
    with pytest.raises(ValueError):
        s.sample(torch.zeros(5), [GREEDY])
    with pytest.raises(ValueError):
        s.sample(x, [GREEDY])
    with pytest.raises(ValueError):
        s.sample(x, [GREEDY] * 2, context_tokens=[[1]])
    with pytest.raises(ValueError):
        s.sample(x, [GREEDY] * 2, request_ids=["a"])
    assert s.sample(torch.zeros(0, 5), []) == SampleResult([], {})


def test_seeded_rows_draw_from_their_own_request_stream():
    """sampler.py:58-73: a seeded request draws from its own stream (keyed by its
    seed, positioned per request id: two requests with one seed do not share a
    position), unaffected by the rest of the batch; forget() starts it over."""
    p = SamplingParams(temperature=1.0, seed=7)
    q = SamplingParams(temperature=1.0)
    a = _NoKernels(generator_seed=1)
    k1 = a._draw_keys([p, q, p], ["r1", "x", "r2"])
    assert k1[0].tolist() == [7, SEEDED_STREAM, 1] and k1[2].tolist() == [7, SEEDED_STREAM, 1]
    assert k1[1].tolist() == [1, SHARED_STREAM, 1]
    b = _NoKernels(generator_seed=99)
    k2 = b._draw_keys([q, q, p], ["y", "z", "r1"])
    assert k2[2].tolist() == k1[0].tolist()         # batch-independent
    assert a._draw_keys([p], ["r1"])[0, 2] == 2      # the stream advances
    a.forget(["r1"])
    assert a._draw_keys([p], ["r1"])[0, 2] == 1      # and restarts after forget
    assert a._draw_keys([GREEDY], ["g"]).tolist() == [[0, 0, 0]]
    assert a._draw_keys([q, q], None)[:, 2].tolist() == [2, 3]   # the shared stream moves on


def test_request_counters_are_capped():
    s = _NoKernels(max_generators=3)
    p = SamplingParams(temperature=1.0, seed=1)
    s._draw_keys([p] * 5, [f"r{i}" for i in range(5)])
    assert list(s._seeded) == ["r2", "r3", "r4"]


def philox_uniform_reference(key0, key1, counter):
    """The draw the kernels derive from (key0, key1, counter), by numpy's own
    Philox4x64-10 (an independent implementation of Salmon et al. 2011): numpy
    advances its counter before a block, so counter - 1 starts at our block."""
    g = np.random.Generator(np.random.Philox(key=int(key0) | (int(key1) << 64), counter=int(counter) - 1))
    return g.random()


def test_draw_formula_is_numpys_philox_generator():
    """The host-side statement of the device draw (first word of the block, 53
    bits) equals numpy's Generator(Philox).random() at that position; the GPU
    test checks the kernel against the same function."""
    M = (1 << 64) - 1
    M0, M1 = 0xD2E7470EE14C6C93, 0xCA5A826395121157
    W0, W1 = 0x9E3779B97F4A7C15, 0xBB67AE8584CAA73B

    def block(ctr, k0, k1):
        x = [ctr, 0, 0, 0]
        for r in range(10):
            if r:
                k0, k1 = (k0 + W0) & M, (k1 + W1) & M
            p0, p1 = M0 * x[0], M1 * x[2]
            x = [(p1 >> 64) ^ x[1] ^ k0, p1 & M, (p0 >> 64) ^ x[3] ^ k1, p0 & M]
        return x

    for k0, k1, c in [(0, 0, 1), (7, SEEDED_STREAM, 3), (M, SHARED_STREAM, 123456789)]:
        assert (block(c, k0, k1)[0] >> 11) * 2.0 ** -53 == philox_uniform_reference(k0, k1, c)


def test_logprob_entries_follow_the_reference_layout():
    """sampler.py:282-290: (chosen, lp) first, then the best alternatives other than
    the chosen token, at most count + 1 entries."""
    params = [SamplingParams(logprobs=2), GREEDY, SamplingParams(temperature=1.0, logprobs=0)]
    out = {"chosen_lp": np.float32([-0.5, 0.0, -1.5]),
           "top_ids": np.array([[4, 9, 1], [0, 0, 0], [-1, -1, -1]]),
           "top_lp": np.float32([[-0.5, -1.0, -2.0], [0, 0, 0], [0, 0, 0]])}
    got = BatchedSampler._logprobs(params, [4, 3, 8], out)
    assert got == {0: [(4, -0.5), (9, -1.0)], 2: [(8, -1.5)]}


# ---------------------------------------------------------------- the C-ABI
def _declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(fie_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_function():
    lib = _lib.load()
    declared = _declared_functions()
    assert len(declared) >= 8
    assert set(declared) == set(_lib.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name


def test_workspace_size():
    lib = _lib.load()
    assert lib.fie_sampler_workspace_size(256, 151936) > 256 * 151936 // 2048 * 64 * 8
    assert lib.fie_sampler_workspace_size(1, 0) == 0
    assert lib.fie_sampler_workspace_size(1, _lib.MAX_VOCAB + 1) == 0
    assert lib.fie_sampler_workspace_size(1024, 151936) <= _lib.SCRATCH_BYTES
    # a workspace for at most 16 rows also holds the span helpers' arrays: per row and
    # 8192-token span, the histogram (20 KiB), the bin offsets and the span's composites
    spans = -(-151936 // 8192)
    helpers = 16 * spans * (1024 * 20 + 1028 * 4 + 8192 * 8)
    assert lib.fie_sampler_workspace_size(16, 151936) >= helpers
    assert lib.fie_sampler_workspace_size(17, 151936) < lib.fie_sampler_workspace_size(16, 151936)
    assert lib.fie_sampler_workspace_size(16, 151936) <= _lib.SCRATCH_BYTES


def _args(**kw):
    a = _lib.SamplerArgs()
    a.dtype, a.rows, a.vocab, a.row_stride, a.lp_cols = _lib.FIE_F32, 2, 100, 100, 0
    for f in ("logits", "tokens", "scale", "top_k", "top_p", "min_p", "flags", "uniform"):
        setattr(a, f, 256)           # never dereferenced: every case fails its checks first
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw, code, text", [
    (dict(dtype=7), _lib.FIE_E_ARG, b"dtype"),
    (dict(rows=-1), _lib.FIE_E_ARG, b"rows"),
    (dict(vocab=0), _lib.FIE_E_ARG, b"vocab"),
    (dict(row_stride=50), _lib.FIE_E_ARG, b"row_stride"),
    (dict(lp_cols=21), _lib.FIE_E_ARG, b"lp_cols"),
    (dict(logits=None), _lib.FIE_E_ARG, b"NULL"),
    (dict(apply_penalties=1), _lib.FIE_E_ARG, b"penalt"),
])
def test_sample_rejects_bad_arguments(kw, code, text):
    lib = _lib.load()
    a = _args(**kw)
    ws = _lib.Workspace(256, 1 << 20, 2, 100)
    assert lib.fie_sampler_sample(ctypes.byref(a), ctypes.byref(ws), None) == code
    assert text in lib.fie_sampler_last_error()


def test_sample_rejects_bad_workspaces():
    lib = _lib.load()
    a = _args()
    need = lib.fie_sampler_workspace_size(2, 100)
    cases = [(_lib.Workspace(None, need, 2, 100), b"missing"),
             (_lib.Workspace(256 + 8, need, 2, 100), b"aligned"),
             (_lib.Workspace(256, need, 1, 100), b"fewer rows"),
             (_lib.Workspace(256, need - 1, 2, 100), b"too small")]
    for ws, text in cases:
        assert lib.fie_sampler_sample(ctypes.byref(a), ctypes.byref(ws), None) == _lib.FIE_E_WORKSPACE
        assert text in lib.fie_sampler_last_error()
    assert lib.fie_sampler_sample(None, None, None) == _lib.FIE_E_ARG
    assert lib.fie_sampler_stage(ctypes.byref(a), ctypes.byref(cases[0][0]), 5, None) == _lib.FIE_E_ARG


def test_lmhead_argument_errors():
    """fie_sampler_lmhead_sample rejects, before any launch, a logits dtype other
    than the model's fp16/bf16 and a hidden size that is not a multiple of 128."""
    lib = _lib.load()
    a = _args()
    ws = _lib.Workspace(256, lib.fie_sampler_workspace_size(2, 100), 2, 100)
    assert lib.fie_sampler_lmhead_sample(ctypes.byref(a), None, None, 128, ctypes.byref(ws), None) == _lib.FIE_E_ARG
    assert b"fp16 or bf16" in lib.fie_sampler_last_error()
    a.dtype = _lib.FIE_BF16
    assert lib.fie_sampler_lmhead_sample(ctypes.byref(a), None, None, 100, ctypes.byref(ws), None) == _lib.FIE_E_ARG
    assert b"multiple of 128" in lib.fie_sampler_last_error()
    assert lib.fie_sampler_lmhead_sample(None, None, None, 128, ctypes.byref(ws), None) == _lib.FIE_E_ARG


def test_zero_rows_is_a_no_op():
    lib = _lib.load()
    a = _args(rows=0)
    assert lib.fie_sampler_sample(ctypes.byref(a), None, None) == _lib.FIE_OK
    assert lib.fie_sampler_sample_noalloc(ctypes.byref(a), None) == _lib.FIE_OK


def test_noalloc_rejects_shapes_beyond_its_array_before_any_device_call():
    lib = _lib.load()
    a = _args(rows=4096, vocab=151936, row_stride=151936)
    assert lib.fie_sampler_sample_noalloc(ctypes.byref(a), None) == _lib.FIE_E_WORKSPACE
    assert b"static scratch" in lib.fie_sampler_last_error()


def test_argmax_and_cexp_argument_errors():
    lib = _lib.load()
    assert lib.fie_sampler_argmax(None, 9, 1, 10, 10, None, None, None) == _lib.FIE_E_ARG
    assert lib.fie_sampler_argmax(None, 0, 1, 10, 5, None, None, None) == _lib.FIE_E_ARG
    assert lib.fie_sampler_argmax(None, 0, 1, 10, 10, None, None, None) == _lib.FIE_E_ARG
    assert lib.fie_sampler_cexp(None, None, -1, None) == _lib.FIE_E_ARG
    assert lib.fie_sampler_cexp(None, None, 0, None) == _lib.FIE_OK
