"""Batched per-row sampling on MI355X: the reference's call surface over HIP kernels.

``BatchedSampler`` keeps the constructor, ``sample``/``forget`` and ``SampleResult``
of the reference (engine/batching/sampler.py:32-117), so the engine's ``_sample``
adapter (engine/batching/continuous_batching.py:1911-1931) can call it unchanged.
What changes is underneath: one packed parameter upload, a fixed chain of fused HIP
kernels, one packed download.  The draw is an inverse-CDF draw against a per-row
uniform that the kernel derives on the device from a counter-based generator
(Philox4x64-10): a seeded request draws from its own stream, keyed by its seed and
advanced per request, so its tokens do not depend on its batch neighbours; the
other rows share one stream keyed by ``generator_seed``.  The host keeps only
counters.
"""

from __future__ import annotations

import operator
import os
from collections import OrderedDict
from dataclasses import dataclass

import numpy as np
import torch

from ..kernel import FLAG_GREEDY, FLAG_PENALTY, FusedSampler, HostParams
from .history import DeviceHistory
from ..runtime.sampling import SamplingParams


@dataclass
class SampleResult:
    """Chosen token per row, plus logprobs for the rows that asked for them
    (engine/batching/sampler.py:32-39)."""

    token_ids: list[int]
    logprobs: dict[int, list[tuple[int, float]]]


def pack_history(contexts: list[list[int]], include: np.ndarray, vocab: int):
    """CSR of the penalty contexts of the rows in `include` (sampler.py:136-144 reads
    only penalised rows), plus, per row, the ids >= vocab that the reference's
    scatter sends to index 0 (sampler.py:156-157): their distinct count, and bit 30
    when one of them first occurs after token 0's first occurrence."""
    rows = len(contexts)
    parts = [np.asarray(c, dtype=np.int64) if include[i] and len(c) else _EMPTY
             for i, c in enumerate(contexts)]
    lengths = np.fromiter((p.shape[0] for p in parts), dtype=np.int64, count=rows)
    offsets = np.zeros(rows + 1, dtype=np.int64)
    np.cumsum(lengths, out=offsets[1:])
    flat = np.concatenate(parts) if offsets[-1] else _EMPTY
    invalid = None
    if flat.size:
        if flat.min() < 0 or flat.max() >= 2**31:
            raise ValueError("penalty context token ids must be in [0, 2**31)")
        bad = flat >= vocab
        if bad.any():
            invalid = np.zeros(rows, dtype=np.int32)
            for r in np.unique(np.searchsorted(offsets, np.nonzero(bad)[0], side="right") - 1):
                ids = parts[r]
                big, first = np.unique(ids[ids >= vocab], return_index=True)
                value = int(big.size)
                zero = np.nonzero(ids == 0)[0]
                if zero.size:
                    # first occurrences of the big ids, as positions in the row
                    pos = np.nonzero(ids >= vocab)[0][first]
                    if (pos > zero[0]).any():
                        value |= 1 << 30
                invalid[r] = value
    longest = int(lengths.max()) if rows else 0
    return offsets, flat.astype(np.int32), invalid, longest


_EMPTY = np.zeros(0, dtype=np.int64)


class ParamTable:
    """Per-row columns of a batch's SamplingParams, from one pass over the objects.

    A decode loop passes the same SamplingParams objects step after step (each
    request keeps its own); the last table is reused when the batch holds exactly the
    same objects in the same order.  The table keeps those objects alive, so an
    identity match cannot be a new object at a recycled address."""

    __slots__ = ("objs", "greedy", "pen", "temps", "top_k", "top_p", "min_p", "lp",
                 "rep", "pres", "freq", "seeded", "seeds", "_resolved")

    def __init__(self, params: list[SamplingParams]):
        self.objs = list(params)
        rows = [(p.greedy, p.has_penalties, p.temperature, p.top_k, p.top_p, p.min_p,
                 -1 if p.logprobs is None else p.logprobs, p.repetition_penalty,
                 p.presence_penalty, p.frequency_penalty,
                 p.seed is not None, 0 if p.seed is None else p.seed) for p in params]
        cols = list(zip(*rows)) if rows else [()] * 12
        self.greedy = np.array(cols[0], dtype=bool)
        self.pen = np.array(cols[1], dtype=bool)
        self.temps = np.array(cols[2], dtype=np.float64)
        self.top_k = np.array(cols[3], dtype=np.int64)
        self.top_p = np.array(cols[4], dtype=np.float64)
        self.min_p = np.array(cols[5], dtype=np.float64)
        self.lp = np.array(cols[6], dtype=np.int32)
        self.rep = np.array(cols[7], dtype=np.float32)
        self.pres = np.array(cols[8], dtype=np.float32)
        self.freq = np.array(cols[9], dtype=np.float32)
        self.seeded = np.array(cols[10], dtype=bool)
        self.seeds = np.array(cols[11], dtype=np.uint64) if rows else np.zeros(0, np.uint64)
        self._resolved: dict[int, tuple] = {}

    def resolved(self, vocab: int) -> tuple:
        """(scale, top_k, top_p, min_p, flags) as the kernels take them, resolved the way
        sampler.py:182-192 does for this vocabulary (computed once per table)."""
        r = self._resolved.get(vocab)
        if r is None:
            greedy, pen = self.greedy, self.pen
            r = (np.where(greedy, 1.0, self.temps).astype(np.float32),
                 np.where((self.top_k > 0) & (self.top_k < vocab) & ~greedy, self.top_k, 0).astype(np.int32),
                 np.where((self.top_p < 1.0) & ~greedy, self.top_p, 1.0).astype(np.float32),
                 np.where((self.min_p > 0.0) & ~greedy, self.min_p, 0.0).astype(np.float32),
                 greedy.astype(np.int32) * FLAG_GREEDY + pen.astype(np.int32) * FLAG_PENALTY)
            self._resolved[vocab] = r
        return r

    def matches(self, params: list[SamplingParams]) -> bool:
        objs = self.objs
        return len(params) == len(objs) and all(map(operator.is_, params, objs))


_last_table: list[ParamTable | None] = [None]


def param_table(params: list[SamplingParams]) -> ParamTable:
    t = _last_table[0]
    if t is None or not t.matches(params):
        t = ParamTable(params)
        _last_table[0] = t
    return t


def resolve_params(params: list[SamplingParams], vocab: int, uniforms: np.ndarray | None,
                   contexts: list[list[int]] | None, rng: np.ndarray | None = None,
                   history: DeviceHistory | None = None,
                   request_ids: list[object] | None = None) -> HostParams:
    """Per-row arrays for the kernels, derived the way sampler.py:109,182-192 does.
    The draws are `uniforms` (float64 [rows]) or, when `rng` (uint64 [rows, 3]) is
    given, derived on the device from it.  With a `history` and `request_ids` the
    penalty contexts are kept on the device across steps (only appended tokens
    move); otherwise they are packed afresh."""
    rows = len(params)
    if uniforms is None:
        uniforms = np.zeros(rows, dtype=np.float64)
    t = param_table(params)
    greedy, pen, temps, top_k, top_p, min_p = t.greedy, t.pen, t.temps, t.top_k, t.top_p, t.min_p
    apply = bool(pen.any()) and contexts is not None
    ends = dst = src = None
    if apply and history is not None and request_ids is not None:
        offsets, ends, invalid, longest, dst, src = history.update(contexts, pen, request_ids, vocab)
        ids = _EMPTY.astype(np.int32)
    elif apply:
        offsets, ids, invalid, longest = pack_history(contexts, pen, vocab)
    else:
        offsets, ids, invalid, longest = np.zeros(rows + 1, np.int64), _EMPTY.astype(np.int32), None, 0
    r_scale, r_top_k, r_top_p, r_min_p, r_flags = t.resolved(vocab)
    return HostParams(
        scale=r_scale,
        top_k=r_top_k,
        top_p=r_top_p,
        min_p=r_min_p,
        flags=r_flags,
        logprobs=t.lp,
        uniform=np.ascontiguousarray(uniforms, dtype=np.float64),
        rep=t.rep,
        pres=t.pres,
        freq=t.freq,
        hist_off=offsets,
        hist_ids=ids,
        apply_penalties=apply,
        hist_invalid=invalid,
        max_row_hist=longest,
        rng=None if rng is None else np.ascontiguousarray(rng, dtype=np.uint64).reshape(rows, 3),
        hist_ends=ends,
        hist_store=history if ends is not None else None,
        hist_write_dst=dst,
        hist_write_src=src,
    )


# Second key words of the two kinds of draw streams: a seeded request's stream is
# keyed (seed, SEEDED), the shared stream (generator_seed, SHARED).
SEEDED_STREAM = 0x5EEDED5EEDED5EED
SHARED_STREAM = 0x5A4ED5A4ED5A4ED5


class BatchedSampler:
    """Applies per-request sampling to one step's logits (sampler.py:42-78).

    Holds no per-request state besides the draw counters of seeded requests:
    penalties come from the token ids the caller passes, so a preempted and rebuilt
    request samples identically.
    """

    def __init__(self, device: torch.device | str, *, generator_seed: int | None = None,
                 max_generators: int = 1024):
        self.device = torch.device(device)
        self._fused = FusedSampler(self.device)
        # The shared stream for rows without their own seed.
        self._shared_key = (int(generator_seed) if generator_seed is not None
                            else int.from_bytes(os.urandom(8), "little")) & 0xFFFFFFFFFFFFFFFF
        self._shared_draws = 0
        # Request id -> draws taken so far (sampler.py:58-61): two requests with one
        # seed must not share a stream position, so counters are kept per request,
        # not per seed; at most max_generators of them, least recently used dropped.
        self._seeded: OrderedDict[object, int] = OrderedDict()
        self._max_generators = max_generators
        # Penalty contexts of the requests, kept on the device between steps.
        self._history = DeviceHistory(self.device)

    def _next_draw(self, request_id: object) -> int:
        n = self._seeded.pop(request_id, 0) + 1
        self._seeded[request_id] = n
        while len(self._seeded) > self._max_generators:
            self._seeded.popitem(last=False)
        return n

    def forget(self, request_ids: list[object]) -> None:
        """Drop the streams of finished requests (sampler.py:75-78)."""
        for request_id in request_ids:
            self._seeded.pop(request_id, None)
        self._history.forget(request_ids)

    def _draw_keys(self, params: list[SamplingParams],
                   request_ids: list[object] | None) -> np.ndarray:
        """uint64 [rows, 3] (key0, key1, counter) per row: a seeded row's request
        stream at its next position, the shared stream in row order otherwise
        (greedy rows draw nothing)."""
        rows = len(params)
        t = param_table(params)
        keys = np.zeros((rows, 3), dtype=np.uint64)
        shared = np.nonzero(~t.greedy & ~t.seeded)[0]
        if shared.size:
            keys[shared, 0] = self._shared_key
            keys[shared, 1] = SHARED_STREAM
            keys[shared, 2] = np.arange(self._shared_draws + 1, self._shared_draws + 1 + shared.size,
                                        dtype=np.uint64)
            self._shared_draws += int(shared.size)
        for r in np.nonzero(~t.greedy & t.seeded)[0].tolist():
            rid = request_ids[r] if request_ids is not None else r
            keys[r] = (int(t.seeds[r]), SEEDED_STREAM, self._next_draw(rid))
        return keys

    # ------------------------------------------------------------------ the step
    def sample(
        self,
        logits: torch.Tensor,
        params: list[SamplingParams],
        context_tokens: list[list[int]] | None = None,
        request_ids: list[object] | None = None,
    ) -> SampleResult:
        """Choose one token per row (sampler.py:81-117)."""
        if logits.ndim != 2:
            raise ValueError("logits must have shape [rows, vocab]")
        rows, vocab = logits.shape
        if len(params) != rows:
            raise ValueError("one SamplingParams per logits row is required")
        if context_tokens is not None and len(context_tokens) != rows:
            raise ValueError("one context per logits row is required")
        if request_ids is not None and len(request_ids) != rows:
            raise ValueError("one request id per logits row is required")
        if rows == 0:
            return SampleResult([], {})

        # the per-row predicates from one pass over the params (reused while a decode
        # loop passes the same SamplingParams objects)
        t = param_table(params)
        wants_logprobs = bool((t.lp >= 0).any())
        plain = bool((t.greedy & ~t.pen).all())
        if plain and not wants_logprobs:
            # sampler.py:103-106: one argmax kernel and one device-to-host copy.
            return SampleResult(self._fused.argmax(logits).tolist(), {})

        hp = resolve_params(params, vocab, None, context_tokens,
                            rng=self._draw_keys(params, request_ids),
                            history=self._history, request_ids=request_ids)
        out, _, _ = self._fused.step(logits, hp)
        tokens = out["tokens"].tolist()
        return SampleResult(tokens, self._logprobs(params, tokens, out) if wants_logprobs else {})

    @staticmethod
    def _logprobs(params: list[SamplingParams], chosen: list[int],
                  out: dict[str, np.ndarray]) -> dict[int, list[tuple[int, float]]]:
        """Chosen-token logprob first, then the row's best alternatives
        (sampler.py:262-291)."""
        result: dict[int, list[tuple[int, float]]] = {}
        for row, p in enumerate(params):
            if p.logprobs is None:
                continue
            count = p.logprobs
            entries = [(chosen[row], float(out["chosen_lp"][row]))]
            ids = out["top_ids"][row][:count]
            vals = out["top_lp"][row][:count]
            entries.extend((int(t), float(v)) for t, v in zip(ids, vals)
                           if t >= 0 and int(t) != chosen[row])
            result[row] = entries[:count + 1]
        return result
