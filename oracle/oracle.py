"""TEST INFRASTRUCTURE ONLY: the CPU checker for the HIP sampler.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module.  The product package never does.

Two restatements of the reference sampler live here:

* ``canonical_step`` drives ``canonical.c`` (built by ``oracle/Makefile``), the
  plain-C restatement with the build's canonical rules for top-p bits, tie order and
  the inverse-CDF draw.  The HIP sampler must match it bit for bit.
* ``torch_reference_step`` follows ``engine/batching/sampler.py:81-291`` op by op with
  PyTorch CPU tensors, as the reference itself executes on a CPU, except that the
  ``torch.multinomial`` draw is replaced by the canonical draw.  It is the CPU
  baseline that ``bench.py`` times, and the model of the reference's own fp32
  rounding that the tests compare kept sets against.

``resolve`` maps ``SamplingParams``-like objects to the per-row arrays both use,
following the reference's predicates line by line.
"""

from __future__ import annotations

import ctypes
import math
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.oracle_cexp.restype = ctypes.c_float
        _lib.oracle_cexp.argtypes = [ctypes.c_float]
        _lib.oracle_sample.restype = ctypes.c_int32
        _lib.oracle_sample.argtypes = [ctypes.c_void_p]
        _lib.oracle_penalize.restype = ctypes.c_int32
        _lib.oracle_cexp_monotone_violations.restype = ctypes.c_int64
        _lib.oracle_cexp_monotone_violations.argtypes = [ctypes.c_float, ctypes.c_float]
        _lib.oracle_minp_bound.restype = ctypes.c_float
        _lib.oracle_minp_bound.argtypes = [ctypes.c_float]
        _lib.oracle_markstein_mismatches.restype = ctypes.c_int64
        _lib.oracle_markstein_mismatches.argtypes = [ctypes.c_float, ctypes.c_int64, ctypes.c_uint32]
    return _lib


def cexp_monotone_violations(lo: float, hi: float) -> int:
    """Adjacent fp32 pairs in [lo, hi] where the canonical exponential decreases."""
    return int(_load().oracle_cexp_monotone_violations(lo, hi))


def minp_bound(mp: float) -> float:
    """Rule R5's bound L: a token survives min-p iff fl(y - M) >= L."""
    return float(_load().oracle_minp_bound(mp))


def markstein_mismatches(s: float, nrandom: int = 1_000_000, seed: int = 1) -> int:
    """Inputs in the guarded range where the kernels' Markstein-corrected divide by
    `s` differs from the IEEE quotient (all fp16, all bf16, `nrandom` fp32)."""
    return int(_load().oracle_markstein_mismatches(s, nrandom, seed))


def cexp(values: np.ndarray) -> np.ndarray:
    """The canonical fp32 exponential, elementwise (scalar calls; small inputs)."""
    lib = _load()
    flat = np.asarray(values, dtype=np.float32).ravel()
    out = np.array([lib.oracle_cexp(float(v)) for v in flat], dtype=np.float32)
    return out.reshape(np.shape(values))


# --------------------------------------------------------------------- parameters
@dataclass
class Resolved:
    """Per-row arrays after the reference's predicates (sampler.py:182-192)."""

    scale: np.ndarray        # float32, divisor (1.0 for greedy rows)
    top_k: np.ndarray        # int32, 0 = off
    top_p: np.ndarray        # float32, 1.0 = off
    min_p: np.ndarray        # float32, 0 = off
    greedy: np.ndarray       # uint8
    logprobs: np.ndarray     # int32, -1 = None
    has_pen: np.ndarray      # uint8
    rep: np.ndarray          # float32
    pres: np.ndarray         # float32
    freq: np.ndarray         # float32


def _greedy(p) -> bool:
    # sampling.py:71-74
    return p.temperature == 0.0 or p.top_k == 1


def _has_pen(p) -> bool:
    # sampling.py:76-79
    return (p.repetition_penalty != 1.0 or p.presence_penalty != 0.0
            or p.frequency_penalty != 0.0)


def resolve(params, vocab: int) -> Resolved:
    g = [_greedy(p) for p in params]
    return Resolved(
        # sampler.py:182-184: torch.tensor of python floats -> float32
        scale=np.array([1.0 if gi else p.temperature for p, gi in zip(params, g)],
                       dtype=np.float32),
        # sampler.py:190
        top_k=np.array([p.top_k if 0 < p.top_k < vocab and not gi else 0
                        for p, gi in zip(params, g)], dtype=np.int32),
        # sampler.py:191 (float32 like the `limit` tensor at :223)
        top_p=np.array([p.top_p if p.top_p < 1.0 and not gi else 1.0
                        for p, gi in zip(params, g)], dtype=np.float32),
        # sampler.py:192
        min_p=np.array([p.min_p if p.min_p > 0.0 and not gi else 0.0
                        for p, gi in zip(params, g)], dtype=np.float32),
        greedy=np.array(g, dtype=np.uint8),
        logprobs=np.array([-1 if p.logprobs is None else p.logprobs for p in params],
                          dtype=np.int32),
        has_pen=np.array([_has_pen(p) for p in params], dtype=np.uint8),
        rep=np.array([p.repetition_penalty for p in params], dtype=np.float32),
        pres=np.array([p.presence_penalty for p in params], dtype=np.float32),
        freq=np.array([p.frequency_penalty for p in params], dtype=np.float32),
    )


def pack_history(contexts, rows: int):
    offsets = np.zeros(rows + 1, dtype=np.int64)
    if contexts is None:
        return offsets, np.zeros(0, dtype=np.int32)
    for i, c in enumerate(contexts):
        offsets[i + 1] = offsets[i] + len(c)
    ids = np.fromiter((t for c in contexts for t in c), dtype=np.int64, count=int(offsets[-1]))
    return offsets, ids.astype(np.int32)


# --------------------------------------------------------------------- canonical C
class _Args(ctypes.Structure):
    _fields_ = [
        ("B", ctypes.c_int32), ("V", ctypes.c_int32),
        ("logits", ctypes.c_void_p),
        ("scale", ctypes.c_void_p), ("top_k", ctypes.c_void_p), ("top_p", ctypes.c_void_p),
        ("min_p", ctypes.c_void_p), ("greedy", ctypes.c_void_p), ("logprobs", ctypes.c_void_p),
        ("uniform", ctypes.c_void_p),
        ("apply_penalties", ctypes.c_int32),
        ("has_pen", ctypes.c_void_p), ("rep", ctypes.c_void_p), ("pres", ctypes.c_void_p),
        ("freq", ctypes.c_void_p), ("hist_off", ctypes.c_void_p), ("hist_ids", ctypes.c_void_p),
        ("lp_cols", ctypes.c_int32),
        ("tokens", ctypes.c_void_p), ("tk_key", ctypes.c_void_p), ("cut_comp", ctypes.c_void_p),
        ("row_max", ctypes.c_void_p), ("kept_mass", ctypes.c_void_p), ("row_mass", ctypes.c_void_p),
        ("kept", ctypes.c_void_p), ("probs", ctypes.c_void_p), ("chosen_lp", ctypes.c_void_p),
        ("top_ids", ctypes.c_void_p), ("top_lp", ctypes.c_void_p),
    ]


@dataclass
class CanonicalResult:
    tokens: np.ndarray
    tk_key: np.ndarray
    cut_comp: np.ndarray
    row_max: np.ndarray
    kept_mass: np.ndarray    # uint64 [B, 2]: low and high 64 bits
    row_mass: np.ndarray     # uint64 [B, 2]
    kept: np.ndarray | None
    probs: np.ndarray | None
    chosen_lp: np.ndarray
    top_ids: np.ndarray
    top_lp: np.ndarray
    penalized: np.ndarray


def _ptr(a):
    return None if a is None else a.ctypes.data


def canonical_step(logits: np.ndarray, res: Resolved, uniform: np.ndarray,
                   contexts=None, want_kept: bool = False,
                   lp_cols: int = 20) -> CanonicalResult:
    """One sampler step on fp32 logits [B, V] (already upcast from the engine dtype)."""
    lib = _load()
    w = np.ascontiguousarray(logits, dtype=np.float32).copy()
    B, V = w.shape
    off, ids = pack_history(contexts, B)
    apply = int(contexts is not None and bool(res.has_pen.any()))
    if apply and ids.size and ids.min() < 0:
        raise ValueError("negative token id in a penalty context")
    uni = np.ascontiguousarray(uniform, dtype=np.float64)
    out = CanonicalResult(
        tokens=np.zeros(B, np.int64), tk_key=np.zeros(B, np.uint32),
        cut_comp=np.zeros(B, np.uint64), row_max=np.zeros(B, np.float32),
        kept_mass=np.zeros((B, 2), np.uint64), row_mass=np.zeros((B, 2), np.uint64),
        kept=np.zeros((B, V), np.uint8) if want_kept else None,
        probs=np.zeros((B, V), np.float32) if want_kept else None,
        chosen_lp=np.zeros(B, np.float32),
        top_ids=np.full((B, lp_cols), -1, np.int64), top_lp=np.zeros((B, lp_cols), np.float32),
        penalized=w,
    )
    keep = [w, res.scale, res.top_k, res.top_p, res.min_p, res.greedy, res.logprobs, uni,
            res.has_pen, res.rep, res.pres, res.freq, off, ids]
    a = _Args(
        B=B, V=V, logits=_ptr(w), scale=_ptr(res.scale), top_k=_ptr(res.top_k),
        top_p=_ptr(res.top_p), min_p=_ptr(res.min_p), greedy=_ptr(res.greedy),
        logprobs=_ptr(res.logprobs), uniform=_ptr(uni), apply_penalties=apply,
        has_pen=_ptr(res.has_pen), rep=_ptr(res.rep), pres=_ptr(res.pres), freq=_ptr(res.freq),
        hist_off=_ptr(off), hist_ids=_ptr(ids) if ids.size else None, lp_cols=lp_cols,
        tokens=_ptr(out.tokens), tk_key=_ptr(out.tk_key), cut_comp=_ptr(out.cut_comp),
        row_max=_ptr(out.row_max), kept_mass=_ptr(out.kept_mass), row_mass=_ptr(out.row_mass),
        kept=_ptr(out.kept), probs=_ptr(out.probs), chosen_lp=_ptr(out.chosen_lp),
        top_ids=_ptr(out.top_ids), top_lp=_ptr(out.top_lp),
    )
    rc = lib.oracle_sample(ctypes.byref(a))
    del keep
    if rc == -2:
        raise ValueError("vocab must be in [1, 2**24)")
    if rc != 0:
        raise ValueError("negative token id in a penalty context")
    return out


def canonical_penalize(logits: np.ndarray, res: Resolved, contexts) -> np.ndarray:
    """The penalty stage alone (sampler.py:120-175) on fp32 logits."""
    lib = _load()
    w = np.ascontiguousarray(logits, dtype=np.float32).copy()
    B, V = w.shape
    off, ids = pack_history(contexts, B)
    lib.oracle_penalize.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32] + \
        [ctypes.c_void_p] * 6
    rc = lib.oracle_penalize(_ptr(w), B, V, _ptr(res.has_pen), _ptr(res.rep), _ptr(res.pres),
                             _ptr(res.freq), _ptr(off), _ptr(ids) if ids.size else None)
    if rc < 0:
        raise ValueError("negative token id in a penalty context")
    return w


def fkey(values: np.ndarray) -> np.ndarray:
    """Order-preserving uint32 key of fp32 values (-0 folded into +0)."""
    v = np.asarray(values, dtype=np.float32) + np.float32(0.0)
    b = v.view(np.uint32)
    return np.where(b & np.uint32(0x80000000), ~b, b | np.uint32(0x80000000)).astype(np.uint32)


# --------------------------------------------------------------------- torch restatement
def torch_reference_step(logits, params, contexts=None, uniform=None):
    """sampler.py:81-291 as PyTorch CPU ops (the reference's own execution model).

    Returns ``(tokens, filtered, working)``: the chosen ids, the filtered fp32 logits
    (``-inf`` where a filter dropped a token, the output of ``_filter``), and the
    penalised, temperature-scaled logits (``working``).  The draw for sampled rows is
    the canonical inverse-CDF rule (R4) on the reference's fp32 probabilities, since the
    reference's ``torch.multinomial`` stream is not reproducible across devices.
    """
    import torch

    rows, vocab = logits.shape
    working = logits.float()
    if any(_has_pen(p) for p in params) and contexts is not None:
        working = _torch_penalties(working, params, contexts)
    scale = torch.tensor([1.0 if _greedy(p) else p.temperature for p in params]).unsqueeze(1)
    working = working / scale
    filtered = _torch_filter(working, params)
    tokens = torch.empty(rows, dtype=torch.long)
    greedy_rows = [r for r, p in enumerate(params) if _greedy(p)]
    if greedy_rows:
        idx = torch.tensor(greedy_rows)
        tokens[idx] = filtered.index_select(0, idx).argmax(dim=-1)
    sampled = [r for r, p in enumerate(params) if not _greedy(p)]
    if sampled:
        probs = filtered.softmax(dim=-1)
        for r in sampled:
            order = torch.sort(filtered[r], descending=True, stable=True).indices
            cdf = probs[r][order].double().cumsum(0)
            u = 0.0 if uniform is None else float(uniform[r])
            pos = int(torch.searchsorted(cdf, torch.tensor([u * float(cdf[-1])],
                                                          dtype=torch.float64), right=True))
            tokens[r] = order[min(pos, vocab - 1)]
    return tokens, filtered, working


def _torch_penalties(logits, params, contexts):
    import torch

    rows, vocab = logits.shape
    pad = vocab
    packed, counts = [], []
    for row, tokens in enumerate(contexts):
        if not _has_pen(params[row]) or not tokens:
            packed.append([])
            counts.append([])
            continue
        occ: dict[int, int] = {}
        for t in tokens:
            occ[t] = occ.get(t, 0) + 1
        packed.append(list(occ))
        counts.append([float(v) for v in occ.values()])
    width = max((len(r) for r in packed), default=0)
    if width == 0:
        return logits
    index = torch.full((rows, width), pad, dtype=torch.long)
    count = torch.zeros((rows, width), dtype=torch.float32)
    for row, (toks, occ) in enumerate(zip(packed, counts)):
        if toks:
            index[row, :len(toks)] = torch.tensor(toks, dtype=torch.long)
            count[row, :len(toks)] = torch.tensor(occ, dtype=torch.float32)
    valid = index < vocab
    safe = index.masked_fill(~valid, 0)
    rep = torch.tensor([p.repetition_penalty for p in params]).unsqueeze(1)
    pres = torch.tensor([p.presence_penalty for p in params]).unsqueeze(1)
    freq = torch.tensor([p.frequency_penalty for p in params]).unsqueeze(1)
    gathered = logits.gather(1, safe)
    pen = torch.where(gathered > 0, gathered / rep, gathered * rep)
    pen = pen - pres - freq * count
    pen = torch.where(valid, pen, gathered)
    return logits.scatter(1, safe, pen)


def _torch_filter(logits, params):
    import torch

    rows, vocab = logits.shape
    g = [_greedy(p) for p in params]
    top_k = [p.top_k if 0 < p.top_k < vocab and not gi else 0 for p, gi in zip(params, g)]
    top_p = [p.top_p if p.top_p < 1.0 and not gi else 1.0 for p, gi in zip(params, g)]
    min_p = [p.min_p if p.min_p > 0.0 and not gi else 0.0 for p, gi in zip(params, g)]
    if any(top_k):
        kth = logits.topk(max(top_k), dim=-1).values
        index = torch.tensor([(k - 1 if k else 0) for k in top_k]).unsqueeze(1)
        threshold = kth.gather(1, index)
        enabled = torch.tensor([bool(k) for k in top_k]).unsqueeze(1)
        logits = torch.where(enabled & (logits < threshold),
                             torch.full_like(logits, float("-inf")), logits)
    if any(v > 0.0 for v in min_p):
        probs = logits.softmax(dim=-1)
        floor = probs.max(dim=-1, keepdim=True).values * torch.tensor(min_p).unsqueeze(1)
        logits = torch.where(probs < floor, torch.full_like(logits, float("-inf")), logits)
    if any(v < 1.0 for v in top_p):
        ordered, order = logits.sort(dim=-1, descending=True)
        cumulative = ordered.softmax(dim=-1).cumsum(dim=-1)
        limit = torch.tensor(top_p).unsqueeze(1)
        drop = cumulative - ordered.softmax(dim=-1) >= limit
        ordered = ordered.masked_fill(drop, float("-inf"))
        logits = torch.empty_like(logits).scatter_(1, order, ordered)
    return logits


def uniforms(rows: int, seed: int) -> np.ndarray:
    return np.random.default_rng(seed).random(rows)


def log_softmax_ref(working_row) -> np.ndarray:
    """fp64 log-softmax of one working row (a tolerance reference for logprobs)."""
    x = np.asarray(working_row, dtype=np.float64)
    m = x.max()
    return x - m - math.log(np.exp(x - m).sum())
