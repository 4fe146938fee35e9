"""Writes the reference-produced kept-set fixtures (run in the build container only).

The reference's sampler is Python over PyTorch.  This script loads its two files by
path, ``engine/runtime/sampling.py`` and ``engine/batching/sampler.py``, under stub
``engine`` / ``engine.runtime`` packages (the real ``engine/runtime/__init__.py``
imports request.py, which needs Python >= 3.11), and runs the stages of
``BatchedSampler.sample`` that decide the kept sets, exactly as sample() chains them
(sampler.py:108-114): ``.float()``, ``_apply_penalties`` when any row has penalties
and contexts are given, ``_apply_temperature``, ``_filter``.  Greedy rows' tokens are
the argmax of the filtered row, as ``_draw`` takes them (sampler.py:236-239).

For each batch it writes ``reference_kept_<name>.npz`` beside this file: the
kept_summary description of every row's kept set plus the greedy tokens.  The
inputs are regenerated from seeds by the tests (fie_amd/workloads.py for C1-C5,
kept_summary.EXTRA for the extra cases), so only outputs are stored.

Usage:  python tests/golden/make_reference_filter.py [--reference /root/reference]
"""

from __future__ import annotations

import argparse
import importlib.util
import os
import sys
import types

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "full-inference-engine_amd"))
sys.path.insert(0, HERE)

import kept_summary as KS  # noqa: E402
from fie_amd import workloads as W  # noqa: E402


def load_reference(root: str):
    for name in ("engine", "engine.runtime", "engine.batching"):
        mod = types.ModuleType(name)
        mod.__path__ = []
        sys.modules[name] = mod

    def load(name, rel):
        spec = importlib.util.spec_from_file_location(name, os.path.join(root, rel))
        mod = importlib.util.module_from_spec(spec)
        sys.modules[name] = mod
        spec.loader.exec_module(mod)
        return mod

    sampling = load("engine.runtime.sampling", "engine/runtime/sampling.py")
    sampler = load("engine.batching.sampler", "engine/batching/sampler.py")
    return sampling, sampler


def reference_filter(sampler_mod, logits, params, contexts):
    s = sampler_mod.BatchedSampler("cpu")
    working = logits.float()
    if any(p.has_penalties for p in params) and contexts is not None:
        working = s._apply_penalties(working, params, contexts)
    working = s._apply_temperature(working, params)
    filtered = s._filter(working, params)
    greedy = np.full(len(params), -1, np.int64)
    rows = [r for r, p in enumerate(params) if p.greedy]
    if rows:
        greedy[rows] = filtered[rows].argmax(dim=-1).numpy()
    return working.numpy(), torch.isfinite(filtered).numpy(), greedy


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    ap.add_argument("--only", nargs="*")
    a = ap.parse_args()
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    sampling, sampler_mod = load_reference(a.reference)
    RefParams = sampling.SamplingParams

    cases = {}
    for cfg in (1, 2, 3, 4, 5):
        cases[f"C{cfg}"] = lambda cfg=cfg: _workload(cfg, RefParams)
    for name, fn in KS.EXTRA.items():
        cases[name] = lambda fn=fn: fn(RefParams)
    for name, make in cases.items():
        if a.only and name not in a.only:
            continue
        logits, params, contexts = make()
        working, kept, greedy = reference_filter(sampler_mod, logits, params, contexts)
        summ = KS.summarize(kept, working)
        sampled = np.array([not p.greedy for p in params])
        path = os.path.join(HERE, f"reference_kept_{name}.npz")
        np.savez_compressed(path, greedy_token=greedy, sampled=sampled, **summ)
        print(f"{name}: {logits.shape[0]} rows, mean kept {summ['count'][sampled].mean():.1f}"
              f" -> {os.path.relpath(path, REPO)}", flush=True)


def _workload(cfg, RefParams):
    """The workload's logits and contexts, with its parameters rebuilt as the
    reference's own SamplingParams (same field values)."""
    w = W.make(cfg)
    fields = ("temperature", "top_p", "top_k", "min_p", "repetition_penalty",
              "presence_penalty", "frequency_penalty", "penalize_prompt", "seed", "logprobs")
    params = [RefParams(**{f: getattr(p, f) for f in fields}) for p in w.params]
    return w.logits, params, w.contexts


if __name__ == "__main__":
    main()
