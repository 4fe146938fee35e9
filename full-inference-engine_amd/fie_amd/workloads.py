"""Synthetic sampler workloads of the benchmark configurations (seeded).

Five shapes, each a [rows, vocab] logits tensor plus per-row ``SamplingParams``,
penalty histories and draw uniforms:

  C1  8 x 151936 fp32, N(0, 3^2); rows 0-3 greedy, rows 4-7 temperature 1.0
  C2  64 x 151936 fp32 "peaked": -1.1*ln(rank+1) + N(0, 0.5^2) over a seeded
      permutation of ranks; temperature 0.7, top-k 50, top-p 0.9 on every row
  C3  256 x 151936 fp16 peaked; quarters greedy / top-k {20,50,100} /
      top-p {0.8,0.9,0.95} / both, temperature 0.7 on sampled rows; repetition
      1.1, frequency 0.5, presence 0.3 over 2048 history ids per row drawn
      Zipf(1.1) on ranks 1..V and mapped to token ids through a seeded permutation
  C4  1024 x 151936 bf16 N(0, 0.3^2); temperature 1.0, top-p 0.95 only
  C5  128 x 262144 fp32 N(0, 2^2) rounded to the fp16 grid (exact ties); top-k in
      {1, 64, 256, 1024} plus top-p 0.9, temperature 1.0; repetition 1.2 over a
      4096-id Zipf history

Seeds are 20261201 + config index unless given.  ``rows`` takes the first rows of
a config, or the listed rows (smaller parity cases keep each row's parameters).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from .runtime.sampling import SamplingParams

BASE_SEED = 20261201
SHAPES = {1: (8, 151936, torch.float32), 2: (64, 151936, torch.float32),
          3: (256, 151936, torch.float16), 4: (1024, 151936, torch.bfloat16),
          5: (128, 262144, torch.float32)}


@dataclass
class Workload:
    name: str
    logits: torch.Tensor              # [rows, vocab] in the config dtype
    params: list[SamplingParams]
    contexts: list[list[int]] | None
    uniforms: np.ndarray              # [rows] float64 in [0, 1)


def _peaked(gen: torch.Generator, rows: int, vocab: int, device) -> torch.Tensor:
    ranks = torch.argsort(torch.rand(rows, vocab, generator=gen, device=device), dim=1)
    base = -1.1 * torch.log(ranks.float() + 1.0)
    return base + 0.5 * torch.randn(rows, vocab, generator=gen, device=device)


def _zipf_history(rng: np.random.Generator, rows: int, length: int, vocab: int,
                  s: float = 1.1) -> list[list[int]]:
    r = np.arange(1, vocab + 1, dtype=np.float64)
    p = r ** -s
    p /= p.sum()
    perm = rng.permutation(vocab)
    ranks = rng.choice(vocab, size=(rows, length), p=p)
    ids = perm[ranks]
    return [row.tolist() for row in ids]


def make(config: int, device: str | torch.device = "cpu", rows=None,
         seed: int | None = None) -> Workload:
    B, V, dtype = SHAPES[config]
    seed = BASE_SEED + config if seed is None else seed
    gen = torch.Generator(device=device).manual_seed(seed)
    rng = np.random.default_rng(seed)
    contexts = None
    if config == 1:
        x = 3.0 * torch.randn(B, V, generator=gen, device=device)
        params = [SamplingParams()] * 4 + [SamplingParams(temperature=1.0)] * 4
    elif config == 2:
        x = _peaked(gen, B, V, device)
        params = [SamplingParams(temperature=0.7, top_k=50, top_p=0.9)] * B
    elif config == 3:
        x = _peaked(gen, B, V, device)
        pen = dict(repetition_penalty=1.1, frequency_penalty=0.5, presence_penalty=0.3)
        params = []
        for i in range(B):
            q = i * 4 // B
            k = (20, 50, 100)[i % 3]
            p = (0.8, 0.9, 0.95)[i % 3]
            if q == 0:
                params.append(SamplingParams(**pen))
            elif q == 1:
                params.append(SamplingParams(temperature=0.7, top_k=k, **pen))
            elif q == 2:
                params.append(SamplingParams(temperature=0.7, top_p=p, **pen))
            else:
                params.append(SamplingParams(temperature=0.7, top_k=k, top_p=p, **pen))
        contexts = _zipf_history(rng, B, 2048, V)
    elif config == 4:
        x = 0.3 * torch.randn(B, V, generator=gen, device=device)
        params = [SamplingParams(temperature=1.0, top_p=0.95)] * B
    elif config == 5:
        x = (2.0 * torch.randn(B, V, generator=gen, device=device)).half().float()
        params = [SamplingParams(temperature=1.0, top_k=(1, 64, 256, 1024)[i % 4], top_p=0.9,
                                 repetition_penalty=1.2) for i in range(B)]
        contexts = _zipf_history(rng, B, 4096, V)
    else:
        raise ValueError(f"unknown config {config}")
    uniforms = rng.random(B)
    logits = x.to(dtype)
    if rows is not None:
        idx = list(range(rows)) if isinstance(rows, int) else list(rows)
        logits = logits[torch.tensor(idx, device=logits.device)].contiguous()
        params = [params[i] for i in idx]
        contexts = [contexts[i] for i in idx] if contexts is not None else None
        uniforms = uniforms[idx]
    return Workload(f"C{config}", logits, params, contexts, uniforms)


def history_bytes(w: Workload) -> int:
    return 0 if w.contexts is None else 4 * sum(len(c) for c in w.contexts)
