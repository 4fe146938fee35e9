"""Benchmark of the fused MI355X sampler on the BASELINE workload (C3 by default).

One step = one fused sampler call (penalties, temperature, filters, draw) over a
[256, 151936] fp16 logits batch already resident in HBM, with the step's
parameters and penalty histories resident too.  Logits rotate through enough
distinct buffers (> 512 MB) that the 256 MB Infinity Cache cannot serve them.

Prints one JSON line: rows/s, us/step, the roofline of the dominant kernel (HIP
events around each kernel of the chain), and the reference algorithm timed on
this host's CPU (the torch-CPU restatement in oracle/, on a bounded sample).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

_REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(_REPO, "full-inference-engine_amd"))

METRIC = "rows/s + µs per sampler step at B=256,V=152k; % of HBM roofline"
HBM_PEAK_GBS = 8000.0
STAGES = ("k_penalty", "k_sample")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=3, help="workload C1..C5 (default C3)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=64)
    ap.add_argument("--ring-mb", type=int, default=640)
    return ap.parse_args()


def main() -> None:
    a = parse()
    if a.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: rows are independent and "
                          "every GPU box has one GPU; run with --gpus 1"}))
        sys.exit(2)
    import numpy as np
    import torch

    from fie_amd import workloads as W
    from fie_amd.batching.sampler import resolve_params
    from fie_amd.kernel import FusedSampler

    dev = torch.device("cuda:0")
    w = W.make(a.config, device=dev)
    B, V = w.logits.shape
    esize = w.logits.element_size()
    hp = resolve_params(w.params, V, w.uniforms, w.contexts)
    hist_total = int(hp.hist_off[-1]) if hp.apply_penalties else 0
    fs = FusedSampler(dev)
    buf = fs.step_buffers(B, hist_total)
    buf.stage(hp)
    stream = torch.cuda.current_stream(dev)
    buf.upload(stream)

    logits_bytes = B * V * esize
    nbuf = max(2, math.ceil(a.ring_mb * 2**20 / logits_bytes))
    ring = [w.logits] + [w.logits.clone() for _ in range(nbuf - 1)]
    args = [fs.build_args(x, buf, hp.apply_penalties, hist_total) for x in ring]
    fs.ensure_workspace(B, V, hist_total)
    torch.cuda.synchronize()

    def one_step(i):
        fs.launch(args[i % nbuf], hist_total)

    for i in range(a.warmup):
        one_step(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(a.steps):
        one_step(i)
    end.record(stream)
    torch.cuda.synchronize()
    ms_per_step = start.elapsed_time(end) / a.steps

    # Per-kernel durations: the same steps, one HIP event between kernels.
    nst = len(STAGES)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(nst + 1)] for _ in range(a.steps)]
    for i in range(a.steps):
        ev[i][0].record(stream)
        for s in range(nst):
            fs.launch_stage(args[i % nbuf], hist_total, s)
            ev[i][s + 1].record(stream)
    torch.cuda.synchronize()
    stage_ms = [statistics.mean(ev[i][s].elapsed_time(ev[i][s + 1]) for i in range(a.steps))
                for s in range(nst)]

    # One checked step: every row resolved on the fast path.
    buf.download(stream)
    torch.cuda.synchronize()
    out = buf.outputs()
    overflow_rows = int((out["status"] & 1 != 0).sum())
    timeout_rows = int((out["status"] & 2 != 0).sum())

    # Algorithmic bytes: logits once, penalty histories, per-row params/uniform/out.
    step_bytes = logits_bytes + 4 * hist_total + 48 * B
    # k_penalty: history ids in, one logit gathered and an (id, value) pair out per id;
    # k_sample: the logits once, the penalty pairs, per-row params and outputs.
    stage_bytes = [4 * hist_total + 2 * hist_total + 8 * hist_total,
                   logits_bytes + 8 * hist_total + 48 * B]
    dom = max(range(nst), key=lambda s: stage_ms[s])
    achieved = stage_bytes[dom] / (stage_ms[dom] * 1e-3) / 1e9
    step_gbs = step_bytes / (ms_per_step * 1e-3) / 1e9

    line = {
        "metric": METRIC,
        "value": B / (ms_per_step * 1e-3),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": ms_per_step,
        "us_per_step": ms_per_step * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": f"{w.name}: B={B}, V={V}, {str(w.logits.dtype).replace('torch.', '')} "
                        "logits, seeded synthetic (fie_amd/workloads.py)",
            "rows": B, "vocab": V, "logits_dtype": str(w.logits.dtype).replace("torch.", ""),
            "history_ids": hist_total, "logits_ring_buffers": nbuf,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": STAGES[dom],
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": None,
        },
        "step_roofline": {"achieved": step_gbs, "frac": step_gbs / HBM_PEAK_GBS,
                          "algorithmic_bytes": step_bytes},
        "stage_us": {STAGES[s]: stage_ms[s] * 1e3 for s in range(nst)},
        "overflow_rows": overflow_rows,
        "timeout_rows": timeout_rows,
    }
    if not a.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(w, a.cpu_rows)
    print(json.dumps(line), flush=True)


def cpu_baseline(w, rows: int) -> dict:
    """The reference algorithm (torch-CPU restatement, oracle/oracle.py) on a sample
    of the same workload: `rows` rows spread evenly over the batch, same params."""
    import numpy as np
    import torch

    sys.path.insert(0, os.path.join(_REPO, "oracle"))
    import oracle as O

    B = w.logits.shape[0]
    rows = min(rows, B)
    idx = np.linspace(0, B - 1, rows).round().astype(int).tolist()
    logits = w.logits[torch.tensor(idx, device=w.logits.device)].cpu()
    params = [w.params[i] for i in idx]
    ctx = [w.contexts[i] for i in idx] if w.contexts is not None else None
    uni = w.uniforms[idx]
    threads = min(os.cpu_count() or 1, 16)
    torch.set_num_threads(threads)
    O.torch_reference_step(logits, params, ctx, uni)          # warm-up
    times = []
    budget = time.perf_counter() + 20.0
    while len(times) < 3 or (time.perf_counter() < budget and len(times) < 10):
        t0 = time.perf_counter()
        O.torch_reference_step(logits, params, ctx, uni)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return {"value": rows / t, "unit": "rows/s", "cores": threads, "kind": "port",
            "sample": f"{rows} of {B} rows of {w.name} (same params and histories), "
                      f"median of {len(times)} steps, {t * 1e3:.1f} ms/step, torch "
                      f"{torch.__version__} CPU, {threads} threads"}


if __name__ == "__main__":
    main()
