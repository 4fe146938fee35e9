"""Benchmark of the fused MI355X sampler on the BASELINE workload (C3 by default).

One step = one fused sampler call (penalties, temperature, top-k / top-p / min-p,
draw, logprobs) over one [B, V] logits batch already resident in HBM, with the
step's parameters and penalty histories resident too: the kernels k_prep, k_scan,
k_finish and, for batches with more rows than CUs, k_deep (idle when no row needs
the full-row path).  Logits rotate through enough distinct buffers (> 512 MB) that the 256 MB
Infinity Cache cannot serve them.

Prints one JSON line: rows/s and us/step for the headline config, the roofline of
the dominant kernel (HIP events on the launch stream around each kernel), the other
configs' times, the end-to-end BatchedSampler.sample() time (host packing, upload,
kernels, download), and the reference algorithm timed on this host's CPU (the
torch-CPU restatement in oracle/, on a bounded sample of rows).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time

_REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(_REPO, "full-inference-engine_amd"))

METRIC = "rows/s + µs per sampler step at B=256,V=152k; % of HBM roofline"
HBM_PEAK_GBS = 8000.0
STAGES = ("k_prep", "k_scan", "k_finish", "k_deep")   # fie_sampler_stage 0, 1, 2, 3


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=3, help="headline workload C1..C5 (default C3)")
    ap.add_argument("--others", default="1,2,4,5", help="other configs to time ('' for none)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--full-row-only", action="store_true",
                    help="time only the full-row path latencies (for a kernel trace of them)")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--ring-mb", type=int, default=640)
    ap.add_argument("--lmhead-dim", type=int, default=4096,
                    help="hidden size of the fused lm_head measurement (0 to skip)")
    return ap.parse_args()


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def measured_traffic(kernel: str, config: int):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (scaled by the copy calibration it states), or None."""
    path = os.path.join(_REPO, "profiles", f"k_scan_C{config}_hbm_traffic.md")
    try:
        with open(path, encoding="utf-8") as f:
            for line in f:
                cells = [c.strip() for c in line.strip().strip("|").split("|")]
                if len(cells) == 6 and cells[0] == f"`{kernel}`":
                    return round((float(cells[4]) + float(cells[5])) * 1e6)
    except (OSError, ValueError):
        pass
    return None


KSCAN_SOURCES = ("scan.h", "common.h", "k_scan.hip")


def kscan_sources_hash() -> str:
    """First 16 hex digits of the sha256 of k_scan's sources, as the committed
    counter summary records the ones it measured."""
    import hashlib

    csrc = os.path.join(_REPO, "full-inference-engine_amd", "csrc")
    h = hashlib.sha256()
    for name in KSCAN_SOURCES:
        with open(os.path.join(csrc, name), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def traffic_sources(config: int):
    """The k_scan sources hash the committed FETCH/WRITE summary was measured on."""
    path = os.path.join(_REPO, "profiles", f"k_scan_C{config}_hbm_traffic.md")
    try:
        with open(path, encoding="utf-8") as f:
            for line in f:
                if line.startswith("k_scan sources measured") and "`" in line:
                    return line.split("`")[1]
    except OSError:
        pass
    return None


def algorithmic_bytes(w, hp) -> dict:
    """Bytes one step must move at least (one read of the logits), per kernel.

    k_scan: the logits once, each penalised row's history ids once, per-row params;
            its outputs (tile partials) are counted too.
    step:   the logits once, the history once, per-row params in and results out
            (48 bytes per row), as BASELINE.md's table counts them.
    """
    B, V = w.logits.shape
    esize = w.logits.element_size()
    hist = 4 * int(hp.hist_off[-1]) if hp.apply_penalties else 0
    logits = B * V * esize
    return {"logits": logits, "history": hist,
            "k_scan": logits + hist + 48 * B,
            "step": logits + hist + 48 * B}


def time_config(config: int, steps: int, warmup: int, ring_mb: int, dev):
    import numpy as np
    import torch

    from fie_amd import _lib
    from fie_amd import workloads as W
    from fie_amd.batching.sampler import resolve_params
    from fie_amd.kernel import FusedSampler

    w = W.make(config, device=dev)
    B, V = w.logits.shape
    hp = resolve_params(w.params, V, w.uniforms, w.contexts)
    fs = FusedSampler(dev)
    hist_total = int(hp.hist_off[-1]) if hp.apply_penalties else 0
    buf = fs.step_buffers(B, hist_total)
    buf.stage(hp)
    stream = torch.cuda.current_stream(dev)
    buf.upload(stream)
    logits_bytes = w.logits.numel() * w.logits.element_size()
    nbuf = max(2, math.ceil(ring_mb * 2**20 / logits_bytes))
    ring = [w.logits] + [w.logits.clone() for _ in range(nbuf - 1)]
    args = [fs.build_args(x, buf, hp) for x in ring]
    fs.ensure_workspace(B, V)
    torch.cuda.synchronize()

    for i in range(warmup):
        fs.launch(args[i % nbuf])
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for i in range(steps):
        fs.launch(args[i % nbuf])
    t1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = t0.elapsed_time(t1) / steps

    # Per-kernel durations: each kernel alone, launched `steps` times back to back on
    # the kernels' stream between one pair of HIP events (a pair per launch would add
    # the event's own few microseconds to every kernel).  Each stage reads what the
    # previous stages left in the workspace, so they run in chain order.
    nst = len(STAGES)
    stage_ms = []
    for s in range(nst):
        fs.launch_stage(args[0], s)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(steps):
            fs.launch_stage(args[i % nbuf], s)
        e1.record(stream)
        torch.cuda.synchronize()
        stage_ms.append(e0.elapsed_time(e1) / steps)
    if not hp.apply_penalties:
        stage_ms[0] = 0.0                                   # k_prep is not launched
    if B <= torch.cuda.get_device_properties(dev).multi_processor_count:
        stage_ms[3] = 0.0                                   # k_finish settles every row: no k_deep

    # One checked step: status bits of the rows (the exact path is informational).
    buf.download(stream)
    torch.cuda.synchronize()
    out = buf.outputs()
    exact_rows = int((out["status"] & _lib.FIE_ROW_EXACT_PATH != 0).sum())
    return {
        "w": w, "hp": hp, "B": B, "V": V, "ms_per_step": ms_per_step,
        "stage_ms": dict(zip(STAGES, stage_ms)), "exact_path_rows": exact_rows,
        "ring": nbuf, "bytes": algorithmic_bytes(w, hp), "fs": fs,
    }


def full_row_us(dev, steps: int = 50) -> dict:
    """Step latency when rows need the full-row path (the draw lies past the streamed
    candidates): C1's plain rows (N(0, 3^2) fp32 logits, temperature 1) with draws
    deep in the tail, one row alone and the four together."""
    import numpy as np
    import torch

    from fie_amd import _lib
    from fie_amd import workloads as W
    from fie_amd.batching.sampler import resolve_params
    from fie_amd.kernel import FusedSampler

    w = W.make(1)
    fs = FusedSampler(dev)
    stream = torch.cuda.current_stream(dev)
    res = {}
    for name, rows in (("one_row", [4]), ("four_rows", [4, 5, 6, 7])):
        x = w.logits[rows].to(dev)
        params = [w.params[r] for r in rows]
        u = np.array([0.95, 0.96, 0.97, 0.98])[:len(rows)]
        hp = resolve_params(params, x.shape[1], u, None)
        buf = fs.step_buffers(len(rows), 0)
        buf.stage(hp)
        buf.upload(stream)
        args = fs.build_args(x, buf, hp)
        for _ in range(5):
            fs.launch(args)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            fs.launch(args)
        e1.record(stream)
        buf.download(stream)
        torch.cuda.synchronize()
        out = buf.outputs()
        res[name] = {"us_per_step": e0.elapsed_time(e1) / steps * 1e3,
                     "exact_path_rows": int((out["status"] & _lib.FIE_ROW_EXACT_PATH != 0).sum())}
    return res


def end_to_end_ms(w, dev, reps: int = 20) -> float:
    """BatchedSampler.sample() as the engine calls it, per decode step: parameter
    resolution, the appended context token per row (the contexts stay on the
    device between steps), upload, the kernels, download and the host lists."""
    import torch

    from fie_amd.batching.sampler import BatchedSampler

    s = BatchedSampler(dev, generator_seed=0)
    x = w.logits
    ids = [f"r{i}" for i in range(x.shape[0])]
    ctx = [list(c) for c in w.contexts] if w.contexts is not None else None
    res = s.sample(x, w.params, ctx, ids)
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        if ctx is not None:
            for c, t in zip(ctx, res.token_ids):
                c.append(t)
        t = time.perf_counter()
        res = s.sample(x, w.params, ctx, ids)
        times.append(time.perf_counter() - t)
    return statistics.median(times) * 1e3


def cpu_baseline(w, seconds: float) -> dict:
    """The reference algorithm (torch-CPU restatement, oracle/oracle.py) on a sample of
    the same workload: rows spread evenly over the batch, same params and histories,
    as many rows as fit about `seconds` of CPU work."""
    import numpy as np
    import torch

    sys.path.insert(0, os.path.join(_REPO, "oracle"))
    import oracle as O

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    B = w.logits.shape[0]

    def sample(rows):
        idx = np.linspace(0, B - 1, rows).round().astype(int).tolist()
        logits = w.logits[torch.tensor(idx, device=w.logits.device)].cpu()
        params = [w.params[i] for i in idx]
        ctx = [w.contexts[i] for i in idx] if w.contexts is not None else None
        return logits, params, ctx, w.uniforms[idx]

    probe = sample(min(8, B))
    t = time.perf_counter()
    O.torch_reference_step(*probe)
    per_row = (time.perf_counter() - t) / probe[0].shape[0]
    rows = int(max(8, min(B, seconds / 4 / max(per_row, 1e-6))))
    data = sample(rows)
    O.torch_reference_step(*data)                        # warm-up
    times = []
    budget = time.perf_counter() + seconds
    while len(times) < 3 or (time.perf_counter() < budget and len(times) < 10):
        t = time.perf_counter()
        O.torch_reference_step(*data)
        times.append(time.perf_counter() - t)
    med = statistics.median(times)
    return {"value": rows / med, "unit": "rows/s", "cores": threads, "kind": "port",
            "sample": f"{rows} of {B} rows of {w.name} (same params and histories), median of "
                      f"{len(times)} steps, {med * 1e3:.1f} ms/step; torch {torch.__version__} CPU, "
                      f"{threads} threads on {cpu_model()}"}


def time_lmhead(w, dev, H: int, steps: int = 20) -> dict:
    """The fused lm_head (fie_sampler_lmhead_sample) against the two-step path it
    replaces: the library GEMM torch.matmul runs for the model's output layer, then
    fie_sampler_sample.  Same rows, parameters and histories as the headline
    workload, fp16 operands.  Hidden states and weight rows are built so the logits
    have the workload's peaked shape (-1.1 ln(rank + 1) + N(0, 0.5^2)): random
    matrices would give flat logits, and every top-p row would take the full-row path."""
    import torch
    from fie_amd.batching.sampler import resolve_params
    from fie_amd.kernel import FusedSampler

    B, V = w.logits.shape
    dt = torch.float16
    g = torch.Generator(device=dev).manual_seed(20261201)
    d = torch.randn(H, generator=g, device=dev)
    d /= d.norm()
    hidden = (d[None, :] + 0.01 * torch.randn(B, H, generator=g, device=dev) / H ** 0.5).to(dt)
    ranks = torch.randperm(V, generator=g, device=dev).float()
    scale = -1.1 * torch.log(ranks + 1.0)
    weight = (scale[:, None] * d[None, :] + 0.5 * torch.randn(V, H, generator=g, device=dev)).to(dt)
    hp = resolve_params(w.params, V, w.uniforms, w.contexts)
    fs = FusedSampler(dev)
    logits = torch.empty(B, V, dtype=dt, device=dev)
    _, args, _, _ = fs.lmhead_step(hidden, weight, hp, logits)
    exact_rows = 0

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(steps):
            fn()
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) * 1e3 / steps

    fused_step = timed(lambda: fs.launch_lmhead(args, hidden, weight))
    kernel = timed(lambda: fs.launch_lmhead(args, hidden, weight, kernel_only=True))
    gemm = timed(lambda: torch.matmul(hidden, weight.T, out=logits))
    scan = timed(lambda: fs.launch_stage(args, 1))
    two_step = timed(lambda: (torch.matmul(hidden, weight.T, out=logits), fs.launch(args)))
    out, _, _ = fs.step(logits, hp)
    exact_rows = int(((out["status"] & 1) != 0).sum())
    wbytes = V * H * 2
    r = {"hidden_dim": H, "rows": B, "vocab": V, "dtype": "float16",
         "fused_step_us": fused_step, "two_step_us": two_step,
         "k_lmhead_us": kernel, "library_gemm_us": gemm, "k_scan_us": scan,
         "k_lmhead_weight_gbs": wbytes / (kernel * 1e-6) / 1e9,
         "k_lmhead_tflops": 2 * B * H * V / (kernel * 1e-6) / 1e12,
         "exact_path_rows": exact_rows}
    del weight, hidden, logits
    torch.cuda.empty_cache()
    return r


def main() -> None:
    a = parse()
    if a.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU (every GPU box here has one); "
                          "rows are independent, so more GPUs shard rows without "
                          "communication; run with --gpus 1"}))
        sys.exit(2)
    import torch

    dev = torch.device("cuda:0")
    if a.full_row_only:
        print(json.dumps({"full_row_path": full_row_us(dev, a.steps)}), flush=True)
        return
    main_r = time_config(a.config, a.steps, a.warmup, a.ring_mb, dev)
    w = main_r["w"]
    B, V = main_r["B"], main_r["V"]
    ms = main_r["ms_per_step"]
    st = main_r["stage_ms"]
    dom = max(STAGES, key=lambda s: st[s])
    by = main_r["bytes"]
    dom_bytes = by[dom] if dom in by else by["step"]
    achieved = dom_bytes / (st[dom] * 1e-3) / 1e9
    step_gbs = by["step"] / (ms * 1e-3) / 1e9
    ldt = str(w.logits.dtype).replace("torch.", "")

    line = {
        "metric": METRIC,
        "value": B / (ms * 1e-3),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": ms,
        "us_per_step": ms * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"{ldt} logits, f32 arithmetic, exact integer masses",
        "data": "synthetic, seeded (fie_amd/workloads.py)",
        "config": {
            "workload": f"{w.name}: B={B}, V={V}, {ldt} logits, mixed per-row greedy/top-k/"
                        "top-p/penalties" if a.config == 3 else f"{w.name}: B={B}, V={V}, {ldt}",
            "rows": B, "vocab": V, "logits_dtype": ldt,
            "history_ids": int(main_r["hp"].hist_off[-1]) if main_r["hp"].apply_penalties else 0,
            "logits_ring_buffers": main_r["ring"],
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dom,
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": measured_traffic(dom, a.config),
            "traffic_source": f"profiles/k_scan_C{a.config}_hbm_traffic.md (rocprofv3 --pmc, scaled)",
            # the summary is of the k_scan sources it names; false: they changed since
            "traffic_matches_sources": traffic_sources(a.config) == kscan_sources_hash(),
            "algorithmic_bytes": dom_bytes,
        },
        "step_roofline": {"achieved": step_gbs, "frac": step_gbs / HBM_PEAK_GBS,
                          "algorithmic_bytes": by["step"]},
        "stage_us": {k: v * 1e3 for k, v in st.items()},
        "exact_path_rows": main_r["exact_path_rows"],
    }
    del main_r
    others = {}
    for c in [int(x) for x in a.others.split(",") if x.strip()]:
        if c == a.config:
            continue
        r = time_config(c, max(20, a.steps // 4), 5, a.ring_mb, dev)
        gbs = r["bytes"]["step"] / (r["ms_per_step"] * 1e-3) / 1e9
        others[f"C{c}"] = {"rows": r["B"], "vocab": r["V"],
                           "dtype": str(r["w"].logits.dtype).replace("torch.", ""),
                           "us_per_step": r["ms_per_step"] * 1e3,
                           "rows_per_s": r["B"] / (r["ms_per_step"] * 1e-3),
                           "stage_us": {k: v * 1e3 for k, v in r["stage_ms"].items()},
                           "step_frac_hbm": gbs / HBM_PEAK_GBS,
                           "exact_path_rows": r["exact_path_rows"]}
        del r
        torch.cuda.empty_cache()
    line["other_configs"] = others
    try:
        line["full_row_path"] = full_row_us(dev)
    except Exception as e:  # report, never hide the main line
        line["full_row_path"] = f"failed: {e}"
    if a.lmhead_dim:
        try:
            line["lmhead_fused"] = time_lmhead(w, dev, a.lmhead_dim)
        except Exception as e:  # report, never hide the main line
            line["lmhead_fused"] = f"failed: {e}"
    try:
        line["end_to_end_ms"] = end_to_end_ms(w, dev)
    except Exception as e:  # report, never hide the main line
        line["end_to_end_ms"] = f"failed: {e}"
    if not a.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(w, a.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
