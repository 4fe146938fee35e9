"""Device-level driver of the fused sampler: workspace, packed parameter upload,
launches on the current stream, packed result download.

``FusedSampler`` is what ``BatchedSampler`` (the reference's call surface) sits on;
tests and the benchmark use it directly to time the kernels on resident inputs.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from ._lib import LP_COLS, SamplerArgs, Workspace

_DTYPES = {torch.float32: _lib.FIE_F32, torch.float16: _lib.FIE_F16,
           torch.bfloat16: _lib.FIE_BF16}

# Per-row parameter arrays in upload order.
PARAM_FIELDS = (
    ("scale", np.float32), ("top_k", np.int32), ("top_p", np.float32), ("min_p", np.float32),
    ("flags", np.int32), ("logprobs", np.int32), ("uniform", np.float64),
    ("rep", np.float32), ("pres", np.float32), ("freq", np.float32),
)
# Per-row outputs in download order.  `status` is uploaded too (as zeros: the
# kernels OR bits into it) and sits first so one copy each way covers it.
OUTPUT_FIELDS = (
    ("status", np.int32, 1), ("tokens", np.int64, 1), ("tk_key", np.uint32, 1),
    ("cut_comp", np.uint64, 1), ("row_max", np.float32, 1), ("kept_mass", np.uint64, 1),
    ("row_mass", np.uint64, 1), ("chosen_lp", np.float32, 1),
    ("top_ids", np.int64, LP_COLS), ("top_lp", np.float32, LP_COLS),
)

FLAG_GREEDY = 1
FLAG_PENALTY = 2


def _align(x: int, a: int = 256) -> int:
    return (x + a - 1) // a * a


@dataclass
class HostParams:
    """Resolved per-row parameters (numpy), what the C ABI consumes."""

    scale: np.ndarray
    top_k: np.ndarray
    top_p: np.ndarray
    min_p: np.ndarray
    flags: np.ndarray
    logprobs: np.ndarray
    uniform: np.ndarray
    rep: np.ndarray
    pres: np.ndarray
    freq: np.ndarray
    hist_off: np.ndarray          # int64 [rows + 1]
    hist_ids: np.ndarray          # int32 [hist_off[-1]]
    apply_penalties: bool

    @property
    def rows(self) -> int:
        return int(self.scale.shape[0])


class DeviceStep:
    """One packed device block holding a step's parameters and outputs."""

    def __init__(self, rows: int, hist_total: int, device: torch.device):
        self.rows = rows
        self.hist_total = hist_total
        offs, o = {}, 0
        for name, dt in PARAM_FIELDS:
            offs[name] = o
            o = _align(o + rows * np.dtype(dt).itemsize)
        offs["hist_off"] = o
        o = _align(o + (rows + 1) * 8)
        offs["hist_ids"] = o
        o = _align(o + max(hist_total, 1) * 4)
        self.out_begin = o
        for name, dt, width in OUTPUT_FIELDS:
            offs[name] = o
            o = _align(o + rows * width * np.dtype(dt).itemsize)
        self.param_bytes = offs[OUTPUT_FIELDS[1][0]]      # params + zeroed status
        self.total = o
        self.offs = offs
        self.dev = torch.empty(self.total, dtype=torch.uint8, device=device)
        self.host = torch.empty(self.total, dtype=torch.uint8, pin_memory=True)
        self.host_np = self.host.numpy()
        self.base = self.dev.data_ptr()

    def host_view(self, name: str, dtype, count: int) -> np.ndarray:
        o = self.offs[name]
        return self.host_np[o:o + count * np.dtype(dtype).itemsize].view(dtype)

    def ptr(self, name: str) -> int:
        return self.base + self.offs[name]

    def device_view(self, name: str, dtype: torch.dtype, count: int) -> torch.Tensor:
        o = self.offs[name]
        size = torch.tensor([], dtype=dtype).element_size()
        return self.dev[o:o + count * size].view(dtype)

    def stage(self, hp: HostParams) -> None:
        for name, dt in PARAM_FIELDS:
            self.host_view(name, dt, self.rows)[:] = getattr(hp, name)
        self.host_view("hist_off", np.int64, self.rows + 1)[:] = hp.hist_off
        n = int(hp.hist_off[-1])
        if n:
            self.host_view("hist_ids", np.int32, n)[:] = hp.hist_ids
        self.host_view("status", np.int32, self.rows)[:] = 0

    def upload(self, stream: torch.cuda.Stream) -> None:
        with torch.cuda.stream(stream):
            self.dev[:self.param_bytes].copy_(self.host[:self.param_bytes], non_blocking=True)

    def download(self, stream: torch.cuda.Stream) -> None:
        with torch.cuda.stream(stream):
            self.host[self.out_begin:].copy_(self.dev[self.out_begin:], non_blocking=True)

    def outputs(self) -> dict[str, np.ndarray]:
        return {name: self.host_view(name, dt, self.rows * w).reshape(self.rows, w)
                if w > 1 else self.host_view(name, dt, self.rows)
                for name, dt, w in OUTPUT_FIELDS}


class FusedSampler:
    """Owns the workspace and launches the HIP sampler on one device."""

    def __init__(self, device: torch.device | str):
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise RuntimeError(
                "the MI355X sampler runs on a HIP device; got device "
                f"{self.device} (there is no CPU path)")
        self.lib = _lib.load()
        self._ws_tensor: torch.Tensor | None = None
        self._ws = Workspace()
        self._ws_dims = (0, 0, 0)
        self._epoch = 0
        self._steps: dict[tuple[int, int], DeviceStep] = {}

    # ------------------------------------------------------------------ workspace
    def ensure_workspace(self, rows: int, vocab: int, hist_total: int) -> Workspace:
        r0, v0, h0 = self._ws_dims
        if rows <= r0 and vocab <= v0 and hist_total <= h0:
            return self._ws
        rows, vocab, hist = max(rows, r0), max(vocab, v0), max(hist_total, h0, 1)
        nbytes = int(self.lib.fie_sampler_workspace_size(rows, vocab, hist))
        self._ws_tensor = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        self._ws = Workspace(self._ws_tensor.data_ptr(), nbytes, rows, vocab, hist)
        self._ws_dims = (rows, vocab, hist)
        _lib.check(self.lib.fie_sampler_workspace_init(ctypes.byref(self._ws), self._stream_ptr()),
                   "fie_sampler_workspace_init")
        return self._ws

    def reset_workspace(self) -> None:
        """Restore the workspace invariants after a failed call."""
        if self._ws_tensor is not None:
            _lib.check(self.lib.fie_sampler_workspace_init(ctypes.byref(self._ws),
                                                           self._stream_ptr()),
                       "fie_sampler_workspace_init")

    def _stream_ptr(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def step_buffers(self, rows: int, hist_total: int) -> DeviceStep:
        key = (rows, _align(max(hist_total, 1), 4096))
        buf = self._steps.get(key)
        if buf is None:
            if len(self._steps) > 32:
                self._steps.clear()
            buf = DeviceStep(rows, key[1], self.device)
            self._steps[key] = buf
        return buf

    # ------------------------------------------------------------------ launches
    @staticmethod
    def _logits_info(logits: torch.Tensor) -> tuple[torch.Tensor, int]:
        if logits.dtype not in _DTYPES:
            logits = logits.float()
        if logits.stride(1) != 1 or logits.stride(0) < logits.shape[1]:
            logits = logits.contiguous()
        return logits, _DTYPES[logits.dtype]

    def build_args(self, logits: torch.Tensor, buf: DeviceStep, apply_penalties: bool,
                   hist_total: int) -> SamplerArgs:
        logits, dt = self._logits_info(logits)
        rows, vocab = logits.shape
        self._epoch += 1
        a = SamplerArgs()
        a.logits = logits.data_ptr()
        a.dtype = dt
        a.rows = rows
        a.vocab = vocab
        a.lp_cols = LP_COLS
        a.row_stride = logits.stride(0)
        a.scale, a.top_k, a.top_p, a.min_p = (buf.ptr("scale"), buf.ptr("top_k"),
                                              buf.ptr("top_p"), buf.ptr("min_p"))
        a.flags, a.logprobs, a.uniform = buf.ptr("flags"), buf.ptr("logprobs"), buf.ptr("uniform")
        a.apply_penalties = 1 if apply_penalties else 0
        a.repetition, a.presence, a.frequency = buf.ptr("rep"), buf.ptr("pres"), buf.ptr("freq")
        a.hist_offsets, a.hist_ids = buf.ptr("hist_off"), buf.ptr("hist_ids")
        a.hist_total = hist_total
        a.epoch = self._epoch
        a.tokens, a.status, a.tk_key = buf.ptr("tokens"), buf.ptr("status"), buf.ptr("tk_key")
        a.cut_comp, a.row_max = buf.ptr("cut_comp"), buf.ptr("row_max")
        a.kept_mass, a.row_mass = buf.ptr("kept_mass"), buf.ptr("row_mass")
        a.chosen_logprob = buf.ptr("chosen_lp")
        a.top_ids, a.top_logprobs = buf.ptr("top_ids"), buf.ptr("top_lp")
        a._keep = logits  # the converted tensor must outlive the launch
        return a

    def launch(self, args: SamplerArgs, hist_total: int) -> None:
        ws = self.ensure_workspace(args.rows, args.vocab, hist_total)
        rc = self.lib.fie_sampler_sample(ctypes.byref(args), ctypes.byref(ws), self._stream_ptr())
        if rc != _lib.FIE_OK:
            self.reset_workspace()
        _lib.check(rc, "fie_sampler_sample")

    def launch_stage(self, args: SamplerArgs, hist_total: int, stage: int) -> None:
        ws = self.ensure_workspace(args.rows, args.vocab, hist_total)
        rc = self.lib.fie_sampler_stage(ctypes.byref(args), ctypes.byref(ws), stage,
                                        self._stream_ptr())
        _lib.check(rc, f"fie_sampler_stage({stage})")

    def resolve_overflow(self, args: SamplerArgs, rows: list[int], hist_total: int) -> None:
        ws = self.ensure_workspace(args.rows, args.vocab, hist_total)
        lst = torch.tensor(rows, dtype=torch.int32, device=self.device)
        rc = self.lib.fie_sampler_resolve_overflow(ctypes.byref(args), lst.data_ptr(), len(rows),
                                                   ctypes.byref(ws), self._stream_ptr())
        _lib.check(rc, "fie_sampler_resolve_overflow")
        self._overflow_rows = lst  # keep alive until the stream passes it

    def kept(self, args: SamplerArgs, want_probs: bool = True):
        rows, vocab = args.rows, args.vocab
        kept = torch.empty((rows, vocab), dtype=torch.uint8, device=self.device)
        probs = torch.empty((rows, vocab), dtype=torch.float32, device=self.device) \
            if want_probs else None
        ws = self._ws
        rc = self.lib.fie_sampler_kept(ctypes.byref(args), kept.data_ptr(),
                                       probs.data_ptr() if probs is not None else None,
                                       ctypes.byref(ws), self._stream_ptr())
        _lib.check(rc, "fie_sampler_kept")
        return kept, probs

    def argmax(self, logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        logits, dt = self._logits_info(logits)
        rows, vocab = logits.shape
        ws = self.ensure_workspace(rows, vocab, 1)
        if out is None:
            out = torch.empty(rows, dtype=torch.int64, device=self.device)
        rc = self.lib.fie_sampler_argmax(logits.data_ptr(), dt, rows, vocab, logits.stride(0),
                                         out.data_ptr(), ctypes.byref(ws), self._stream_ptr())
        _lib.check(rc, "fie_sampler_argmax")
        return out

    def cexp(self, values: torch.Tensor) -> torch.Tensor:
        values = values.contiguous().float()
        out = torch.empty_like(values)
        _lib.check(self.lib.fie_sampler_cexp(values.data_ptr(), out.data_ptr(), values.numel(),
                                             self._stream_ptr()), "fie_sampler_cexp")
        return out

    # ------------------------------------------------------------------ a full step
    def step(self, logits: torch.Tensor, hp: HostParams, sync: bool = True):
        """Upload, launch, download; returns the output arrays (after one sync)."""
        rows = logits.shape[0]
        hist_total = int(hp.hist_off[-1]) if hp.apply_penalties else 0
        buf = self.step_buffers(rows, hist_total)
        buf.stage(hp)
        stream = torch.cuda.current_stream(self.device)
        buf.upload(stream)
        args = self.build_args(logits, buf, hp.apply_penalties, hist_total)
        self.launch(args, hist_total)
        buf.download(stream)
        stream.synchronize()
        out = buf.outputs()
        over = np.nonzero(out["status"])[0]
        if over.size:
            if (out["status"] & _lib.FIE_ROW_TIMEOUT).any():
                self.reset_workspace()
            self.resolve_overflow(args, [int(r) for r in over], hist_total)
            buf.download(stream)
            stream.synchronize()
            out = buf.outputs()
        return out, args, buf
