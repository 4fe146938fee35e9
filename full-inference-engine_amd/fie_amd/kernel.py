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

# Per-row parameter arrays in upload order: (name, dtype, values per row).
PARAM_FIELDS = (
    ("scale", np.float32, 1), ("top_k", np.int32, 1), ("top_p", np.float32, 1),
    ("min_p", np.float32, 1), ("flags", np.int32, 1), ("logprobs", np.int32, 1),
    ("uniform", np.float64, 1), ("rng", np.uint64, 3),
    ("rep", np.float32, 1), ("pres", np.float32, 1), ("freq", np.float32, 1),
    ("hist_invalid", np.int32, 1),
)
# Per-row outputs in download order: (name, dtype, values per row).
OUTPUT_FIELDS = (
    ("status", np.int32, 1), ("tokens", np.int64, 1), ("tk_key", np.uint32, 1),
    ("cut_comp", np.uint64, 1), ("row_max", np.float32, 1), ("kept_mass", np.uint64, 2),
    ("row_mass", np.uint64, 2), ("chosen_lp", np.float32, 1),
    ("top_ids", np.int64, LP_COLS), ("top_lp", np.float32, LP_COLS),
)

# Columns that come from the cached per-batch parameter table (never written after
# they are built), so an identical object means identical contents.
_TABLE_FIELDS = frozenset(("scale", "top_k", "top_p", "min_p", "flags", "logprobs", "rep", "pres", "freq"))

FLAG_GREEDY = _lib.FIE_FLAG_GREEDY
FLAG_PENALTY = _lib.FIE_FLAG_PENALTY
# Batches of at most this many rows run k_finish's span helpers, in a workspace
# sized for exactly this many rows (kHelpRows in the library).
HELP_ROWS = 16


def _align(x: int, a: int = 256) -> int:
    return (x + a - 1) // a * a


def u128(pair) -> int:
    """A (low, high) uint64 pair as a Python int."""
    return int(pair[0]) | (int(pair[1]) << 64)


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
    hist_invalid: np.ndarray | None = None   # int32 [rows], rows with ids >= vocab
    max_row_hist: int = 0
    rng: np.ndarray | None = None            # uint64 [rows, 3]: on-device draws (key0, key1, counter)
    # A device-resident history (DeviceHistory): hist_off then holds the rows'
    # starts [rows] and hist_ends their ends in hist_store.ids; hist_write_dst/src
    # are the appended tokens to write there before the step.
    hist_ends: np.ndarray | None = None
    hist_store: object | None = None
    hist_write_dst: np.ndarray | None = None
    hist_write_src: np.ndarray | None = None

    def tail_ints(self) -> int:
        """int32 words of the step block's variable tail: the CSR ids, or the
        (int64 position, int32 id) pairs of a device-resident history's appends."""
        if not self.apply_penalties:
            return 0
        if self.hist_ends is not None:
            return 3 * int(self.hist_write_dst.shape[0]) + 2
        return int(self.hist_off[-1])

    @property
    def rows(self) -> int:
        return int(self.scale.shape[0])


class DeviceStep:
    """One packed device block holding a step's parameters, history and outputs,
    with a pinned host mirror: one upload and one download per step."""

    def __init__(self, rows: int, hist_cap: int, device: torch.device):
        self.rows = rows
        self.hist_cap = hist_cap
        offs, o = {}, 0
        for name, dt, width in PARAM_FIELDS:
            offs[name] = o
            o = _align(o + max(rows, 1) * width * np.dtype(dt).itemsize)
        offs["hist_off"] = o
        o = _align(o + (rows + 1) * 8)
        offs["hist_end"] = o
        o = _align(o + max(rows, 1) * 8)
        offs["hist_ids"] = o
        o = _align(o + max(hist_cap, 1) * 4)
        self.out_begin = o
        for name, dt, width in OUTPUT_FIELDS:
            offs[name] = o
            o = _align(o + max(rows, 1) * width * np.dtype(dt).itemsize)
        self.total = o
        self.offs = offs
        self.dev = torch.empty(self.total, dtype=torch.uint8, device=device)
        self.host = torch.empty(self.total, dtype=torch.uint8, pin_memory=True)
        self.host_np = self.host.numpy()
        self.base = self.dev.data_ptr()
        self.param_bytes = self.out_begin
        self._staged: dict[str, np.ndarray] = {}

    def host_view(self, name: str, dtype, count: int) -> np.ndarray:
        o = self.offs[name]
        return self.host_np[o:o + count * np.dtype(dtype).itemsize].view(dtype)

    def ptr(self, name: str) -> int:
        return self.base + self.offs[name]

    def stage(self, hp: HostParams) -> None:
        # a per-row column staged at the last step and passed again (the same object:
        # the parameter table of an unchanged batch, which nothing writes) is already
        # in place; draws and the history fields are copied every step
        last = self._staged
        for name, dt, width in PARAM_FIELDS:
            src = getattr(hp, name)
            if src is None:
                continue
            if name in _TABLE_FIELDS:
                if last.get(name) is src:
                    continue
                last[name] = src
            self.host_view(name, dt, self.rows * width)[:] = np.asarray(src).reshape(-1)
        self.host_view("hist_off", np.int64, len(hp.hist_off))[:] = hp.hist_off
        if hp.hist_ends is not None:
            # device-resident history: row ranges, then the appended (position, id) pairs
            self.host_view("hist_end", np.int64, self.rows)[:] = hp.hist_ends
            n = int(hp.hist_write_dst.shape[0])
            o = self.offs["hist_ids"]
            self.host_np[o:o + 8 * n].view(np.int64)[:] = hp.hist_write_dst
            self.host_np[o + 8 * n:o + 12 * n].view(np.int32)[:] = hp.hist_write_src
            self.param_bytes = o + 12 * n
            return
        n = int(hp.hist_off[-1])
        if n:
            self.host_view("hist_ids", np.int32, n)[:] = hp.hist_ids
        # history ids are the tail of the parameter block: upload only what is used
        self.param_bytes = self.offs["hist_ids"] + 4 * n

    def upload(self, stream: torch.cuda.Stream) -> None:
        if stream == torch.cuda.current_stream(self.dev.device):
            self.dev[:self.param_bytes].copy_(self.host[:self.param_bytes], non_blocking=True)
            return
        with torch.cuda.stream(stream):
            self.dev[:self.param_bytes].copy_(self.host[:self.param_bytes], non_blocking=True)

    def download(self, stream: torch.cuda.Stream) -> None:
        if stream == torch.cuda.current_stream(self.dev.device):
            self.host[self.out_begin:].copy_(self.dev[self.out_begin:], non_blocking=True)
            return
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
        # Two workspaces: batches of at most HELP_ROWS rows use one sized for
        # HELP_ROWS, which also holds the span helpers' arrays (the library runs
        # k_finish's helpers only in such a workspace); larger batches use one that
        # grows with the largest batch seen.
        self._wss: dict[bool, tuple[torch.Tensor | None, Workspace, tuple[int, int]]] = {
            True: (None, Workspace(), (0, 0)), False: (None, Workspace(), (0, 0))}
        self._steps: dict[tuple[int, int], DeviceStep] = {}

    # ------------------------------------------------------------------ workspace
    def ensure_workspace(self, rows: int, vocab: int) -> Workspace:
        small = rows <= HELP_ROWS
        tensor, ws, (r0, v0) = self._wss[small]
        if rows <= r0 and vocab <= v0:
            return ws
        rows = HELP_ROWS if small else max(rows, r0, 1)
        vocab = max(vocab, v0)
        nbytes = int(self.lib.fie_sampler_workspace_size(rows, vocab))
        if nbytes == 0:
            raise ValueError(f"unsupported sampler shape rows={rows} vocab={vocab} "
                             f"(vocab must be in [1, {_lib.MAX_VOCAB}])")
        tensor = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        ws = Workspace(tensor.data_ptr(), nbytes, rows, vocab)
        self._wss[small] = (tensor, ws, (rows, vocab))
        return ws

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

    def build_args(self, logits: torch.Tensor, buf: DeviceStep, hp: HostParams) -> SamplerArgs:
        logits, dt = self._logits_info(logits)
        rows, vocab = logits.shape
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
        a.apply_penalties = 1 if hp.apply_penalties else 0
        a.max_row_hist = int(hp.max_row_hist)
        a.repetition, a.presence, a.frequency = buf.ptr("rep"), buf.ptr("pres"), buf.ptr("freq")
        a.hist_offsets, a.hist_ids = buf.ptr("hist_off"), buf.ptr("hist_ids")
        if hp.hist_ends is not None:
            a.hist_ends = buf.ptr("hist_end")
            a.hist_ids = hp.hist_store.ids.data_ptr()
        a.hist_invalid = buf.ptr("hist_invalid") if hp.hist_invalid is not None else None
        a.tokens, a.status, a.tk_key = buf.ptr("tokens"), buf.ptr("status"), buf.ptr("tk_key")
        a.cut_comp, a.row_max = buf.ptr("cut_comp"), buf.ptr("row_max")
        a.kept_mass, a.row_mass = buf.ptr("kept_mass"), buf.ptr("row_mass")
        a.chosen_logprob = buf.ptr("chosen_lp")
        a.top_ids, a.top_logprobs = buf.ptr("top_ids"), buf.ptr("top_lp")
        a.rng = buf.ptr("rng") if hp.rng is not None else None
        a._keep = logits  # the converted tensor must outlive the launch
        return a

    def launch(self, args: SamplerArgs) -> None:
        ws = self.ensure_workspace(args.rows, args.vocab)
        rc = self.lib.fie_sampler_sample(ctypes.byref(args), ctypes.byref(ws), self._stream_ptr())
        _lib.check(rc, "fie_sampler_sample")

    def launch_stage(self, args: SamplerArgs, stage: int) -> None:
        ws = self.ensure_workspace(args.rows, args.vocab)
        rc = self.lib.fie_sampler_stage(ctypes.byref(args), ctypes.byref(ws), stage,
                                        self._stream_ptr())
        _lib.check(rc, f"fie_sampler_stage({stage})")

    def kept(self, args: SamplerArgs, want_probs: bool = True):
        """Kept mask and draw probabilities of the last launch with these args."""
        rows, vocab = args.rows, args.vocab
        kept = torch.empty((rows, vocab), dtype=torch.uint8, device=self.device)
        probs = torch.empty((rows, vocab), dtype=torch.float32, device=self.device) \
            if want_probs else None
        rc = self.lib.fie_sampler_kept(ctypes.byref(args), kept.data_ptr(),
                                       probs.data_ptr() if probs is not None else None,
                                       ctypes.byref(self.ensure_workspace(rows, vocab)), self._stream_ptr())
        _lib.check(rc, "fie_sampler_kept")
        return kept, probs

    def argmax(self, logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """logits.argmax(-1), first index on ties (sampler.py:106)."""
        logits, dt = self._logits_info(logits)
        rows, vocab = logits.shape
        ws = self.ensure_workspace(rows, vocab)
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

    def uniforms(self, rng: torch.Tensor) -> torch.Tensor:
        """The on-device draws of uint64 (key0, key1, counter) triples [rows, 3]
        (verification of what the sampler derives when ``HostParams.rng`` is set)."""
        rows = rng.shape[0]
        out = torch.empty(rows, dtype=torch.float64, device=self.device)
        _lib.check(self.lib.fie_sampler_uniforms(rng.data_ptr(), out.data_ptr(), rows,
                                                 self._stream_ptr()), "fie_sampler_uniforms")
        return out

    def launch_lmhead(self, args: SamplerArgs, hidden: torch.Tensor, weight: torch.Tensor,
                      kernel_only: bool = False) -> None:
        """The fused lm_head step: args.logits receives hidden @ weight.T and the
        sampler runs on it (fie_sampler_lmhead_sample); with kernel_only, the fused
        kernel alone (fie_sampler_lmhead_stage, for timing)."""
        ws = self.ensure_workspace(args.rows, args.vocab)
        fn = self.lib.fie_sampler_lmhead_stage if kernel_only else self.lib.fie_sampler_lmhead_sample
        rc = fn(ctypes.byref(args), hidden.data_ptr(), weight.data_ptr(), hidden.shape[1], ctypes.byref(ws),
                self._stream_ptr())
        _lib.check(rc, "fie_sampler_lmhead_stage" if kernel_only else "fie_sampler_lmhead_sample")

    def lmhead_step(self, hidden: torch.Tensor, weight: torch.Tensor, hp: HostParams,
                    logits: torch.Tensor | None = None):
        """One step from the last hidden states: logits = hidden @ weight.T (the model's
        output layer, continuous_batching.py:1345) fused with the sampler.  hidden
        [rows, H] and weight [vocab, H] share one dtype, fp16 or bf16, which the logits
        take too.  Returns (outputs, args, buffers, logits) after one sync."""
        if hidden.dtype not in (torch.float16, torch.bfloat16) or weight.dtype != hidden.dtype:
            raise ValueError("hidden and weight must share one dtype, float16 or bfloat16")
        if hidden.dim() != 2 or weight.dim() != 2 or hidden.shape[1] != weight.shape[1]:
            raise ValueError("hidden [rows, H] and weight [vocab, H] must agree on H")
        hidden, weight = hidden.contiguous(), weight.contiguous()
        rows, vocab = hidden.shape[0], weight.shape[0]
        if logits is None:
            logits = torch.empty((rows, vocab), dtype=hidden.dtype, device=self.device)
        elif (logits.dtype != hidden.dtype or tuple(logits.shape) != (rows, vocab)
              or logits.stride(1) != 1 or logits.stride(0) < vocab):
            raise ValueError("logits must be a [rows, vocab] buffer of the model dtype with unit column stride")
        buf = self.step_buffers(rows, hp.tail_ints())
        buf.stage(hp)
        stream = torch.cuda.current_stream(self.device)
        buf.upload(stream)
        if hp.hist_ends is not None and hp.hist_write_dst.shape[0]:
            n = int(hp.hist_write_dst.shape[0])
            o = buf.ptr("hist_ids")
            _lib.check(self.lib.fie_sampler_history_write(hp.hist_store.ids.data_ptr(), o, o + 8 * n, n,
                                                          self._stream_ptr()), "fie_sampler_history_write")
        args = self.build_args(logits, buf, hp)
        self.launch_lmhead(args, hidden, weight)
        buf.download(stream)
        stream.synchronize()
        return buf.outputs(), args, buf, logits

    # ------------------------------------------------------------------ a full step
    def step(self, logits: torch.Tensor, hp: HostParams):
        """Upload, launch, download; returns (outputs, args, buffers) after one sync.
        Everything the host prepares (the staged block, the argument struct, the
        workspace) is ready before the first enqueue, so the device runs the copy,
        the history append, the kernels and the copy back without waiting on Python."""
        rows = logits.shape[0]
        buf = self.step_buffers(rows, hp.tail_ints())
        buf.stage(hp)
        args = self.build_args(logits, buf, hp)
        ws = self.ensure_workspace(args.rows, args.vocab)
        stream = torch.cuda.current_stream(self.device)
        sptr = stream.cuda_stream
        lib = self.lib
        n = int(hp.hist_write_dst.shape[0]) if hp.hist_ends is not None else 0
        ids_ptr = hp.hist_store.ids.data_ptr() if n else 0
        buf.upload(stream)
        if n:
            o = buf.ptr("hist_ids")
            _lib.check(lib.fie_sampler_history_write(ids_ptr, o, o + 8 * n, n, sptr),
                       "fie_sampler_history_write")
        _lib.check(lib.fie_sampler_sample(ctypes.byref(args), ctypes.byref(ws), sptr), "fie_sampler_sample")
        buf.download(stream)
        stream.synchronize()
        return buf.outputs(), args, buf
