"""fie_sampler_sample_noalloc against fie_sampler_sample, through the C ABI.

The no-allocation entry point runs the same kernels on a static device array
instead of a caller workspace; its outputs must be bit-identical to the
workspace entry point's, on two calls in a row, the second with a smaller input
(fewer rows and a smaller vocabulary), so that state left in the array by the
first call cannot leak into the second.
"""

import ctypes

import numpy as np
import pytest
import torch

from fie_amd import _lib
from fie_amd import workloads as W
from fie_amd.batching.sampler import resolve_params
from fie_amd.kernel import FusedSampler

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _outputs(fs, w, use_noalloc):
    B, V = w.logits.shape
    hp = resolve_params(w.params, V, w.uniforms, w.contexts)
    buf = fs.step_buffers(B, int(hp.hist_off[-1]) if hp.apply_penalties else 0)
    buf.stage(hp)
    stream = torch.cuda.current_stream(DEV)
    buf.upload(stream)
    logits = w.logits.to(DEV)
    args = fs.build_args(logits, buf, hp)
    if use_noalloc:
        rc = fs.lib.fie_sampler_sample_noalloc(ctypes.byref(args), ctypes.c_void_p(stream.cuda_stream))
        _lib.check(rc, "fie_sampler_sample_noalloc")
    else:
        fs.launch(args)
    buf.download(stream)
    stream.synchronize()
    return {k: v.copy() for k, v in buf.outputs().items()}


def test_noalloc_matches_the_workspace_entry_point_twice():
    fs = FusedSampler(DEV)
    cases = [W.make(3, rows=list(range(0, 256, 4)), device=DEV),   # 64 rows, V=151936
             W.make(2, rows=list(range(10)), device=DEV)]           # fewer rows
    small = W.make(1, rows=[0, 4, 5], device=DEV)
    small.logits = small.logits[:, :50000].contiguous()              # and a smaller vocab
    cases.append(small)
    for w in cases:
        print(f"  case: {w.name} rows={w.logits.shape[0]} vocab={w.logits.shape[1]}", flush=True)
        want = _outputs(fs, w, use_noalloc=False)
        got = _outputs(fs, w, use_noalloc=True)
        for name in want:
            np.testing.assert_array_equal(got[name], want[name], err_msg=name)


def test_noalloc_rejects_inputs_beyond_the_array():
    fs = FusedSampler(DEV)
    rows, vocab = 4096, 151936
    need = fs.lib.fie_sampler_workspace_size(rows, vocab)
    assert need > _lib.SCRATCH_BYTES
    args = _lib.SamplerArgs()
    x = torch.zeros(1, dtype=torch.float32, device=DEV)
    args.logits = x.data_ptr()
    args.dtype = _lib.FIE_F32
    args.rows, args.vocab, args.row_stride, args.lp_cols = rows, vocab, vocab, 0
    for f in ("tokens", "scale", "top_k", "top_p", "min_p", "flags", "uniform"):
        setattr(args, f, x.data_ptr())
    rc = fs.lib.fie_sampler_sample_noalloc(ctypes.byref(args), None)
    assert rc == _lib.FIE_E_WORKSPACE
    assert b"static scratch" in fs.lib.fie_sampler_last_error()


def test_noalloc_replays_in_a_hip_graph():
    """The no-allocation entry point captured once in a HIP graph and replayed over
    fresh logits written (eagerly) into the same buffer: every replay matches an eager
    fie_sampler_sample on the same logits.  The kernels record no memset and allocate
    nothing, and every word a call reads is written earlier in that call."""
    fs = FusedSampler(DEV)
    w = W.make(3, rows=list(range(0, 256, 8)), device=DEV)          # 32 rows, penalties, all row kinds
    B, V = w.logits.shape
    hp = resolve_params(w.params, V, w.uniforms, w.contexts)
    buf = fs.step_buffers(B, int(hp.hist_off[-1]))
    buf.stage(hp)
    stream = torch.cuda.current_stream(DEV)
    buf.upload(stream)
    logits = w.logits.to(DEV).clone()
    args = fs.build_args(logits, buf, hp)
    lib = fs.lib
    _lib.check(lib.fie_sampler_sample_noalloc(ctypes.byref(args), ctypes.c_void_p(stream.cuda_stream)),
               "fie_sampler_sample_noalloc")                          # resolves the array eagerly
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cap = torch.cuda.current_stream(DEV)
        _lib.check(lib.fie_sampler_sample_noalloc(ctypes.byref(args), ctypes.c_void_p(cap.cuda_stream)),
                   "fie_sampler_sample_noalloc (captured)")
    g = torch.Generator(device=DEV).manual_seed(3)
    for rep in range(4):
        print(f"  replay {rep}", flush=True)
        perm = torch.randperm(V, generator=g, device=DEV)
        logits.copy_(w.logits.to(DEV)[:, perm])                     # new values, same buffer
        graph.replay()
        buf.download(stream)
        stream.synchronize()
        got = {k: v.copy() for k, v in buf.outputs().items()}
        fs.launch(args)
        buf.download(stream)
        stream.synchronize()
        for name, want in buf.outputs().items():
            np.testing.assert_array_equal(got[name], want, err_msg=f"{name} replay {rep}")
