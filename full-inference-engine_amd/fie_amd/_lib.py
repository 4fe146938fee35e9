"""ctypes binding of the C ABI in include/fie_sampler.h.

The shared library is built in-tree by ``fie_amd.build`` into ``fie_amd/_native``.
There is no fallback: if the library cannot be loaded, every entry point raises.
"""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_native", "libfie_sampler.so")

FIE_OK = 0
FIE_E_ARG, FIE_E_WORKSPACE, FIE_E_LAUNCH = -1, -2, -3
FIE_F32, FIE_F16, FIE_BF16 = 0, 1, 2
FIE_FLAG_GREEDY, FIE_FLAG_PENALTY = 1, 2
FIE_ROW_EXACT_PATH = 1
FIE_ROW_UNCOUNTED_IDS = 2
FIE_STAGE_PREP, FIE_STAGE_SCAN, FIE_STAGE_FINISH, FIE_STAGE_DEEP = 0, 1, 2, 3
LP_COLS = 20
TILE = 8192
MAX_VOCAB = 64 * TILE

_vp = ctypes.c_void_p


class SamplerArgs(ctypes.Structure):
    """Mirror of ``fie_sampler_args``."""

    _fields_ = [
        ("logits", _vp), ("dtype", ctypes.c_int32), ("rows", ctypes.c_int32),
        ("vocab", ctypes.c_int32), ("lp_cols", ctypes.c_int32), ("row_stride", ctypes.c_int64),
        ("scale", _vp), ("top_k", _vp), ("top_p", _vp), ("min_p", _vp), ("flags", _vp),
        ("logprobs", _vp), ("uniform", _vp),
        ("apply_penalties", ctypes.c_int32), ("max_row_hist", ctypes.c_int32),
        ("repetition", _vp), ("presence", _vp), ("frequency", _vp),
        ("hist_offsets", _vp), ("hist_ids", _vp), ("hist_invalid", _vp),
        ("tokens", _vp), ("status", _vp), ("tk_key", _vp), ("cut_comp", _vp),
        ("row_max", _vp), ("kept_mass", _vp), ("row_mass", _vp), ("chosen_logprob", _vp),
        ("top_ids", _vp), ("top_logprobs", _vp), ("rng", _vp), ("hist_ends", _vp),
    ]


class Workspace(ctypes.Structure):
    """Mirror of ``fie_workspace``."""

    _fields_ = [("ptr", _vp), ("bytes", ctypes.c_size_t), ("max_rows", ctypes.c_int32),
                ("vocab", ctypes.c_int32)]


# Every symbol include/fie_sampler.h declares.
EXPORTS = (
    "fie_sampler_workspace_size", "fie_sampler_sample", "fie_sampler_stage",
    "fie_sampler_argmax", "fie_sampler_kept", "fie_sampler_cexp", "fie_sampler_last_error",
    "fie_sampler_sample_noalloc", "fie_sampler_uniforms", "fie_sampler_history_write",
    "fie_sampler_lmhead_sample", "fie_sampler_lmhead_stage",
)
SCRATCH_BYTES = 64 << 20

_lib = None


class NativeError(RuntimeError):
    pass


def load():
    """Load the HIP library (import torch first so both share one HIP runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    import torch  # noqa: F401  -- the HIP runtime must come from torch's process image

    if not os.path.exists(LIB_PATH):
        raise NativeError(
            f"the HIP sampler library is not built ({LIB_PATH}); run fie_amd.build.build()")
    lib = ctypes.CDLL(LIB_PATH)
    bind(lib)
    _lib = lib
    return lib


def bind(lib) -> None:
    """Declare argument and result types of every exported function."""
    lib.fie_sampler_workspace_size.restype = ctypes.c_size_t
    lib.fie_sampler_workspace_size.argtypes = [ctypes.c_int32, ctypes.c_int32]
    lib.fie_sampler_sample.argtypes = [ctypes.POINTER(SamplerArgs), ctypes.POINTER(Workspace), _vp]
    lib.fie_sampler_stage.argtypes = [
        ctypes.POINTER(SamplerArgs), ctypes.POINTER(Workspace), ctypes.c_int32, _vp]
    lib.fie_sampler_argmax.argtypes = [
        _vp, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int64, _vp,
        ctypes.POINTER(Workspace), _vp]
    lib.fie_sampler_kept.argtypes = [
        ctypes.POINTER(SamplerArgs), _vp, _vp, ctypes.POINTER(Workspace), _vp]
    lib.fie_sampler_cexp.argtypes = [_vp, _vp, ctypes.c_int64, _vp]
    lib.fie_sampler_sample_noalloc.argtypes = [ctypes.POINTER(SamplerArgs), _vp]
    lib.fie_sampler_uniforms.argtypes = [_vp, _vp, ctypes.c_int32, _vp]
    lib.fie_sampler_history_write.argtypes = [_vp, _vp, _vp, ctypes.c_int64, _vp]
    for name in ("fie_sampler_lmhead_sample", "fie_sampler_lmhead_stage"):
        getattr(lib, name).argtypes = [ctypes.POINTER(SamplerArgs), _vp, _vp, ctypes.c_int32,
                                       ctypes.POINTER(Workspace), _vp]
    lib.fie_sampler_last_error.restype = ctypes.c_char_p
    for name in EXPORTS:
        if name not in ("fie_sampler_workspace_size", "fie_sampler_last_error"):
            getattr(lib, name).restype = ctypes.c_int


def check(rc: int, what: str) -> None:
    if rc != FIE_OK:
        msg = _lib.fie_sampler_last_error().decode() if _lib is not None else ""
        raise NativeError(f"{what} failed ({rc}): {msg}")
