"""ctypes binding of `libvelograd_kernels.so` (C ABI: include/velograd_kernels.h).

torch is imported before the library is opened: torch ships the HIP runtime
(`libamdhip64.so.7`) that owns its streams and allocations, and the dynamic loader then binds
this library to that same runtime instead of loading a second copy.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must be loaded before the HIP library; see module docstring)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib",
                        "libvelograd_kernels.so")

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2

TORCH_DTYPE_CODES = {
    torch.float32: DTYPE_F32,
    torch.float16: DTYPE_F16,
    torch.bfloat16: DTYPE_BF16,
}

MX_E4M3 = 0
MX_E2M1 = 1

ROPE_HALF = 0
ROPE_INTERLEAVED = 1

ERR_INVALID_ARGUMENT = -1
ERR_UNSUPPORTED_DTYPE = -2
ERR_WORKSPACE_TOO_SMALL = -3
ERR_DEVICE_QUERY = -4

_c_i32 = ctypes.c_int32
_c_i64 = ctypes.c_int64
_c_ptr = ctypes.c_void_p
_c_size = ctypes.c_size_t

# name -> (restype, argtypes); kept in the order of include/velograd_kernels.h.
SIGNATURES = {
    "velograd_rmsnorm_residual_fwd": (
        _c_i32,
        [_c_ptr, _c_ptr, _c_ptr,            # x, residual, weight
         _c_ptr, _c_ptr, _c_ptr,            # y, h, inv_rms
         _c_i64, _c_i64,                    # rows, dim
         _c_i64, _c_i64, _c_i64, _c_i64,    # ld_x, ld_res, ld_y, ld_h
         _c_i32, _c_i32, ctypes.c_float,    # dtype, w_dtype, eps
         _c_ptr],                           # hip_stream
    ),
    "velograd_rmsnorm_fwd": (
        _c_i32,
        [_c_ptr, _c_ptr, _c_ptr,            # x, residual, weight
         _c_ptr, _c_ptr, _c_ptr,            # y, h, inv_rms
         _c_i64, _c_i64,                    # rows, dim
         _c_i64, _c_i64, _c_i64, _c_i64,    # ld_x, ld_res, ld_y, ld_h
         _c_i32, _c_i32,                    # dtype, w_dtype
         ctypes.c_float, ctypes.c_float,    # eps, min_mean_sq
         _c_ptr],                           # hip_stream
    ),
    "velograd_rmsnorm_rope_fwd": (
        _c_i32,
        [_c_ptr, _c_ptr, _c_ptr,            # x, residual, weight
         _c_ptr, _c_ptr, _c_ptr,            # y, h, inv_rms
         _c_i64, _c_i64,                    # rows, dim
         _c_i64, _c_i64, _c_i64, _c_i64,    # ld_x, ld_res, ld_y, ld_h
         _c_i64, _c_i32, _c_i32,            # seq, dtype, w_dtype
         ctypes.c_float, ctypes.c_float,    # eps, min_mean_sq
         ctypes.c_float, _c_ptr],           # base, hip_stream
    ),
    "velograd_rmsnorm_residual_fwd_fp8": (
        _c_i32,
        [_c_ptr, _c_ptr, _c_ptr,            # x, residual, weight
         _c_ptr, _c_ptr,                    # y_fp8, y_scale
         _c_ptr, _c_ptr,                    # h, inv_rms
         _c_i64, _c_i64,                    # rows, dim
         _c_i64, _c_i64, _c_i64, _c_i64,    # ld_x, ld_res, ld_y (bytes), ld_h
         _c_i32, _c_i32, ctypes.c_float,    # dtype, w_dtype, eps
         _c_ptr],                           # hip_stream
    ),
    "velograd_rmsnorm_residual_fwd_mx": (
        _c_i32,
        [_c_ptr, _c_ptr, _c_ptr,            # x, residual, weight
         _c_ptr, _c_ptr,                    # y_q, y_scales
         _c_ptr, _c_ptr,                    # h, inv_rms
         _c_i64, _c_i64,                    # rows, dim
         _c_i64, _c_i64, _c_i64, _c_i64,    # ld_x, ld_res, ld_yq (bytes), ld_scales (bytes)
         _c_i64,                            # ld_h
         _c_i32, _c_i32, _c_i32,            # dtype, w_dtype, mx_format
         ctypes.c_float, _c_ptr],           # eps, hip_stream
    ),
    "velograd_rmsnorm_residual_bwd": (
        _c_i32,
        [_c_ptr, _c_ptr, _c_i32,            # grad_y, saved, saved_is_h
         _c_ptr, _c_ptr, _c_ptr,            # weight, inv_rms, grad_h
         _c_ptr, _c_ptr, _c_ptr,            # dx, dres, dweight
         _c_ptr, _c_size,                   # workspace, ws_bytes
         _c_i64, _c_i64,                    # rows, dim
         _c_i64, _c_i64, _c_i64,            # ld_g, ld_saved, ld_grad_h
         _c_i64, _c_i64,                    # ld_dx, ld_dres
         _c_i32, _c_i32,                    # dtype, w_dtype
         _c_ptr],                           # hip_stream
    ),
    "velograd_rmsnorm_residual_bwd_noalloc": (
        _c_i32,
        [_c_ptr, _c_ptr, _c_i32,            # grad_y, saved, saved_is_h
         _c_ptr, _c_ptr, _c_ptr,            # weight, inv_rms, grad_h
         _c_ptr, _c_ptr, _c_ptr,            # dx, dres, dweight
         _c_i64, _c_i64,                    # rows, dim
         _c_i64, _c_i64, _c_i64,            # ld_g, ld_saved, ld_grad_h
         _c_i64, _c_i64,                    # ld_dx, ld_dres
         _c_i32, _c_i32,                    # dtype, w_dtype
         _c_ptr],                           # hip_stream
    ),
    "velograd_rmsnorm_rope_bwd": (
        _c_i32,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr,    # grad_y, h, weight, inv_rms
         _c_ptr, _c_ptr,                    # dx, dweight
         _c_ptr, _c_size,                   # workspace, ws_bytes
         _c_i64, _c_i64,                    # rows, dim
         _c_i64, _c_i64, _c_i64,            # ld_g, ld_h, ld_dx
         _c_i64, _c_i32, _c_i32,            # seq, dtype, w_dtype
         ctypes.c_float, _c_ptr],           # base, hip_stream
    ),
    "velograd_rmsnorm_residual_bwd_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i32]),
    "velograd_rope": (
        _c_i32,
        [_c_ptr, _c_ptr,                    # x, out
         _c_i64, _c_i64, _c_i64, _c_i64,    # outer, seq, heads, dim
         _c_i64, ctypes.c_float, _c_i32,    # rot_dim, theta, inverse
         _c_i32, _c_i32, _c_ptr],           # pairing, dtype, hip_stream
    ),
    "velograd_kernels_last_error": (ctypes.c_char_p, []),
    "velograd_kernels_version": (ctypes.c_char_p, []),
}

_lock = threading.Lock()
_lib = None


class KernelLibraryMissing(RuntimeError):
    """The HIP library has not been built; there is deliberately no CPU fallback."""


def load() -> ctypes.CDLL:
    """Open the HIP library once and attach the C signatures."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise KernelLibraryMissing(
                    f"{LIB_PATH} is missing: build it with `python -m velograd_amd.build` "
                    "(or __graft_entry__.build()); velograd_amd has no CPU fallback")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = lib
    return _lib


_fast = None
_fast_tried = False


def fastpath():
    """The optional pybind11 fast path (`velograd_amd._fastpath`, built next to the library by
    velograd_amd.build) for launch-bound forward calls, or None when it is not built or when
    VELOGRAD_NO_FASTPATH=1.  Loaded once, after the kernels library."""
    global _fast, _fast_tried
    if not _fast_tried:
        load()
        with _lock:
            if not _fast_tried:
                if os.environ.get("VELOGRAD_NO_FASTPATH", "0") != "1":
                    try:
                        from . import _fastpath as fp
                        _fast = fp
                    except ImportError:
                        _fast = None
                _fast_tried = True
    return _fast


def last_error() -> str:
    msg = load().velograd_kernels_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(rc: int, what: str) -> None:
    """Turn a C status into a Python exception (ValueError/TypeError for argument errors)."""
    if rc == 0:
        return
    msg = f"{what} failed (status {rc}): {last_error()}"
    if rc == ERR_UNSUPPORTED_DTYPE:
        raise TypeError(msg)
    if rc in (ERR_INVALID_ARGUMENT, ERR_WORKSPACE_TOO_SMALL):
        raise ValueError(msg)
    raise RuntimeError(msg)
