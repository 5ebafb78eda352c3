"""Drop-in `velograd.kernels` fused RMSNorm + residual functions on MI355X HIP kernels.

Same names, positional order, defaults and return arity as the reference:

  fused_rmsnorm_residual_forward(x, residual=None, weight=None, eps=1e-6) -> (y, h, inv_rms)
      python/velograd/kernels/fused.py:28-46
  fused_rmsnorm_residual_backward(grad_out, normed_input, weight, inv_rms) -> (grad_x, grad_weight)
      python/velograd/kernels/fused.py:48-66
  fused_rmsnorm_residual(x, residual=None, weight=None, eps=1e-6) -> y
      python/velograd/kernels/__init__.py:19-32

Inputs
  * torch tensors on a ROCm device (torch's device type is named "cuda") run in their own dtype
    (float32, float16 or bfloat16; fp32 arithmetic inside): y, h and grad_x come back in that
    dtype, inv_rms ([..., 1]) and grad_weight ([D]) in float32.
  * NumPy arrays, lists and CPU tensors follow the reference wrapper
    (python/velograd/kernels/__init__.py:21-27): they are cast to float32, computed on the GPU
    and returned as float32 NumPy arrays.
There is no CPU implementation behind these functions: without the HIP library or a visible
ROCm device they raise.

Reference semantics kept: the last axis is normalised and every leading axis is a row;
`residual=None` makes `h` the very object `x` (fused.py:39); `weight=None` skips the scale and
returns `grad_weight=None` (fused.py:44-45, 62-65); NaN and Inf propagate (no clamping);
`normed_input` of the backward is xhat = h * inv_rms, before the weight.  Since h = x + residual,
`grad_x` is also the gradient of `residual`.

Additions (keyword-only, off by default): `saved_is_h=True` lets the backward take h instead of
xhat (xhat is then formed in registers; same bytes moved), `dresidual_out=` receives a second
copy of grad_x in a caller-owned buffer, and `grad_h=` adds the residual-stream gradient (the
gradient reaching h from the next residual add) to grad_x in the same pass.
`fused_rmsnorm_residual_forward_fp8` returns y as fp8 E4M3 codes with one scale per row, and
`fused_rmsnorm_residual_forward_mx` as MXFP8 / MXFP4 blocks (one E8M0 scale per 32 elements).
`rmsnorm_forward` is the residual-free form of the reference's module (nn.py:338-355), with its
floor on the mean square.
"""

from __future__ import annotations

import math
from typing import Any, Optional, Tuple

import numpy as np
import torch

from .. import _lib

__all__ = [
    "fused_rmsnorm_residual",
    "fused_rmsnorm_residual_forward",
    "fused_rmsnorm_residual_backward",
    "fused_rmsnorm_residual_forward_fp8",
    "fused_rmsnorm_residual_forward_mx",
    "rmsnorm_forward",
    "rmsnorm_rope_forward",
    "rmsnorm_rope_backward",
    "fused_rope",
    "fused_rope_forward",
    "fused_rope_backward",
    "fused_rope_interleaved",
    "bwd_workspace_bytes",
]


# ---------------------------------------------------------------------------------------------
# Argument handling
# ---------------------------------------------------------------------------------------------
def _is_device_tensor(t: Any) -> bool:
    return isinstance(t, torch.Tensor) and t.device.type == "cuda"


def _require_gpu() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError(
            "velograd_amd.kernels computes on an MI355X and no ROCm device is visible; "
            "there is no CPU fallback")
    return torch.device("cuda", torch.cuda.current_device())


def _rows_view(t: torch.Tensor, name: str) -> torch.Tensor:
    """[..., D] -> [rows, D] with unit stride along D (a view when possible, else a copy)."""
    if t.dim() == 0:
        raise ValueError(f"{name} must have at least one dimension")
    d = t.shape[-1]
    rows = math.prod(t.shape[:-1])
    if t.dim() == 1:
        t2 = t.unsqueeze(0)
    else:
        try:
            t2 = t.view(rows, d)
        except RuntimeError:
            t2 = t.reshape(rows, d)
    if d > 0 and t2.shape[0] > 0 and t2.stride(-1) != 1:
        t2 = t2.contiguous()
    return t2


def _ld(t2: torch.Tensor) -> int:
    # Row stride in elements; a single row may report any stride, use D then.
    return t2.stride(0) if t2.shape[0] > 1 else t2.shape[1]


def _dtype_code(t: torch.Tensor, name: str) -> int:
    code = _lib.TORCH_DTYPE_CODES.get(t.dtype)
    if code is None:
        raise TypeError(f"{name}: unsupported dtype {t.dtype}; use float32, float16 or bfloat16")
    return code


def _prep_weight(weight: Optional[torch.Tensor], d: int, act_dtype: torch.dtype,
                 device: torch.device) -> Tuple[Optional[torch.Tensor], int]:
    """Weight as a contiguous [D] tensor in the activation dtype or float32."""
    if weight is None:
        return None, _lib.TORCH_DTYPE_CODES[act_dtype]
    if not isinstance(weight, torch.Tensor):
        weight = torch.as_tensor(np.asarray(weight, dtype=np.float32), device=device)
    if weight.device != device:
        raise ValueError(f"weight is on {weight.device}, activations on {device}")
    if weight.numel() != d:
        raise ValueError(f"weight has {weight.numel()} elements, expected {d} (shape [D] or [1, D])")
    w = weight.reshape(d)
    if w.dtype not in (act_dtype, torch.float32):
        w = w.to(torch.float32)
    w = w.contiguous()
    return w, _lib.TORCH_DTYPE_CODES[w.dtype]


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


# torch's current-stream handle as a plain integer, without building a Stream object (the public
# torch.cuda.current_stream(device).cuda_stream costs ~2.6 us per call, a fifth of a decode call)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device: torch.device) -> int:
    """The hipStream_t of torch's current stream on `device` (the capture stream under graph
    capture)."""
    if _raw_stream is not None:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(idx)
    return torch.cuda.current_stream(device).cuda_stream


def bwd_workspace_bytes(rows: int, dim: int, device: Optional[torch.device] = None) -> int:
    """Bytes of scratch the backward needs for the two-stage dweight reduction."""
    dev = device if device is not None else _require_gpu()
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    return int(_lib.load().velograd_rmsnorm_residual_bwd_workspace_bytes(rows, dim, idx))


# ---------------------------------------------------------------------------------------------
# Device paths
# ---------------------------------------------------------------------------------------------
def _forward_fast(x: torch.Tensor, residual: Optional[torch.Tensor],
                  weight: Optional[torch.Tensor], eps: float, min_mean_sq: float = 0.0):
    """The common case without views or copies, for launch-latency-bound (decode) calls:
    contiguous tensors of one dtype on the current device, weight [D] in that dtype or fp32.
    Returns None when the call does not qualify (the general path then handles it)."""
    fp = _lib.fastpath()
    if fp is not None:
        if not ((residual is None or isinstance(residual, torch.Tensor))
                and (weight is None or isinstance(weight, torch.Tensor))):
            return None
        out = fp.forward(x, residual, weight, float(eps), float(min_mean_sq))
        if not out:
            return None
        return out[0], (x if residual is None else out[1]), out[2]
    code = _lib.TORCH_DTYPE_CODES.get(x.dtype)
    if code is None or x.dim() == 0 or not x.is_contiguous():
        return None
    d = x.shape[-1]
    rows = x.numel() // d if d > 0 else 0
    if rows == 0:
        return None
    dev = x.device
    if dev.index != torch.cuda.current_device():
        return None
    if residual is not None and not (
            isinstance(residual, torch.Tensor) and residual.dtype == x.dtype
            and residual.shape == x.shape and residual.is_contiguous() and residual.device == dev):
        return None
    wcode = code
    if weight is not None:
        if not (isinstance(weight, torch.Tensor) and weight.dim() == 1 and weight.shape[0] == d
                and weight.is_contiguous() and weight.device == dev):
            return None
        wcode = _lib.TORCH_DTYPE_CODES.get(weight.dtype)
        if wcode != code and wcode != _lib.DTYPE_F32:
            return None
    y = torch.empty_like(x)
    h = torch.empty_like(x) if residual is not None else x
    inv_rms = torch.empty(x.shape[:-1] + (1,), dtype=torch.float32, device=dev)
    lib = _lib.load()
    args = (x.data_ptr(), None if residual is None else residual.data_ptr(),
            None if weight is None else weight.data_ptr(),
            y.data_ptr(), None if residual is None else h.data_ptr(), inv_rms.data_ptr(),
            rows, d, d, d, d, d, code, wcode, float(eps))
    if min_mean_sq > 0.0:
        _lib.check(lib.velograd_rmsnorm_fwd(*args, min_mean_sq, _stream(dev)),
                   "velograd_rmsnorm_fwd")
    else:
        _lib.check(lib.velograd_rmsnorm_residual_fwd(*args, _stream(dev)),
                   "velograd_rmsnorm_residual_fwd")
    return y, h, inv_rms


def _check_min_mean_sq(min_mean_sq: float) -> float:
    min_mean_sq = float(min_mean_sq)
    if not (math.isfinite(min_mean_sq) and min_mean_sq >= 0.0):
        raise ValueError(f"min_mean_sq must be finite and >= 0, got {min_mean_sq}")
    return min_mean_sq


def _forward_device(x: torch.Tensor, residual: Optional[torch.Tensor],
                    weight: Optional[torch.Tensor], eps: float, fp8: bool = False,
                    mx: Optional[str] = None, min_mean_sq: float = 0.0):
    min_mean_sq = _check_min_mean_sq(min_mean_sq)
    if min_mean_sq > 0.0 and (fp8 or mx is not None):
        raise ValueError("min_mean_sq applies to the forward with y in the input dtype only")
    if not fp8 and mx is None:
        fast = _forward_fast(x, residual, weight, eps, min_mean_sq)
        if fast is not None:
            return fast
    lib = _lib.load()
    device = x.device
    code = _dtype_code(x, "x")
    if residual is not None:
        if not isinstance(residual, torch.Tensor) or residual.device != device:
            raise ValueError("residual must be a tensor on the same device as x")
        if residual.dtype != x.dtype:
            raise TypeError(f"residual dtype {residual.dtype} differs from x dtype {x.dtype}")
        if residual.shape != x.shape:
            # NumPy broadcasting of `x + residual` (fused.py:39), materialised.
            x, residual = torch.broadcast_tensors(x, residual)
            x, residual = x.contiguous(), residual.contiguous()
    out_shape = x.shape
    d = out_shape[-1] if x.dim() > 0 else 0
    w, wcode = _prep_weight(weight, d, x.dtype, device)

    x2 = _rows_view(x, "x")
    rows = x2.shape[0]
    if mx is not None and d % 32 != 0:
        raise ValueError(f"MX blocks need a last dimension that is a multiple of 32, got {d}")
    # fp8 / MX codes are allocated as bytes and handed back viewed as their torch dtypes
    y_last = d // 2 if mx == "e2m1" else d
    y = torch.empty(tuple(out_shape[:-1]) + (y_last,),
                    dtype=torch.uint8 if (fp8 or mx) else x.dtype, device=device)
    h = torch.empty(out_shape, dtype=x.dtype, device=device) if residual is not None else x
    stat_shape = tuple(out_shape[:-1]) + (1,)
    inv_rms = torch.empty(stat_shape, dtype=torch.float32, device=device)
    y_scale = torch.empty(stat_shape, dtype=torch.float32, device=device) if fp8 else None
    mx_scale = (torch.empty(tuple(out_shape[:-1]) + (d // 32,), dtype=torch.uint8, device=device)
                if mx is not None else None)

    def result():
        if fp8:
            return y.view(torch.float8_e4m3fn), y_scale, h, inv_rms
        if mx is not None:
            yq = y.view(torch.float8_e4m3fn) if mx == "e4m3" else y.view(torch.float4_e2m1fn_x2)
            return yq, mx_scale.view(torch.float8_e8m0fnu), h, inv_rms
        return y, h, inv_rms

    if rows == 0:
        return result()
    if d == 0:
        # mean over an empty axis is NaN in NumPy; y and h are empty.
        inv_rms.fill_(float("nan"))
        if fp8:
            y_scale.fill_(float("nan"))
        return result()
    if mx is not None:
        r2 = _rows_view(residual, "residual") if residual is not None else None
        y2 = y.view(-1, y_last)
        h2 = h.view(-1, d) if residual is not None else None
        with torch.cuda.device(device):
            rc = lib.velograd_rmsnorm_residual_fwd_mx(
                x2.data_ptr(), _ptr(r2), _ptr(w),
                y2.data_ptr(), mx_scale.data_ptr(), _ptr(h2), inv_rms.data_ptr(),
                rows, d,
                _ld(x2), _ld(r2) if r2 is not None else d, y_last, d // 32, d,
                code, wcode, _lib.MX_E4M3 if mx == "e4m3" else _lib.MX_E2M1, float(eps),
                _stream(device))
        _lib.check(rc, "velograd_rmsnorm_residual_fwd_mx")
        return result()

    r2 = _rows_view(residual, "residual") if residual is not None else None
    y2 = y.view(-1, d)
    h2 = h.view(-1, d) if residual is not None else None
    with torch.cuda.device(device):
        if fp8:
            rc = lib.velograd_rmsnorm_residual_fwd_fp8(
                x2.data_ptr(), _ptr(r2), _ptr(w),
                y2.data_ptr(), y_scale.data_ptr(), _ptr(h2), inv_rms.data_ptr(),
                rows, d,
                _ld(x2), _ld(r2) if r2 is not None else d, d, d,
                code, wcode, float(eps), _stream(device))
        else:
            args = (x2.data_ptr(), _ptr(r2), _ptr(w),
                    y2.data_ptr(), _ptr(h2), inv_rms.data_ptr(),
                    rows, d,
                    _ld(x2), _ld(r2) if r2 is not None else d, d, d,
                    code, wcode, float(eps))
            if min_mean_sq > 0.0:
                rc = lib.velograd_rmsnorm_fwd(*args, min_mean_sq, _stream(device))
            else:
                rc = lib.velograd_rmsnorm_residual_fwd(*args, _stream(device))
    _lib.check(rc, "velograd_rmsnorm_residual_fwd_fp8" if fp8 else
               ("velograd_rmsnorm_fwd" if min_mean_sq > 0.0 else "velograd_rmsnorm_residual_fwd"))
    return result()


def _backward_device(grad_out: torch.Tensor, saved: torch.Tensor,
                     weight: Optional[torch.Tensor], inv_rms: torch.Tensor,
                     saved_is_h: bool, dresidual_out: Optional[torch.Tensor],
                     grad_h: Optional[torch.Tensor] = None):
    lib = _lib.load()
    device = grad_out.device
    code = _dtype_code(grad_out, "grad_out")
    if not isinstance(saved, torch.Tensor) or saved.device != device:
        raise ValueError("normed_input must be a tensor on the same device as grad_out")
    if saved.dtype != grad_out.dtype:
        raise TypeError(f"normed_input dtype {saved.dtype} differs from grad_out dtype "
                        f"{grad_out.dtype}")
    if saved.shape != grad_out.shape:
        raise ValueError(f"normed_input shape {tuple(saved.shape)} differs from grad_out shape "
                         f"{tuple(grad_out.shape)}")
    shape = grad_out.shape
    d = shape[-1] if grad_out.dim() > 0 else 0
    w, wcode = _prep_weight(weight, d, grad_out.dtype, device)

    g2 = _rows_view(grad_out, "grad_out")
    s2 = _rows_view(saved, "normed_input")
    rows = g2.shape[0]
    if not isinstance(inv_rms, torch.Tensor) or inv_rms.device != device:
        raise ValueError("inv_rms must be a tensor on the same device as grad_out")
    if inv_rms.numel() != rows:
        raise ValueError(f"inv_rms has {inv_rms.numel()} elements, expected one per row ({rows})")
    r = inv_rms.reshape(rows)
    if r.dtype != torch.float32:
        r = r.to(torch.float32)
    r = r.contiguous()
    gh2 = None
    if grad_h is not None:
        if (not isinstance(grad_h, torch.Tensor) or grad_h.device != device
                or grad_h.dtype != grad_out.dtype or grad_h.shape != shape):
            raise ValueError("grad_h must be a tensor shaped and typed like grad_out on the same "
                             "device")
        gh2 = _rows_view(grad_h, "grad_h") if d > 0 else None

    dx = torch.empty(shape, dtype=grad_out.dtype, device=device)
    dres2 = None
    if dresidual_out is not None:
        if (not isinstance(dresidual_out, torch.Tensor) or dresidual_out.shape != shape
                or dresidual_out.dtype != grad_out.dtype or dresidual_out.device != device
                or not dresidual_out.is_contiguous()):
            raise ValueError("dresidual_out must be a contiguous tensor shaped and typed like "
                             "grad_out on the same device")
        dres2 = dresidual_out.view(-1, d) if d > 0 else None
    dweight = torch.empty((d,), dtype=torch.float32, device=device) if w is not None else None
    if d == 0:
        return dx, dweight
    if rows == 0:
        if dweight is not None:
            dweight.zero_()
        return dx, dweight

    ws = None
    ws_bytes = 0
    if dweight is not None:
        ws_bytes = bwd_workspace_bytes(rows, d, device)
        ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=device)
    dx2 = dx.view(-1, d)
    with torch.cuda.device(device):
        rc = lib.velograd_rmsnorm_residual_bwd(
            g2.data_ptr(), s2.data_ptr(), 1 if saved_is_h else 0,
            _ptr(w), r.data_ptr(), _ptr(gh2),
            dx2.data_ptr(), _ptr(dres2), _ptr(dweight),
            _ptr(ws), ws_bytes,
            rows, d,
            _ld(g2), _ld(s2), _ld(gh2) if gh2 is not None else d, d, d,
            code, wcode, _stream(device))
    _lib.check(rc, "velograd_rmsnorm_residual_bwd")
    return dx, dweight


# ---------------------------------------------------------------------------------------------
# Host (array-like) inputs: reference wrapper semantics, computed on the GPU.
# ---------------------------------------------------------------------------------------------
def _host_to_device_f32(a: Any, device: torch.device) -> torch.Tensor:
    if isinstance(a, torch.Tensor):
        a = a.detach().cpu().numpy()
    arr = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    return torch.from_numpy(arr).to(device)


def _to_host(t: Optional[torch.Tensor]) -> Optional[np.ndarray]:
    return None if t is None else t.cpu().numpy()


# ---------------------------------------------------------------------------------------------
# Public API
# ---------------------------------------------------------------------------------------------
def fused_rmsnorm_residual_forward(x: Any, residual: Optional[Any] = None,
                                   weight: Optional[Any] = None, eps: float = 1e-6, *,
                                   min_mean_sq: float = 0.0):
    """(x + residual) -> RMS-normalise over the last axis -> scale by weight.

    Returns (normed_output, combined_residual, inv_rms) like fused.py:28-46.  `min_mean_sq`
    (an extension, keyword only) floors mean(h^2) before eps as the reference's module does
    (nn.py:349 uses 1e-12; a NaN mean square becomes the floor, as with Python's max); the
    default 0 is fused.py's unclamped statistic.
    """
    if _is_device_tensor(x):
        return _forward_device(x, residual, weight, eps, min_mean_sq=min_mean_sq)
    device = _require_gpu()
    xd = _host_to_device_f32(x, device)
    rd = _host_to_device_f32(residual, device) if residual is not None else None
    wd = _host_to_device_f32(weight, device) if weight is not None else None
    if wd is not None and wd.numel() != xd.shape[-1]:
        raise ValueError(f"weight has {wd.numel()} elements, expected {xd.shape[-1]}")
    y, h, inv_rms = _forward_device(xd, rd, wd, eps, min_mean_sq=min_mean_sq)
    y_np = _to_host(y)
    # With residual=None the reference returns its (float32) x as h.
    h_np = _to_host(h) if residual is not None else np.asarray(x, dtype=np.float32)
    return y_np, h_np, _to_host(inv_rms)


def fused_rmsnorm_residual_backward(grad_out: Any, normed_input: Any, weight: Optional[Any],
                                    inv_rms: Any, *, saved_is_h: bool = False,
                                    dresidual_out: Optional[torch.Tensor] = None,
                                    grad_h: Optional[Any] = None):
    """Analytic backward of the forward; returns (grad_x, grad_weight) like fused.py:48-66.

    `normed_input` is xhat = h * inv_rms (or h itself with saved_is_h=True); grad_weight is None
    when weight is None.  `grad_h`, the gradient reaching h from its other consumer (the next
    residual add of a pre-norm block), is added to grad_x in the same pass.
    """
    if _is_device_tensor(grad_out):
        return _backward_device(grad_out, normed_input, weight, inv_rms, saved_is_h,
                                dresidual_out, grad_h)
    if dresidual_out is not None:
        raise ValueError("dresidual_out is only supported for device tensors")
    device = _require_gpu()
    gd = _host_to_device_f32(grad_out, device)
    sd = _host_to_device_f32(normed_input, device)
    wd = _host_to_device_f32(weight, device) if weight is not None else None
    rd = _host_to_device_f32(inv_rms, device)
    ghd = _host_to_device_f32(grad_h, device) if grad_h is not None else None
    dx, dw = _backward_device(gd, sd, wd, rd, saved_is_h, None, ghd)
    return _to_host(dx), _to_host(dw)


def fused_rmsnorm_residual_forward_fp8(x: torch.Tensor, residual: Optional[torch.Tensor] = None,
                                       weight: Optional[torch.Tensor] = None, eps: float = 1e-6):
    """The forward with y quantised to fp8 E4M3 for the next GEMM, in the same pass.

    Returns (y_fp8, y_scale, h, inv_rms): y_fp8 is a float8_e4m3fn tensor shaped like x,
    y_scale ([..., 1], float32) is amax(|y|) / 448 per row, the codes are e4m3(y * (1 /
    y_scale)), and y ~= y_fp8.float() * y_scale; h and inv_rms as
    fused_rmsnorm_residual_forward.  Rounding is to nearest even, saturating at +-448.
    Device tensors only (an extension: the reference has no quantising forward; its E4M3
    format is include/velograd/kernels.h:29-37, 58-73).
    """
    if not _is_device_tensor(x):
        raise TypeError("fused_rmsnorm_residual_forward_fp8 takes torch tensors on a ROCm device")
    return _forward_device(x, residual, weight, eps, fp8=True)


# ---------------------------------------------------------------------------------------------
# Fused RoPE (python/velograd/kernels/fused.py:72-130, wrapper kernels/__init__.py:34-48)
# ---------------------------------------------------------------------------------------------
def _rope_q_layout(q_shape, h_dim: int):
    """(outer, seq, heads, dim) of q as fused.py:83-97 reads it, and whether q is the 2-D
    [seq, heads * head_dim] form that the reference reshapes into heads."""
    if len(q_shape) < 2:
        raise ValueError("fused_rope: q must have at least 2 dimensions ([seq, dim] or "
                         "[..., seq, heads, dim])")
    if h_dim < 2 or h_dim % 2 != 0:
        raise ValueError(f"fused_rope: head_dim={h_dim} must be even and >= 2")
    last = q_shape[-1]
    if len(q_shape) == 2:
        if last > h_dim:                                                   # fused.py:88-94
            if last % h_dim != 0:
                raise ValueError(f"fused_rope: last dimension {last} is not a multiple of "
                                 f"head_dim={h_dim}")
            return (1, q_shape[0], last // h_dim, h_dim), True
        if last < h_dim:
            raise ValueError(f"fused_rope: head_dim={h_dim} exceeds the last dimension {last}")
        return (1, q_shape[0], 1, last), False
    if last < h_dim:
        raise ValueError(f"fused_rope: head_dim={h_dim} exceeds the last dimension {last}")
    return (math.prod(q_shape[:-3]), q_shape[-3], q_shape[-2], last), False


def _rope_k_layout(k_shape, q_shape, q_layout, q_split: bool, h_dim: int):
    seq = q_layout[1]
    if q_split:
        # the reference reshapes k with q's head count and k_rot back to q's shape (:91-94,
        # :126-129): only a k shaped like q is meaningful
        if tuple(k_shape) != tuple(q_shape):
            raise ValueError("fused_rope: with q of shape [seq, heads * head_dim], k must have "
                             "q's shape")
        return q_layout
    if len(q_shape) == 2:
        if len(k_shape) != 2 or k_shape[0] != seq:
            raise ValueError(f"fused_rope: k must be [seq={seq}, dim] like q")
        if k_shape[-1] < h_dim:
            raise ValueError(f"fused_rope: head_dim={h_dim} exceeds k's last dimension")
        return (1, seq, 1, k_shape[-1])
    if len(k_shape) != len(q_shape) or k_shape[-3] != seq:
        # the reference would broadcast other leading axes or a length-1 sequence axis
        # against q's tables (fused.py:106-121); the device API takes k with q's positions
        raise ValueError(f"fused_rope: k must be [..., seq={seq}, heads, dim] with q's number of "
                         f"axes (positions on axis -3, like q)")
    if k_shape[-1] < h_dim:
        raise ValueError(f"fused_rope: head_dim={h_dim} exceeds k's last dimension")
    return (math.prod(k_shape[:-3]), k_shape[-3], k_shape[-2], k_shape[-1])


def _rope_device(t: torch.Tensor, layout, h_dim: int, theta: float, inverse: bool,
                 out: Optional[torch.Tensor] = None,
                 pairing: int = _lib.ROPE_HALF) -> torch.Tensor:
    code = _dtype_code(t, "q/k")
    src = t.contiguous()
    dst = torch.empty_like(src) if out is None else out
    outer, seq, heads, dim = layout
    if src.numel() == 0:
        return dst.view(t.shape)
    with torch.cuda.device(src.device):
        rc = _lib.load().velograd_rope(src.data_ptr(), dst.data_ptr(), outer, seq, heads, dim,
                                       h_dim, float(theta), 1 if inverse else 0, pairing,
                                       code, _stream(src.device))
    _lib.check(rc, "velograd_rope")
    return dst.view(t.shape)


def _rope(q: Any, k: Optional[Any], head_dim: Optional[int], theta: float, inverse: bool):
    on_device = _is_device_tensor(q)
    if not on_device:
        device = _require_gpu()
        q_np = np.asarray(q.detach().cpu().numpy() if isinstance(q, torch.Tensor) else q,
                          dtype=np.float32)
        qd = torch.from_numpy(np.ascontiguousarray(q_np)).to(device)
        kd = None
        if isinstance(k, (np.ndarray, torch.Tensor)):       # fused.py:92,124 use k only if an array
            k_np = k.detach().cpu().numpy() if isinstance(k, torch.Tensor) else k
            kd = torch.from_numpy(np.ascontiguousarray(k_np, dtype=np.float32)).to(device)
    else:
        qd, kd = q, k
        if kd is not None and (not isinstance(kd, torch.Tensor) or kd.device != qd.device):
            raise ValueError("k must be a tensor on q's device")
    h_dim = head_dim or qd.shape[-1]                                       # fused.py:83
    q_layout, split = _rope_q_layout(tuple(qd.shape), h_dim)
    k_layout = (_rope_k_layout(tuple(kd.shape), tuple(qd.shape), q_layout, split, h_dim)
                if kd is not None else None)
    q_rot = _rope_device(qd, q_layout, h_dim, theta, inverse)
    k_rot = _rope_device(kd, k_layout, h_dim, theta, inverse) if kd is not None else None
    if on_device:
        return q_rot, k_rot
    return _to_host(q_rot), _to_host(k_rot)


def fused_rope_forward(q: Any, k: Optional[Any] = None, head_dim: Optional[int] = None,
                       theta: float = 10000.0):
    """Rotary position embedding of q (and k), "rotate half" pairing; (q_rot, k_rot) like
    fused.py:72-130.  Positions run along axis -3 ([..., seq, heads, dim]) or axis 0 for 2-D
    input, whose last axis is split into heads of head_dim when it is longer; the last axis past
    head_dim passes through.  Device tensors keep their dtype; arrays are computed in float32
    on the GPU and returned as float32 ndarrays (k only when it is an array, as the reference).

    Inputs the reference takes only through NumPy broadcasting raise ValueError here: an odd
    head_dim or one longer than the last axis, and a k whose positions are not q's (another
    sequence length, a length-1 sequence axis on one side, or another number of axes)."""
    return _rope(q, k, head_dim, theta, inverse=False)


def fused_rope_backward(grad_q: Any, grad_k: Optional[Any] = None,
                        head_dim: Optional[int] = None, theta: float = 10000.0):
    """Gradients of fused_rope_forward: the inverse rotation of grad_q (and grad_k).  An
    extension: the reference's fused RoPE has no backward (its rotary backward rule is
    src/ops.rs:501-530)."""
    return _rope(grad_q, grad_k, head_dim, theta, inverse=True)


def fused_rope(x: Any, k: Optional[Any] = None, head_dim: Optional[int] = None,
               base: float = 10000.0):
    """Wrapper like kernels/__init__.py:34-48: q_rot, or (q_rot, k_rot) when k is given."""
    if not _is_device_tensor(x) and k is not None and not isinstance(k, (np.ndarray, torch.Tensor)):
        k = np.asarray(k, dtype=np.float32)                                # :37
    q_rot, k_rot = fused_rope_forward(x, k, head_dim=head_dim, theta=base)
    if k is not None:
        return q_rot, k_rot
    return q_rot


def fused_rope_interleaved(x: torch.Tensor, base: float = 10000.0,
                           inverse: bool = False) -> torch.Tensor:
    """RoPE with interleaved pairs, as the reference's model applies it: apply_rotary_emb
    (python/velograd/functional.py:287-315; models/llama.py:49 rotates the normalised attention
    input with it) and src/ops.rs:465-499.  x is [..., seq, dim]: positions run along axis -2,
    the pairs (x_2i, x_2i+1) of the whole last axis rotate by pos * base^(-2i / dim).
    `inverse=True` rotates back: the backward (functional.py:316-345, ops.rs:501-530).  Returns
    a new tensor in x's dtype; device tensors only, dim even (above 8192 the rows must be
    16-byte aligned, as contiguous torch allocations are)."""
    if not _is_device_tensor(x):
        raise TypeError("fused_rope_interleaved takes torch tensors on a ROCm device")
    if x.dim() < 2:
        raise ValueError("fused_rope_interleaved: x must be [..., seq, dim]")
    seq, dim = x.shape[-2], x.shape[-1]
    if dim % 2 != 0:
        raise ValueError(f"fused_rope_interleaved: dim={dim} must be even (RoPE pairs)")
    if dim == 0:
        return torch.empty_like(x)
    outer = math.prod(x.shape[:-2])
    return _rope_device(x, (outer, seq, 1, dim), dim, base, inverse,
                        pairing=_lib.ROPE_INTERLEAVED)


def fused_rmsnorm_residual_forward_mx(x: torch.Tensor, residual: Optional[torch.Tensor] = None,
                                      weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
                                      fmt: str = "e4m3"):
    """The forward with y quantised to an OCP MX block format, in the same pass.

    fmt "e4m3" (MXFP8) or "e2m1" (MXFP4).  Returns (y_q, y_scales, h, inv_rms): y_q is a
    float8_e4m3fn tensor shaped like x, or float4_e2m1fn_x2 with the last dimension halved (two
    elements per byte, the even one in the low nibble); y_scales is float8_e8m0fnu [..., D/32],
    one power-of-two scale per 32 consecutive elements of a row (2^(floor(log2(amax)) - emax)).
    D must be a multiple of 32.  Device tensors only; the element formats are the reference's
    (include/velograd/kernels.h:29-37, 47-51).
    """
    if not _is_device_tensor(x):
        raise TypeError("fused_rmsnorm_residual_forward_mx takes torch tensors on a ROCm device")
    if fmt not in ("e4m3", "e2m1"):
        raise ValueError(f"fmt must be 'e4m3' or 'e2m1', got {fmt!r}")
    return _forward_device(x, residual, weight, eps, mx=fmt)


def rmsnorm_forward(x: torch.Tensor, weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
                    min_mean_sq: float = 1e-12) -> Tuple[torch.Tensor, torch.Tensor]:
    """Residual-free RMSNorm as the reference module computes it (python/velograd/nn.py:338-355).

    mean_sq = max(min_mean_sq, mean(x^2)) per row (the reference floors at 1e-12, nn.py:349; as
    Python's max does, a NaN mean square becomes the floor), inv_rms = 1 / sqrt(mean_sq + eps),
    y = x * inv_rms * weight.  Returns (y, inv_rms) with y in x's dtype and inv_rms float32
    [..., 1].  min_mean_sq = 0 is fused_rmsnorm_residual_forward without a residual.  Device
    tensors only; the module's backward is fused_rmsnorm_residual_backward(g, x, weight,
    inv_rms, saved_is_h=True).
    """
    if not _is_device_tensor(x):
        raise TypeError("rmsnorm_forward takes torch tensors on a ROCm device")
    if x.dim() == 0 or x.shape[-1] == 0:
        raise ValueError("rmsnorm_forward needs a non-empty last dimension")
    y, _, inv_rms = _forward_device(x, None, weight, eps, min_mean_sq=min_mean_sq)
    return y, inv_rms


def rmsnorm_rope_forward(x: torch.Tensor, weight: Optional[torch.Tensor] = None,
                         eps: float = 1e-6, base: float = 10000.0,
                         residual: Optional[torch.Tensor] = None,
                         min_mean_sq: float = 1e-12):
    """The reference model's attention-branch input in one pass: `attention_norm(x)` (its
    module RMSNorm, nn.py:338-355, with the 1e-12 floor) then `F.apply_rotary_emb` of the result
    (functional.py:287-315, interleaved pairs, positions along axis -2), as models/llama.py:48-49
    chains them; with `residual`, h = x + residual is normalised (and returned).

    Returns (y, h, inv_rms): y the rotated normalised rows in x's dtype, h as
    fused_rmsnorm_residual_forward (x itself without residual), inv_rms float32 [..., 1].  The
    backward is the inverse rotation of grad_y (fused_rope_interleaved(..., inverse=True)) then
    fused_rmsnorm_residual_backward with saved_is_h=True, which rmsnorm_rope_backward does in
    one pass (nn.rms_norm_rope uses it).  Device tensors only; x is [..., seq, dim] with dim
    even.
    """
    if not _is_device_tensor(x):
        raise TypeError("rmsnorm_rope_forward takes torch tensors on a ROCm device")
    if x.dim() < 2:
        raise ValueError("rmsnorm_rope_forward: x must be [..., seq, dim]")
    min_mean_sq = _check_min_mean_sq(min_mean_sq)
    seq, d = x.shape[-2], x.shape[-1]
    if d % 2 != 0:
        raise ValueError(f"rmsnorm_rope_forward: dim={d} must be even (RoPE pairs)")
    code = _dtype_code(x, "x")
    device = x.device
    if residual is not None:
        if (not isinstance(residual, torch.Tensor) or residual.device != device
                or residual.dtype != x.dtype or residual.shape != x.shape):
            raise ValueError("residual must be a tensor shaped and typed like x on its device")
    w, wcode = _prep_weight(weight, d, x.dtype, device)
    y = torch.empty(x.shape, dtype=x.dtype, device=device)
    h = torch.empty(x.shape, dtype=x.dtype, device=device) if residual is not None else x
    inv_rms = torch.empty(tuple(x.shape[:-1]) + (1,), dtype=torch.float32, device=device)
    if x.numel() == 0:
        return y, h, inv_rms
    x2 = x.contiguous().view(-1, d)
    r2 = residual.contiguous().view(-1, d) if residual is not None else None
    rows = x2.shape[0]
    with torch.cuda.device(device):
        rc = _lib.load().velograd_rmsnorm_rope_fwd(
            x2.data_ptr(), _ptr(r2), _ptr(w), y.data_ptr(),
            h.data_ptr() if residual is not None else None, inv_rms.data_ptr(),
            rows, d, d, d, d, d, seq, code, wcode, float(eps), min_mean_sq, float(base),
            _stream(device))
    _lib.check(rc, "velograd_rmsnorm_rope_fwd")
    return y, h, inv_rms


def rmsnorm_rope_backward(grad_y: torch.Tensor, h: torch.Tensor,
                          weight: Optional[torch.Tensor], inv_rms: torch.Tensor,
                          base: float = 10000.0):
    """Backward of rmsnorm_rope_forward in one pass (velograd_rmsnorm_rope_bwd): grad_y is
    rotated back pair by pair (functional.py:316-345) and the norm's backward runs on it with
    h saved (nn.py:357-383, fused.py:48-66); the same result as
    fused_rmsnorm_residual_backward(fused_rope_interleaved(grad_y, base, inverse=True), h,
    weight, inv_rms, saved_is_h=True) without the intermediate tensor.

    Returns (grad_x, grad_weight): grad_x in grad_y's dtype (also the residual's gradient when
    the forward had one), grad_weight float32 [D] or None without weight.  h is the forward's
    h (x itself without residual); device tensors [..., seq, dim] only.
    """
    if not _is_device_tensor(grad_y):
        raise TypeError("rmsnorm_rope_backward takes torch tensors on a ROCm device")
    if grad_y.dim() < 2:
        raise ValueError("rmsnorm_rope_backward: grad_y must be [..., seq, dim]")
    seq, d = grad_y.shape[-2], grad_y.shape[-1]
    if d % 2 != 0:
        raise ValueError(f"rmsnorm_rope_backward: dim={d} must be even (RoPE pairs)")
    code = _dtype_code(grad_y, "grad_y")
    device = grad_y.device
    if (not isinstance(h, torch.Tensor) or h.device != device or h.dtype != grad_y.dtype
            or h.shape != grad_y.shape):
        raise ValueError("h must be a tensor shaped and typed like grad_y on its device")
    rows = math.prod(grad_y.shape[:-1])
    if not isinstance(inv_rms, torch.Tensor) or inv_rms.device != device:
        raise ValueError("inv_rms must be a tensor on the same device as grad_y")
    if inv_rms.numel() != rows:
        raise ValueError(f"inv_rms has {inv_rms.numel()} elements, expected one per row ({rows})")
    r = inv_rms.reshape(rows).to(torch.float32).contiguous()
    w, wcode = _prep_weight(weight, d, grad_y.dtype, device)
    dx = torch.empty(grad_y.shape, dtype=grad_y.dtype, device=device)
    dweight = torch.empty((d,), dtype=torch.float32, device=device) if w is not None else None
    if rows == 0 or d == 0:
        if dweight is not None:
            dweight.zero_()
        return dx, dweight
    g2 = grad_y.contiguous().view(-1, d)
    h2 = h.contiguous().view(-1, d)
    ws = None
    ws_bytes = 0
    if dweight is not None:
        ws_bytes = bwd_workspace_bytes(rows, d, device)
        ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=device)
    with torch.cuda.device(device):
        rc = _lib.load().velograd_rmsnorm_rope_bwd(
            g2.data_ptr(), h2.data_ptr(), _ptr(w), r.data_ptr(), dx.data_ptr(), _ptr(dweight),
            _ptr(ws), ws_bytes, rows, d, d, d, d, seq, code, wcode, float(base),
            _stream(device))
    _lib.check(rc, "velograd_rmsnorm_rope_bwd")
    return dx, dweight


def fused_rmsnorm_residual(x: Any, residual: Optional[Any] = None, weight: Optional[Any] = None,
                           eps: float = 1e-6):
    """Wrapper returning only the normalised output, like kernels/__init__.py:19-32."""
    return fused_rmsnorm_residual_forward(x, residual, weight, eps)[0]
