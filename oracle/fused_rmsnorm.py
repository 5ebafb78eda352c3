"""CPU oracle of VeloGrad's fused RMSNorm + residual path — TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import
this module, and only as the checker or the reported CPU baseline.  The product
(`velograd_amd`) never calls it: it has no CPU fallback.

What it is: a NumPy restatement, operation for operation, of the reference's CPU path
  * forward   python/velograd/kernels/fused.py:28-46
  * backward  python/velograd/kernels/fused.py:48-66
  * wrapper   python/velograd/kernels/__init__.py:19-32 (array-like inputs only)
The functions are dtype-generic: float32 inputs reproduce the reference's float32 rounding
sequence on the same NumPy build; float64 inputs give the "truth" used to judge rounding.

How it is pinned (tests/test_oracle.py):
  * golden vectors in tests/golden/ computed by tests/golden/make_golden.py with exact
    rational arithmetic and 60-digit decimals, independent of NumPy; the backward's vectors come
    from central finite differences of the forward, not from the analytic formula;
  * the reference's own known answers: the Rust RMSNorm test
    (tests/core_engine_tests.rs:243-247, y0 = 0.365148 for x = [1,2,3,4]) and the gradcheck
    inputs of tests/test_velograd_beast.py:121 and tests/test_velograd_omnibus_grand_master.py:125
    checked with the reference's finite-difference rule (python/velograd/autograd.py:55-128);
  * an independent library: torch.nn.functional.rms_norm and torch autograd on the CPU;
  * closed forms (constant row, zero row), invariants (scale invariance, sum(dh*h) ~ 0 as
    eps -> 0) and NaN/Inf propagation.
Parity status: forward and backward are pinned; bit-exactness to the reference's own NumPy
rounding sequence is not separately pinned (the reference module is not imported), which the
stated tolerances make unnecessary.

Beyond the reference's RMSNorm functions (pins in tests/test_fp8_codec.py and
tests/test_rope_oracle.py):
  * backward_with_residual_grad: torch autograd of the pre-norm block (tests/test_oracle.py);
  * rmsnorm_module_forward / rmsnorm_module_backward (the reference module velograd.nn.RMSNorm,
    python/velograd/nn.py:338-383, with its 1e-12 floor on the mean square;
    tests/test_rmsnorm_module_oracle.py): the reference test's own ground-truth loop
    (tests/test_velograd_v41_enterprise_verification.py:221-229), the Rust known answer, torch's
    rms_norm and autograd where the floor is inactive, closed forms where it is active (eps = 0
    zero and tiny rows, the boundary), Python's max on NaN and Inf, and the reference's gradcheck
    rule on its own input;
  * e4m3fn_decode / e4m3fn_encode / quantize_rows_e4m3 / fused_rmsnorm_residual_forward_fp8
    (the fp8 output epilogue, format of include/velograd/kernels.h:29-37,58-73): torch's
    float8_e4m3fn casts over every code and a dense set of values, the reference decoder's
    values, round-trip and rounding bounds, and the per-row scale facts (largest element maps
    to 448, dequantisation error bound);
  * rope_tables / fused_rope_forward / fused_rope (fused.py:72-130, kernels/__init__.py:34-48):
    float64 truth from the exact angles and torch's rotate-half form within an angle-scaled
    tolerance, position 0 = identity, pair norms, the relative-position property, the adjoint
    identity of the inverse rotation, and the reference test's own call.
Each set of pins is shown to catch planted mistakes.  No function here is "parity unpinned".
"""

from __future__ import annotations

from typing import Optional, Tuple

import numpy as np


def fused_rmsnorm_residual_forward(x: np.ndarray, residual: Optional[np.ndarray] = None,
                                   weight: Optional[np.ndarray] = None,
                                   eps: float = 1e-6) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """fused.py:28-46: returns (normed, h, inv_rms) with the reference's op order."""
    h = x if residual is None else (x + residual)                 # fused.py:39
    mean_sq = np.mean(h ** 2, axis=-1, keepdims=True)              # fused.py:41
    inv_rms = 1.0 / np.sqrt(mean_sq + eps)                         # fused.py:42
    normed = h * inv_rms                                           # fused.py:43
    if weight is not None:                                         # fused.py:44-45
        normed = normed * weight
    return normed, h, inv_rms


def fused_rmsnorm_residual_backward(grad_out: np.ndarray, normed_input: np.ndarray,
                                    weight: Optional[np.ndarray],
                                    inv_rms: np.ndarray) -> Tuple[np.ndarray, Optional[np.ndarray]]:
    """fused.py:48-66: returns (grad_x, grad_weight); normed_input is xhat = h * inv_rms."""
    gw = grad_out if weight is None else (grad_out * weight)                     # fused.py:58
    mean_gw_x = np.mean(gw * normed_input, axis=-1, keepdims=True)             # fused.py:59
    grad_x = inv_rms * (gw - normed_input * mean_gw_x)                         # fused.py:60
    grad_weight = None
    if weight is not None:                                                     # fused.py:62-65
        axes_to_sum = tuple(range(normed_input.ndim - 1))
        grad_weight = np.sum(grad_out * normed_input, axis=axes_to_sum)
    return grad_x, grad_weight


def backward_from_h(grad_out: np.ndarray, h: np.ndarray, weight: Optional[np.ndarray],
                    inv_rms: np.ndarray) -> Tuple[np.ndarray, Optional[np.ndarray]]:
    """Backward when the caller saved h: xhat = h * inv_rms (fused.py:43), then fused.py:48-66."""
    return fused_rmsnorm_residual_backward(grad_out, h * inv_rms, weight, inv_rms)


def backward_with_residual_grad(grad_out: np.ndarray, normed_input: np.ndarray,
                                weight: Optional[np.ndarray], inv_rms: np.ndarray,
                                grad_h: np.ndarray) -> Tuple[np.ndarray, Optional[np.ndarray]]:
    """fused.py:48-66 plus the gradient that reaches h from its other consumer.

    In a pre-norm block h = x + residual feeds both the norm and the next residual add
    (python/velograd/models/llama.py:48-56), so dL/dh = (norm backward, fused.py:60) + grad_h,
    added once in the working precision.  dweight is unchanged.
    """
    grad_x, grad_weight = fused_rmsnorm_residual_backward(grad_out, normed_input, weight, inv_rms)
    return grad_x + grad_h, grad_weight


def fused_rmsnorm_residual(x, residual=None, weight=None, eps: float = 1e-6) -> np.ndarray:
    """kernels/__init__.py:19-32 for array-like inputs: cast to float32, return only y."""
    x_arr = np.asarray(x, dtype=np.float32)                                     # :21
    res_arr = None if residual is None else np.asarray(residual, dtype=np.float32)   # :22-24
    w_arr = None if weight is None else np.asarray(weight, dtype=np.float32)   # :25-27
    normed, _, _ = fused_rmsnorm_residual_forward(x_arr, res_arr, w_arr, eps)   # :29
    return normed                                                               # :32


# ---------------------------------------------------------------------------------------------
# The reference's module `velograd.nn.RMSNorm` (python/velograd/nn.py:328-389): residual-free,
# mean square floored at 1e-12, computed in Python floats (float64), row by row.
# ---------------------------------------------------------------------------------------------
MODULE_MIN_MEAN_SQ = 1e-12                                                      # nn.py:349


def rmsnorm_module_forward(x, weight=None, eps: float = 1e-6,
                           min_mean_sq: float = MODULE_MIN_MEAN_SQ):
    """nn.py:338-355 in float64: returns (y, inv_rms [..., 1])."""
    x = np.asarray(x, dtype=np.float64)
    dim = x.shape[-1]
    # nn.py:349 sum(x ** 2 for x in row) / dim, summed left to right (cumsum is sequential)
    mean_sq = np.cumsum(x ** 2, axis=-1)[..., -1:] / dim
    # nn.py:349 max(1e-12, mean_sq): Python's max keeps its first argument unless a later one
    # compares greater, so a NaN mean square becomes the floor
    mean_sq = np.where(mean_sq > min_mean_sq, mean_sq, min_mean_sq)
    rms = np.sqrt(mean_sq + eps)                                                # nn.py:350
    inv_rms = 1.0 / rms                                                         # nn.py:351
    y = x * inv_rms                                                             # nn.py:355
    if weight is not None:
        y = y * np.asarray(weight, dtype=np.float64).reshape(-1)
    return y, inv_rms


def rmsnorm_module_backward(grad, x, weight, inv_rms):
    """nn.py:357-383 in float64: returns (grad_x, grad_weight [dim] or None)."""
    g = np.asarray(grad, dtype=np.float64)
    x = np.asarray(x, dtype=np.float64)
    inv = np.asarray(inv_rms, dtype=np.float64)
    dim = x.shape[-1]
    w = np.ones(dim) if weight is None else np.asarray(weight, dtype=np.float64).reshape(-1)
    grad_w = None
    if weight is not None:                                                      # nn.py:361-367
        grad_w = np.sum((g * x * inv).reshape(-1, dim), axis=0)
    sum_dy_w_x = np.sum(g * w * x, axis=-1, keepdims=True)                      # nn.py:376-378
    dy_w = g * w                                                                # nn.py:381
    grad_x = inv * (dy_w - x * (inv ** 2) * sum_dy_w_x / dim)                   # nn.py:382
    return grad_x, grad_w


# ---------------------------------------------------------------------------------------------
# fp8 output epilogue (quantised y for the next GEMM).  The reference has no fused quantising
# forward; its E4M3 format is fixed by include/velograd/kernels.h:29-37 (PrecisionMode::FP8_E4M3)
# and the decoder at kernels.h:58-73 (bias 7, subnormals 2^-6 * m/8, S.1111.111 not a number).
# ---------------------------------------------------------------------------------------------
E4M3_MAX = np.float32(448.0)


def e4m3fn_decode(codes: np.ndarray) -> np.ndarray:
    """OCP e4m3fn byte -> float32: (-1)^s * 2^(e-7) * (1 + m/8), subnormal 2^-6 * m/8, NaN at
    S.1111.111 (kernels.h:58-73 decodes the same values but returns 0 for the NaN codes)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    e = (c >> 3) & 0xF
    m = c & 7
    mag = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    mag = np.where((c & 0x7F) == 0x7F, np.nan, mag)
    return np.where((c >> 7) == 1, -mag, mag).astype(np.float32)


# The 127 non-negative finite values, codes 0x00..0x7E, in ascending order.
_E4M3_TABLE = e4m3fn_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)


def e4m3fn_encode(v: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn byte: the nearest finite value (ties to the even code), saturating at
    +-448 (infinities included); NaN -> 0x7F with v's sign.  Written as a nearest-value search
    over the table above, not with the bit arithmetic the device code uses."""
    v = np.asarray(v, dtype=np.float32)
    with np.errstate(invalid="ignore"):  # signalling-NaN bit patterns
        a = np.abs(v).astype(np.float64)
    nan = np.isnan(a)
    a = np.where(nan, 0.0, np.minimum(a, 448.0))
    hi = np.clip(np.searchsorted(_E4M3_TABLE, a, side="left"), 1, 0x7E)
    lo = hi - 1
    d_lo = a - _E4M3_TABLE[lo]
    d_hi = _E4M3_TABLE[hi] - a
    code = np.where(d_lo < d_hi, lo, np.where(d_hi < d_lo, hi, np.where(lo % 2 == 0, lo, hi)))
    code = np.where(nan, 0x7F, code)
    return (code | (np.signbit(v).astype(np.int64) << 7)).astype(np.uint8)


def e4m3_inverse_scale(scale: np.ndarray) -> np.ndarray:
    """1 / scale in float32, or 1 where scale is below the smallest normal float (zero rows, and
    scales whose reciprocal could overflow); NaN stays NaN."""
    scale = np.asarray(scale, dtype=np.float32)
    tiny = np.float32(np.finfo(np.float32).tiny)
    with np.errstate(divide="ignore", invalid="ignore"):
        return np.where(scale < tiny, np.float32(1), np.float32(1) / scale).astype(np.float32)


def quantize_rows_e4m3(y: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """Per-row fp8 quantisation: amax = max|y| over the last axis (NaN propagates),
    scale = amax / 448 in float32, codes = e4m3(y * e4m3_inverse_scale(scale))."""
    y = np.asarray(y, dtype=np.float32)
    amax = np.max(np.abs(y), axis=-1, keepdims=True)
    scale = (amax / E4M3_MAX).astype(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        v = y * e4m3_inverse_scale(scale)
    return e4m3fn_encode(v), scale


def fused_rmsnorm_residual_forward_fp8(x: np.ndarray, residual: Optional[np.ndarray] = None,
                                       weight: Optional[np.ndarray] = None, eps: float = 1e-6,
                                       inv_rms: Optional[np.ndarray] = None):
    """fused.py:28-46 followed by quantize_rows_e4m3 of y.  Returns (codes, scale, h, inv_rms).

    Given `inv_rms` (e.g. the device's), y = (h * inv_rms) * weight is formed from it instead of
    the recomputed statistic, so that every later step is elementwise and exactly reproducible.
    """
    y, h, r = fused_rmsnorm_residual_forward(x, residual, weight, eps)
    if inv_rms is not None:
        r = np.asarray(inv_rms, dtype=h.dtype).reshape(r.shape)
        y = h * r
        if weight is not None:
            y = y * weight
    codes, scale = quantize_rows_e4m3(y)
    return codes, scale, h, r


# ---------------------------------------------------------------------------------------------
# Fused RoPE (rotary position embedding), the reference's second fused kernel:
#   python/velograd/kernels/fused.py:72-130 (fused_rope_forward) and the wrapper
#   python/velograd/kernels/__init__.py:34-48 (fused_rope).  Pairs are (j, j + half) of each
# head vector ("rotate half"), the position is the index along axis -3 (axis 0 for 2-D input),
# and the last axis beyond head_dim passes through unchanged.
# ---------------------------------------------------------------------------------------------
def rope_tables(seq_len: int, head_dim: int, theta: float = 10000.0, dtype=np.float32):
    """fused.py:98-103: (cos, sin) of shape [seq_len, head_dim // 2] in `dtype`."""
    half = head_dim // 2
    pos = np.arange(seq_len, dtype=dtype)                               # :98
    dim_pairs = np.arange(half, dtype=dtype)                            # :99
    freqs = 1.0 / (theta ** (2.0 * dim_pairs / head_dim))              # :100
    angles = np.outer(pos, freqs)                                        # :101
    return np.cos(angles), np.sin(angles)                                # :102-103


def fused_rope_forward(q: np.ndarray, k: Optional[np.ndarray] = None,
                       head_dim: Optional[int] = None, theta: float = 10000.0,
                       inverse: bool = False):
    """fused.py:72-130 op for op.  `inverse=True` rotates by -angle instead (the adjoint, i.e.
    the backward: the reference's rotary backward rule, src/ops.rs:501-530, for this pairing)."""
    orig_shape = q.shape
    h_dim = head_dim or q.shape[-1]                                      # :83
    half_dim = h_dim // 2                                                # :84
    need_reshape = False
    if q.ndim == 2 and q.shape[-1] > h_dim:                              # :88-94
        need_reshape = True
        num_heads = q.shape[-1] // h_dim
        q = q.reshape(q.shape[0], num_heads, h_dim)
        if k is not None and isinstance(k, np.ndarray) and k.ndim == 2:
            k = k.reshape(k.shape[0], num_heads, h_dim)
    seq_dim = -3 if q.ndim >= 3 else 0                                   # :96
    seq_len = q.shape[seq_dim]                                           # :97
    cos_vals, sin_vals = rope_tables(seq_len, h_dim, theta)              # float32, :98-103
    if inverse:
        sin_vals = -sin_vals
    shape_pad = [1] * q.ndim                                             # :106-111
    shape_pad[seq_dim] = seq_len
    shape_pad[-1] = half_dim
    cos_vals = cos_vals.reshape(shape_pad)
    sin_vals = sin_vals.reshape(shape_pad)

    def _apply_rope(t):                                                  # :113-121
        x1 = t[..., :half_dim]
        x2 = t[..., half_dim:h_dim]
        rot_1 = x1 * cos_vals - x2 * sin_vals
        rot_2 = x1 * sin_vals + x2 * cos_vals
        res = np.concatenate([rot_1, rot_2], axis=-1)
        if t.shape[-1] > h_dim:
            res = np.concatenate([res, t[..., h_dim:]], axis=-1)
        return res

    q_rot = _apply_rope(q)                                               # :123
    k_rot = _apply_rope(k) if (k is not None and isinstance(k, np.ndarray)) else None
    if need_reshape:                                                     # :126-129
        q_rot = q_rot.reshape(orig_shape)
        if k_rot is not None:
            k_rot = k_rot.reshape(orig_shape)
    return q_rot, k_rot


def fused_rope(x, k=None, head_dim: Optional[int] = None, base: float = 10000.0):
    """kernels/__init__.py:34-48 for array-like inputs: float32 casts; q_rot, or (q_rot, k_rot)
    when k is given."""
    x_arr = np.asarray(x, dtype=np.float32)                              # :36
    k_arr = np.asarray(k, dtype=np.float32) if k is not None else None  # :37
    q_rot, k_rot = fused_rope_forward(x_arr, k_arr, head_dim=head_dim, theta=base)   # :39
    if k is not None:                                                    # :46-48
        return q_rot, k_rot
    return q_rot


def apply_rotary_emb(x, base: float = 10000.0, inverse: bool = False,
                     positions=None) -> np.ndarray:
    """python/velograd/functional.py:287-315 (forward) and :316-345 (inverse = the backward's
    rotation) in float64, the precision of the reference's Python floats: interleaved pairs
    (x_2i, x_2i+1) of the last axis, position = index along axis -2.  `positions` (one per index
    of axis -2) replaces that index, for rows taken out of a longer sequence."""
    x = np.asarray(x, dtype=np.float64)
    seq_len, dim = x.shape[-2], x.shape[-1]                              # :289-290
    assert dim % 2 == 0, "Dimension must be even for RoPE pairs"         # :291
    i = np.arange(dim // 2, dtype=np.float64)
    theta = 1.0 / (base ** ((2.0 * i) / float(dim)))                     # :302
    pos = (np.arange(seq_len, dtype=np.float64) if positions is None
           else np.asarray(positions, dtype=np.float64).reshape(seq_len))
    angle = pos[:, None] * theta                                         # :303
    cos_val, sin_val = np.cos(angle), np.sin(angle)                      # :304-305
    if inverse:
        sin_val = -sin_val
    x0, x1 = x[..., 0::2], x[..., 1::2]                                  # :307-311
    out = np.empty_like(x)
    out[..., 0::2] = x0 * cos_val - x1 * sin_val                         # :313
    out[..., 1::2] = x0 * sin_val + x1 * cos_val                         # :314
    return out


# ---------------------------------------------------------------------------------------------
# OCP Microscaling (MX) block quantisation of y: blocks of 32 consecutive elements of a row share
# one E8M0 scale 2^s with s = floor(log2(amax)) - emax (8 for E4M3, 2 for E2M1), clamped to
# [-127, 127]; elements are round-to-nearest-even, saturating codes of y / 2^s.  All-zero blocks
# take scale code 0; blocks with a non-finite amax take the NaN scale 0xFF and zero codes.  The
# reference's E2M1 table is include/velograd/kernels.h:47-51, its block decode :97-101, 339-347
# (one scale per 32 elements, the even element in the low nibble).
# ---------------------------------------------------------------------------------------------
MX_BLOCK = 32
MX_EMAX = {"e4m3": 8, "e2m1": 2}
E2M1_VALUES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def e2m1_decode(nibbles: np.ndarray) -> np.ndarray:
    """E2M1 nibble -> float32: (-1)^s * 2^(e-1) * (1 + m/2), subnormal 0.5 * m (bias 1)."""
    n = np.asarray(nibbles).astype(np.int64) & 0xF
    e = (n >> 1) & 3
    m = n & 1
    mag = np.where(e == 0, 0.5 * m, np.exp2(e - 1.0) * (1.0 + 0.5 * m))
    return np.where((n >> 3) == 1, -mag, mag).astype(np.float32)


def e2m1_encode(v: np.ndarray) -> np.ndarray:
    """float32 -> E2M1 nibble: the nearest of the 8 magnitudes (ties to the even code),
    saturating at 6; NaN -> 0.  A nearest-value search, not the device's comparison chain."""
    v = np.asarray(v, dtype=np.float32)
    with np.errstate(invalid="ignore"):
        a = np.abs(v).astype(np.float64)
    nan = np.isnan(a)
    a = np.where(nan, 0.0, np.minimum(a, 6.0))
    hi = np.clip(np.searchsorted(E2M1_VALUES, a, side="left"), 1, 7)
    lo = hi - 1
    d_lo, d_hi = a - E2M1_VALUES[lo], E2M1_VALUES[hi] - a
    code = np.where(d_lo < d_hi, lo, np.where(d_hi < d_lo, hi, np.where(lo % 2 == 0, lo, hi)))
    code = np.where(nan, 0, code)
    return (code | (np.signbit(v).astype(np.int64) << 3)).astype(np.uint8)


def e8m0_decode(codes: np.ndarray) -> np.ndarray:
    """E8M0 scale code -> float64 2^(code - 127); 0xFF is NaN."""
    c = np.asarray(codes).astype(np.int64)
    return np.where(c == 0xFF, np.nan, np.exp2(c - 127.0))


def mx_quantize_rows(y: np.ndarray, fmt: str):
    """MX quantisation along the last axis (a multiple of 32).  Returns (codes, scales):
    e4m3 codes [..., D] uint8; e2m1 nibbles packed two per byte [..., D/2] (even element in the
    low nibble); scales [..., D/32] uint8 E8M0 codes."""
    y = np.asarray(y, dtype=np.float32)
    d = y.shape[-1]
    assert d % MX_BLOCK == 0, "MX blocks need a last axis that is a multiple of 32"
    blocks = y.reshape(y.shape[:-1] + (d // MX_BLOCK, MX_BLOCK))
    with np.errstate(invalid="ignore"):
        amax = np.max(np.abs(blocks), axis=-1)
    finite = np.isfinite(amax)
    pos = finite & (amax > 0)
    _, ex = np.frexp(np.where(pos, amax, 1.0).astype(np.float64))  # amax = f * 2^ex, f in [.5,1)
    s = np.where(pos, np.clip(ex - 1 - MX_EMAX[fmt], -127, 127), -127)
    scales = np.where(finite, s + 127, 0xFF).astype(np.uint8)
    factor = np.ldexp(np.float32(1.0), (-np.where(finite, s, 0)).astype(np.int32))[..., None]
    with np.errstate(invalid="ignore", over="ignore"):
        v = (blocks * factor.astype(np.float32)).astype(np.float32)
    if fmt == "e4m3":
        codes = e4m3fn_encode(v)
    else:
        codes = e2m1_encode(v)
    codes = np.where(finite[..., None], codes, 0).astype(np.uint8).reshape(y.shape)
    if fmt == "e2m1":
        codes = (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)
    return codes, scales


def mx_dequantize_rows(codes: np.ndarray, scales: np.ndarray, fmt: str) -> np.ndarray:
    """Inverse of mx_quantize_rows up to the element rounding (float64 values)."""
    if fmt == "e2m1":
        nib = np.stack([codes & 0xF, codes >> 4], axis=-1).reshape(codes.shape[:-1] + (-1,))
        vals = e2m1_decode(nib).astype(np.float64)
    else:
        vals = e4m3fn_decode(codes).astype(np.float64)
    sc = np.repeat(e8m0_decode(scales), MX_BLOCK, axis=-1)
    return vals * sc


def fused_rmsnorm_residual_forward_mx(x, residual=None, weight=None, eps: float = 1e-6,
                                      fmt: str = "e4m3", inv_rms=None):
    """fused.py:28-46 followed by mx_quantize_rows of y (given `inv_rms`, y is formed from it,
    as in fused_rmsnorm_residual_forward_fp8).  Returns (codes, scales, h, inv_rms)."""
    y, h, r = fused_rmsnorm_residual_forward(x, residual, weight, eps)
    if inv_rms is not None:
        r = np.asarray(inv_rms, dtype=h.dtype).reshape(r.shape)
        y = h * r
        if weight is not None:
            y = y * weight
    codes, scales = mx_quantize_rows(y, fmt)
    return codes, scales, h, r
