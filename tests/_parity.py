"""Tolerances and seeded inputs shared by the parity tests.

Tolerances (the north star's gates, written out):
  * fp32 outputs: max over elements of |a - b| / (|b| + 1e-6) <= 1e-5 (the reference's
    relative-error convention, tests/test_velograd_v41_enterprise_verification.py:213).
  * bf16 / fp16 outputs y and h: within 1 ulp of the fp32 oracle evaluated on the same upcast
    inputs and rounded to nearest even (h is in fact bit-exact).
  * dx in bf16 / fp16: 1 ulp as above, or |a - b| <= 2^-20 * S + half an output ulp, where
    S = |r*gw| + |r*xhat| * mean(|gw*xhat|) is the operand scale of dx = r*(gw - xhat*m): the
    first term bounds the subtraction, the second bounds the error of the row mean m, whose
    terms cancel (so no order of summation makes |m| itself the scale).
  * dx in fp32: |a - b| <= 1e-5 * S.
  * with a residual-stream gradient grad_h added to dx, S also includes |grad_h|.
  * dweight (fp32): |a - b| <= 1e-3 * max(|b|, rms(b)) elementwise.
"""

from __future__ import annotations

import numpy as np
import torch

FP32_REL_TOL = 1e-5
DWEIGHT_REL_TOL = 1e-3
DX_FLOOR = 2.0 ** -20


def rel_err(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    if a.size == 0:
        return 0.0
    return float(np.max(np.abs(a - b) / (np.abs(b) + 1e-6)))


def _ordered_bits(t: torch.Tensor) -> torch.Tensor:
    """Map 16-bit float patterns to integers whose order and spacing follow the float line."""
    bits = t.contiguous().view(torch.int16).to(torch.int32)
    mag = bits & 0x7FFF
    return torch.where(bits < 0, -mag, mag)


def ulp_distance(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Distance in units of the last place between two bf16/fp16 tensors (NaN==NaN -> 0)."""
    assert a.dtype == b.dtype and a.dtype in (torch.bfloat16, torch.float16)
    d = (_ordered_bits(a) - _ordered_bits(b)).abs()
    both_nan = torch.isnan(a) & torch.isnan(b)
    return torch.where(both_nan, torch.zeros_like(d), d)


def round_like(ref32: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    """fp32 oracle result rounded to `dtype` nearest-even (torch's CPU cast)."""
    return torch.from_numpy(np.ascontiguousarray(ref32, dtype=np.float32)).to(dtype)


def assert_within_ulp(got: torch.Tensor, ref32: np.ndarray, ulps: int = 1, what: str = ""):
    got = got.detach().cpu()
    ref = round_like(ref32, got.dtype).reshape(got.shape)
    d = ulp_distance(got, ref)
    worst = int(d.max()) if d.numel() else 0
    assert worst <= ulps, f"{what}: {worst} ulp apart (allowed {ulps}); " \
                          f"{int((d > ulps).sum())} elements over"


def dx_scale(gw: np.ndarray, xhat: np.ndarray, r: np.ndarray) -> np.ndarray:
    """Operand scale S of dx = r*(gw - xhat*m) (see the module docstring)."""
    gw = np.asarray(gw, np.float64)
    xhat = np.asarray(xhat, np.float64)
    r = np.asarray(r, np.float64)
    return np.abs(r * gw) + np.abs(r * xhat) * np.mean(np.abs(gw * xhat), axis=-1, keepdims=True)


def assert_dx_fp32(got: torch.Tensor, ref32: np.ndarray, gw, xhat, r, what: str = "dx"):
    g = got.detach().cpu().numpy().reshape(ref32.shape).astype(np.float64)
    err = np.abs(g - ref32.astype(np.float64)) / (dx_scale(gw, xhat, r) + 1e-30)
    assert float(np.max(err)) <= FP32_REL_TOL, f"{what}: scaled error {float(np.max(err)):.3e}"


def dx_check(got: torch.Tensor, ref32: np.ndarray, gw: np.ndarray, xhat: np.ndarray,
             r: np.ndarray, what: str = "dx", grad_h=None) -> int:
    """1-ulp test with the operand-scaled fp32 floor; returns how many needed the floor.
    With a residual-stream gradient added to dx, |grad_h| joins the operand scale."""
    got_c = got.detach().cpu()
    ref = round_like(ref32, got_c.dtype).reshape(got_c.shape)
    d = ulp_distance(got_c, ref).numpy()
    bad = d > 1
    n_floor = int(bad.sum())
    if n_floor:
        g = got_c.float().numpy().reshape(ref32.shape).astype(np.float64)
        diff = np.abs(g - ref32.astype(np.float64))
        scale = dx_scale(gw, xhat, r)
        if grad_h is not None:
            scale = scale + np.abs(np.asarray(grad_h, np.float64))
        floor = DX_FLOOR * scale
        # Rounding the fp32 value to the output dtype adds up to half an ulp of it.
        half_ulp = np.abs(ref.float().numpy().reshape(ref32.shape)) * 2.0 ** -8
        ok = diff <= floor + half_ulp
        assert np.all(ok[bad]), f"{what}: {int((~ok & bad).sum())} elements beyond 1 ulp and floor"
    return n_floor


def assert_dweight(got: np.ndarray, ref: np.ndarray, what: str = "dweight"):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    scale = np.maximum(np.abs(ref), np.sqrt(np.mean(ref * ref)) if ref.size else 0.0)
    err = np.abs(got - ref)
    assert np.all(err <= DWEIGHT_REL_TOL * scale), \
        f"{what}: worst scaled error {float(np.max(err / np.maximum(scale, 1e-30))):.3e}"


# ---------------------------------------------------------------------------------------------
# Seeded inputs (numpy default_rng in fp32, cast to the target dtype with torch RNE).
# ---------------------------------------------------------------------------------------------
def gaussian(rng: np.random.Generator, shape, std: float = 1.0) -> np.ndarray:
    a = rng.standard_normal(shape, dtype=np.float32)
    if std != 1.0:
        a *= np.float32(std)  # in place: the same float32 products, no extra copy
    return a


def weight_vec(rng: np.random.Generator, d: int) -> np.ndarray:
    return (1.0 + 0.1 * rng.standard_normal(d, dtype=np.float32)).astype(np.float32)


def with_outliers(rng: np.random.Generator, a: np.ndarray, frac: float = 1e-3,
                  factor: float = 50.0, inplace: bool = False) -> np.ndarray:
    """`a` with round(frac * size) distinct, uniformly chosen entries scaled by `factor`."""
    n = a.size
    k = max(1, int(round(n * frac)))
    idx = rng.choice(n, size=k, replace=False)
    out = a if inplace else a.copy()
    out.reshape(-1)[idx] *= np.float32(factor)
    return out


def to_device(a: np.ndarray, dtype: torch.dtype, device="cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(device)


def upcast(t: torch.Tensor) -> np.ndarray:
    """The values a reduced-precision tensor really holds, as fp32 numpy."""
    return t.detach().float().cpu().numpy()


# ---------------------------------------------------------------------------------------------
# Fused RoPE.  A float32 RoPE computes the angle pos * freq in float32, so a difference of a few
# float32 ulps in freq (NumPy's float32 power is faithful, not correctly rounded) moves the angle
# by a few ulps of |angle|, and the output by that many radians times |x1| + |x2|; cos and sin
# add ~1.5 ulp each and the products and the sum a few more ulps of |x1| + |x2|.  The tolerance
# for each rotated element of a pair (x1, x2) at angle a:
#     |got - want| <= (ROPE_ANGLE_ULPS * 2^-24 * max(|a|, 1) + 2^-21) * (|x1| + |x2|)
# Elements past head_dim are copied and must be exact.
# ---------------------------------------------------------------------------------------------
ROPE_ANGLE_ULPS = 16


def rope_canonical(a: np.ndarray, head_dim: int) -> np.ndarray:
    """View an input as [T, S, H, D] the way fused.py:86-96 reads it."""
    a = np.asarray(a)
    if a.ndim == 2:
        if a.shape[-1] > head_dim:
            return a.reshape(1, a.shape[0], a.shape[1] // head_dim, head_dim)
        return a.reshape(1, a.shape[0], 1, a.shape[1])
    return a.reshape(-1, *a.shape[-3:])


def rope_angles(seq_len: int, head_dim: int, theta: float) -> np.ndarray:
    """Exact (float64) angles pos * theta^(-2j/head_dim), shape [seq_len, head_dim // 2]."""
    j = np.arange(head_dim // 2, dtype=np.float64)
    return np.outer(np.arange(seq_len, dtype=np.float64), theta ** (-2.0 * j / head_dim))


def rope_truth(x: np.ndarray, head_dim: int, theta: float, inverse: bool = False) -> np.ndarray:
    """float64 rotate-half RoPE of a canonical [T, S, H, D] array, from the exact angles."""
    x = np.asarray(x, dtype=np.float64)
    half = head_dim // 2
    ang = rope_angles(x.shape[1], head_dim, theta)[None, :, None, :]
    c, s = np.cos(ang), np.sin(ang) * (-1.0 if inverse else 1.0)
    x1, x2 = x[..., :half], x[..., half:head_dim]
    return np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c, x[..., head_dim:]], axis=-1)


def rope_bound(x: np.ndarray, head_dim: int, theta: float) -> np.ndarray:
    """Per-element tolerance for a canonical [T, S, H, D] input (see the comment above)."""
    x = np.abs(np.asarray(x, dtype=np.float64))
    half = head_dim // 2
    ang = np.maximum(np.abs(rope_angles(x.shape[1], head_dim, theta)), 1.0)[None, :, None, :]
    mag = x[..., :half] + x[..., half:head_dim]
    b = (ROPE_ANGLE_ULPS * 2.0 ** -24 * ang + 2.0 ** -21) * mag
    return np.concatenate([b, b, np.zeros_like(x[..., head_dim:])], axis=-1)


def assert_rope_close(got: np.ndarray, want: np.ndarray, x: np.ndarray, head_dim: int,
                      theta: float, extra: float = 0.0, what: str = "rope"):
    """|got - want| <= rope_bound + extra * |want| elementwise (canonical arrays); `extra`
    allows the rounding of a reduced-precision output."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    tol = rope_bound(x, head_dim, theta) + extra * np.abs(want)
    err = np.abs(got - want)
    bad = err > tol
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} elements out of tolerance; "
                           f"worst excess {float((err - tol).max()):.3e}")
