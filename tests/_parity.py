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
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def weight_vec(rng: np.random.Generator, d: int) -> np.ndarray:
    return (1.0 + 0.1 * rng.standard_normal(d, dtype=np.float32)).astype(np.float32)


def with_outliers(rng: np.random.Generator, a: np.ndarray, frac: float = 1e-3,
                  factor: float = 50.0) -> np.ndarray:
    n = a.size
    k = max(1, int(round(n * frac)))
    idx = rng.choice(n, size=k, replace=False)
    out = a.copy().reshape(-1)
    out[idx] *= np.float32(factor)
    return out.reshape(a.shape)


def to_device(a: np.ndarray, dtype: torch.dtype, device="cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(device)


def upcast(t: torch.Tensor) -> np.ndarray:
    """The values a reduced-precision tensor really holds, as fp32 numpy."""
    return t.detach().float().cpu().numpy()
