"""The residual-free forward of the reference's module `velograd.nn.RMSNorm` (nn.py:338-383) on the
GPU, through `rmsnorm_forward` (C entry point velograd_rmsnorm_fwd) and the autograd module,
against the oracle `rmsnorm_module_forward` / `rmsnorm_module_backward` (float64 on the values the
device tensors hold).  Tolerances as tests/_parity.py: fp32 y and inv_rms |a-b|/(|b|+1e-6) <=
1e-5; bf16/fp16 y within 1 ulp; dx with the operand-scaled floor; dweight 1e-3.  Rows where the
1e-12 floor acts (zero and tiny rows, eps = 0), a NaN and an Inf element, and rows just above
the floor are in every case."""

import numpy as np
import pytest
import torch

from oracle import fused_rmsnorm as ora
from tests import _parity as P
from velograd_amd import kernels as vk
from velograd_amd import nn as vnn

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def _rows(rng, rows, d):
    """Gaussian rows, then: 0 zeros, 1 tiny constant (mean square 1e-16), 2 one NaN, 3 one Inf,
    4 constant 1.5e-6 (mean square 2.25e-12, above the floor)."""
    x = P.gaussian(rng, (rows, d))
    x[0] = 0.0
    x[1] = 1e-8
    x[2, d // 2] = np.nan
    x[3, d // 3] = np.inf
    x[4] = 1.5e-6
    return x


def _assert_close_nan_aware(got: np.ndarray, want: np.ndarray, what: str):
    got = np.asarray(got, np.float64).reshape(want.shape)
    assert np.array_equal(np.isnan(got), np.isnan(want)), f"{what}: NaN pattern differs"
    fin = ~np.isnan(want)
    assert np.array_equal(got[fin & np.isinf(want)], want[fin & np.isinf(want)]), what
    m = fin & np.isfinite(want)
    err = np.abs(got[m] - want[m]) / (np.abs(want[m]) + 1e-6)
    assert err.size == 0 or float(err.max()) <= P.FP32_REL_TOL, f"{what}: {float(err.max()):.3e}"


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("d", [4, 768, 1000, 4096, 9000])
@pytest.mark.parametrize("eps", [1e-6, 0.0])
def test_rmsnorm_forward_matches_module_oracle(dtype, d, eps):
    print(f"rmsnorm_forward {dtype} d={d} eps={eps}", flush=True)
    rng = np.random.default_rng(d)
    rows = 37
    x = P.to_device(_rows(rng, rows, d), dtype)
    w = P.to_device(P.weight_vec(rng, d), dtype)
    y, inv = vk.rmsnorm_forward(x, w, eps)
    assert y.dtype == dtype and y.shape == x.shape
    assert inv.dtype == torch.float32 and inv.shape == (rows, 1)
    x64, w64 = P.upcast(x).astype(np.float64), P.upcast(w).astype(np.float64)
    with np.errstate(all="ignore"):
        ry, rinv = ora.rmsnorm_module_forward(x64, w64, eps)
    _assert_close_nan_aware(P.upcast(inv), rinv, "inv_rms")
    # the floor acted on rows 0 and 1 (and row 2's NaN mean square), not on row 4
    floor_inv = 1.0 / np.sqrt(np.float64(np.float32(1e-12)) + np.float32(eps))
    assert np.allclose(P.upcast(inv)[:3, 0], floor_inv, rtol=1e-6)
    # only the NaN element of row 2 is NaN (the others are x * inv_rms: in fp16 at eps = 0,
    # x * 1e6 may overflow to Inf, as the float64 value rounded to fp16 does)
    assert not np.isnan(P.upcast(y)[2, 0]) and np.isnan(P.upcast(y)[2, d // 2])
    if dtype == torch.float32:
        _assert_close_nan_aware(P.upcast(y), ry, "y")
    else:
        P.assert_within_ulp(y, ry.astype(np.float32), 1, "y")


def test_zero_floor_is_the_fused_forward_bitwise():
    rng = np.random.default_rng(5)
    for dtype in DTYPES:
        x = P.to_device(P.gaussian(rng, (300, 2048)), dtype)
        w = P.to_device(P.weight_vec(rng, 2048), torch.float32)
        y, inv = vk.rmsnorm_forward(x, w, 1e-5, min_mean_sq=0.0)
        fy, h, finv = vk.fused_rmsnorm_residual_forward(x, None, w, 1e-5)
        assert h is x and torch.equal(y, fy) and torch.equal(inv, finv)


def test_strided_rows_and_leading_dims():
    rng = np.random.default_rng(6)
    wide = P.to_device(P.gaussian(rng, (3, 5, 1100)), torch.bfloat16)
    x = wide[..., 7:7 + 1024]
    w = P.to_device(P.weight_vec(rng, 1024), torch.bfloat16)
    y, inv = vk.rmsnorm_forward(x, w)
    assert y.shape == (3, 5, 1024) and inv.shape == (3, 5, 1)
    ry, rinv = ora.rmsnorm_module_forward(P.upcast(x).astype(np.float64),
                                          P.upcast(w).astype(np.float64))
    P.assert_within_ulp(y, ry.astype(np.float32), 1, "y")
    _assert_close_nan_aware(P.upcast(inv), rinv, "inv_rms")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_module_autograd_matches_module_oracle(dtype):
    rng = np.random.default_rng(7)
    d = 4096
    xs = P.gaussian(rng, (2, 33, d))
    xs[0, 0] = 1e-8   # floored row: the reference's backward still uses its (floored) inv_rms
    xs[1, 5] = 0.0
    mod = vnn.RMSNorm(d, device="cuda", dtype=dtype)
    with torch.no_grad():
        mod.weight.copy_(P.to_device(P.weight_vec(rng, d), dtype))
    x = P.to_device(xs, dtype).requires_grad_(True)
    y = mod(x)
    g = P.to_device(P.gaussian(rng, (2, 33, d)), dtype)
    y.backward(g)
    assert x.grad.dtype == dtype and mod.weight.grad.shape == (d,)

    x64 = P.upcast(x).astype(np.float64)
    w64 = P.upcast(mod.weight).astype(np.float64)
    g64 = P.upcast(g).astype(np.float64)
    ry, rinv = ora.rmsnorm_module_forward(x64, w64, mod.eps)
    if dtype == torch.float32:
        _assert_close_nan_aware(P.upcast(y), ry, "y")
    else:
        P.assert_within_ulp(y, ry.astype(np.float32), 1, "y")
    # backward on the device's own inv_rms (the saved statistic), as the reference does
    _, inv = vk.rmsnorm_forward(x.detach(), mod.weight.detach(), mod.eps)
    inv64 = P.upcast(inv).astype(np.float64)
    rdx, rdw = ora.rmsnorm_module_backward(g64, x64, w64, inv64)
    xhat = x64 * inv64
    gw = g64 * w64
    if dtype == torch.float32:
        err = np.abs(P.upcast(x.grad) - rdx) / (P.dx_scale(gw, xhat, inv64) + 1e-30)
        assert float(err.max()) <= P.FP32_REL_TOL
    else:
        P.dx_check(x.grad, rdx.astype(np.float32), gw, xhat, inv64, "dx")
    got = P.upcast(mod.weight.grad).astype(np.float64)
    if dtype == torch.float32:
        P.assert_dweight(got, rdw)
    else:
        # plus the rounding of the fp32 dweight to the bf16 parameter's gradient (2^-9
        # relative; 2^-8 allows for either side)
        tol = P.DWEIGHT_REL_TOL * np.maximum(np.abs(rdw), np.sqrt(np.mean(rdw * rdw))) + \
            2.0 ** -8 * np.abs(rdw)
        assert np.all(np.abs(got - rdw) <= tol)


def test_module_at_eps_zero_keeps_zero_rows_finite():
    """The reference module's floor keeps a zero row finite at eps = 0 (inv_rms = 1e6, y = 0,
    dx = 1e6 * g * w), where the unclamped fused forward gives inv_rms = inf and y = NaN."""
    d = 512
    mod = vnn.RMSNorm(d, eps=0.0).cuda()
    x = torch.zeros(2, d, device="cuda", requires_grad=True)
    y = mod(x)
    assert torch.equal(y.detach(), torch.zeros_like(y))
    g = torch.ones_like(y)
    y.backward(g)
    assert torch.isfinite(x.grad).all()
    assert torch.allclose(x.grad, torch.full_like(x.grad, 1e6), rtol=1e-6)
    fy, _, finv = vk.fused_rmsnorm_residual_forward(x.detach(), None, None, 0.0)
    assert torch.isinf(finv).all() and torch.isnan(fy).all()


def test_min_mean_sq_is_validated():
    x = torch.ones(2, 64, device="cuda")
    with pytest.raises(ValueError):
        vk.rmsnorm_forward(x, None, 1e-6, min_mean_sq=-1.0)
    with pytest.raises(ValueError):
        vk.rmsnorm_forward(x, None, 1e-6, min_mean_sq=float("nan"))
    with pytest.raises(TypeError):
        vk.rmsnorm_forward(x.cpu(), None)


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16", "f16"])
def test_residual_add_then_module_norm(dtype):
    """The reference model's `h = x + attn_out; ffn_norm(h)` (models/llama.py:52-54) in one pass:
    fused_rmsnorm_residual_forward(..., min_mean_sq=1e-12) against the module oracle applied to
    the fp32 sum; rows where h is zero (x = -residual) or tiny stay finite at eps = 0."""
    rng = np.random.default_rng(11)
    d = 4096
    xs = P.gaussian(rng, (40, d))
    rs = P.gaussian(rng, (40, d))
    rs[0] = -xs[0]                     # h = 0
    xs[1], rs[1] = 1e-8, 0.0           # tiny h
    xs[2, 7] = np.nan                  # NaN mean square -> the floor
    x, r = P.to_device(xs, dtype), P.to_device(rs, dtype)
    w = P.to_device(P.weight_vec(rng, d), dtype)
    for eps in (1e-6, 0.0):
        y, h, inv = vk.fused_rmsnorm_residual_forward(x, r, w, eps, min_mean_sq=1e-12)
        h32 = P.upcast(x) + P.upcast(r)
        if dtype == torch.float32:
            assert np.array_equal(P.upcast(h), h32, equal_nan=True)
        else:
            P.assert_within_ulp(h, h32, 0, "h")
        with np.errstate(all="ignore"):
            ry, rinv = ora.rmsnorm_module_forward(h32.astype(np.float64), P.upcast(w).astype(
                np.float64), eps)
        _assert_close_nan_aware(P.upcast(inv), rinv, "inv_rms")
        if dtype == torch.float32:
            _assert_close_nan_aware(P.upcast(y), ry, "y")
        else:
            P.assert_within_ulp(y, ry.astype(np.float32), 1, "y")
        assert np.all(np.isfinite(P.upcast(inv)))
        # without the floor (fused.py) the zero row at eps = 0 has inv_rms = inf
        _, _, inv0 = vk.fused_rmsnorm_residual_forward(x, r, w, eps)
        assert np.isinf(P.upcast(inv0)[0, 0]) == (eps == 0.0)


def test_fused_add_module_floors_and_backpropagates():
    d = 1024
    mod = vnn.FusedAddRMSNorm(d, eps=0.0).cuda()
    assert mod.min_mean_sq == 1e-12
    x = torch.randn(3, d, device="cuda", requires_grad=True)
    r = (-x.detach()).clone().requires_grad_(True)       # h = 0 on every row
    y, h = mod(x, r)
    assert torch.equal(y.detach(), torch.zeros_like(y))
    (y.sum() + h.sum()).backward()
    # dx = dres = inv_rms * g * w + grad_h = 1e6 + 1 per element
    assert torch.isfinite(x.grad).all() and torch.equal(x.grad, r.grad)
    assert torch.allclose(x.grad, torch.full_like(x.grad, 1e6 + 1), rtol=1e-6)
    # floor off: fused.py semantics, inf * 0 = NaN
    y0, _ = vnn.fused_add_rmsnorm(x.detach(), r.detach(), mod.weight.detach(), 0.0)
    assert torch.isnan(y0).all()


def test_min_mean_sq_host_arrays():
    xs = np.zeros((2, 64), dtype=np.float32)
    y, h, inv = vk.fused_rmsnorm_residual_forward(xs, None, None, 0.0, min_mean_sq=1e-12)
    assert isinstance(y, np.ndarray) and np.all(y == 0) and np.allclose(inv, 1e6, rtol=1e-6)
    with pytest.raises(ValueError):
        vk.fused_rmsnorm_residual_forward(xs, None, None, 0.0, min_mean_sq=-1.0)
