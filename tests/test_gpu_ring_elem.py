"""The element-strided kernels (fwd_elem_kernel, bwd_ring_elem_kernel): rows the chunked kernels
cannot take (odd lengths, streams that start anywhere inside a 16-byte line) up to 4096
elements, each lane holding columns lt, lt + tpr, ... of its row group.  Checked against the
oracle with tests/_parity.py's tolerances over dtypes, weights (same dtype, fp32, none), the
residual-stream gradient, a second dresidual buffer, row strides from wider tensors, row counts
from one row to more rows than row slots (up to 16384 rows of 4095), rows of 1 to 4095 elements
(4 and 8 elements a lane, one to eight row groups a workgroup), and bitwise repeatable dx and
dweight."""

import numpy as np
import pytest
import torch

from oracle import fused_rmsnorm as ora
from tests import _parity as P
from velograd_amd import kernels as vk

pytestmark = pytest.mark.gpu

BF16, F16, F32 = torch.bfloat16, torch.float16, torch.float32

CASES = [
    # rows, dim, dtype, weight ("same", "f32", None), grad_h, dres, row stride or None
    (5000, 99, BF16, "same", False, False, None),     # 4 a lane, eight 64-thread row groups
    (3000, 255, F16, "f32", True, True, None),       # 64 lanes, one partly idle
    (1, 1, BF16, "same", False, False, None),         # one element, one row
    (2, 3, F32, None, True, False, None),
    (1700, 1001, F32, "same", False, True, None),     # 8 a lane: 126 of 128 lanes, four groups
    (2049, 2047, BF16, "same", True, False, None),    # 8 a lane, two 256-thread row groups
    (1000, 2049, F16, "same", False, False, None),    # 257 lanes: one 320-thread row group
    (777, 4095, BF16, "f32", True, True, None),       # 8 a lane, 512 threads, one idle lane
    (600, 1001, BF16, "same", False, False, 1013),    # odd row strides
    (600, 4096, F16, "same", True, False, 4099),      # aligned length, rows of odd stride
    (16384, 4095, BF16, "same", False, False, None),  # bench.py --config O: 64 rows a slot
    (16384, 4095, BF16, "same", True, False, None),   # the same with grad_h
]


def _dev(rng, rows, d, dtype, stride):
    if stride is None:
        return P.to_device(P.gaussian(rng, (rows, d)), dtype)
    return P.to_device(P.gaussian(rng, (rows, stride)), dtype)[:, :d]


@pytest.mark.parametrize("rows,d,dtype,wkind,gh,dres,stride", CASES,
                         ids=[f"{r}x{d}-{str(t).split('.')[-1]}" for r, d, t, *_ in CASES])
def test_element_ring_matches_oracle(rows, d, dtype, wkind, gh, dres, stride):
    print(f"element ring {rows}x{d} {dtype} w={wkind} grad_h={gh} dres={dres} stride={stride}",
          flush=True)
    rng = np.random.default_rng(rows * 3 + d)
    h = _dev(rng, rows, d, dtype, stride)
    g = _dev(rng, rows, d, dtype, stride)
    w = None
    if wkind is not None:
        w = P.to_device(P.weight_vec(rng, d), dtype if wkind == "same" else F32)
    ghv = _dev(rng, rows, d, dtype, stride) if gh else None
    _, _, inv = vk.fused_rmsnorm_residual_forward(h.contiguous(), None, w, 1e-5)
    dres_t = torch.empty(rows, d, device="cuda", dtype=dtype) if dres else None
    dx, dw = vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True, grad_h=ghv,
                                                dresidual_out=dres_t)
    torch.cuda.synchronize()
    g32, h32, r32 = P.upcast(g), P.upcast(h), P.upcast(inv)
    w32 = P.upcast(w) if w is not None else None
    xhat = h32 * r32
    gw = g32 * w32 if w32 is not None else g32
    if ghv is None:
        rdx, rdw = ora.fused_rmsnorm_residual_backward(g32, xhat, w32, r32)
    else:
        rdx, rdw = ora.backward_with_residual_grad(g32, xhat, w32, r32, P.upcast(ghv))
    if dtype == F32:
        scale = P.dx_scale(gw, xhat, r32) + (np.abs(P.upcast(ghv)) if ghv is not None else 0.0)
        err = np.abs(P.upcast(dx).astype(np.float64) - rdx) / (scale + 1e-30)
        assert float(np.max(err)) <= P.FP32_REL_TOL
    else:
        P.dx_check(dx, rdx, gw, xhat, r32, f"{rows}x{d}",
                   grad_h=P.upcast(ghv) if ghv is not None else None)
    if dres:
        assert torch.equal(dres_t, dx)
    if w is None:
        assert dw is None
    else:
        P.assert_dweight(P.upcast(dw), rdw.reshape(-1), f"{rows}x{d}")
        acc = np.einsum("rd,rd->d", g32.astype(np.float64), xhat.astype(np.float64))
        P.assert_dweight(P.upcast(dw), acc, "dweight vs float64")
    dx2, dw2 = vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True, grad_h=ghv)
    assert torch.equal(dx, dx2)
    if w is not None:
        assert torch.equal(dw, dw2)


@pytest.mark.parametrize("rows,d,dtype,wkind,gh,dres,stride", CASES,
                         ids=[f"{r}x{d}-{str(t).split('.')[-1]}" for r, d, t, *_ in CASES])
def test_element_forward_matches_oracle(rows, d, dtype, wkind, gh, dres, stride):
    """The forward over the same rows (element-strided up to 1024 elements, the generic kernel
    beyond): with a residual (y and h written) when the case has a residual-stream gradient,
    else without one (the module form's plain norm)."""
    print(f"element forward {rows}x{d} {dtype} w={wkind} residual={gh} stride={stride}",
          flush=True)
    rng = np.random.default_rng(rows * 5 + d)
    x = _dev(rng, rows, d, dtype, stride)
    res = _dev(rng, rows, d, dtype, stride) if gh else None
    w = None
    if wkind is not None:
        w = P.to_device(P.weight_vec(rng, d), dtype if wkind == "same" else F32)
    y, h, inv = vk.fused_rmsnorm_residual_forward(x, res, w, 1e-5)
    torch.cuda.synchronize()
    ry, rh, rinv = ora.fused_rmsnorm_residual_forward(
        P.upcast(x), P.upcast(res) if res is not None else None,
        P.upcast(w) if w is not None else None, 1e-5)
    if dtype == F32:
        assert np.array_equal(P.upcast(h), rh)
        assert P.rel_err(P.upcast(y), ry) <= P.FP32_REL_TOL
    else:
        P.assert_within_ulp(h, rh, 0, "h")
        P.assert_within_ulp(y, ry, 1, "y")
    assert P.rel_err(P.upcast(inv), rinv) <= P.FP32_REL_TOL
