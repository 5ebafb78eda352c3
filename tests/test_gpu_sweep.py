"""A seeded random sweep over the forward + backward's argument space on the GPU against the
oracle, with the tolerances of tests/_parity.py: dtype and weight dtype (or no weight), residual
or none, leading dimensions, row strides from slicing wider tensors, the saved tensor (h or
xhat), a residual-stream gradient, and a second dresidual buffer; row lengths from 1 to 9000
(the register paths, whole rows and rows that leave lanes idle, rows of 8-byte alignment, and the
generic path)."""

import numpy as np
import pytest
import torch

from oracle import fused_rmsnorm as ora
from tests import _parity as P
from velograd_amd import kernels as vk

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
DIMS = [1, 2, 7, 8, 16, 31, 64, 96, 200, 508, 512, 640, 1000, 1024, 1028, 2048, 2052, 2056, 3000,
        3576, 4000, 4096, 4100, 5120, 9000]


def _case(i):
    rng = np.random.default_rng(1000 + i)
    dtype = DTYPES[rng.integers(3)]
    wkind = ["same", "f32", "none"][rng.integers(3)]
    d = int(DIMS[rng.integers(len(DIMS))])
    lead = [(int(rng.integers(1, 40)),), (int(rng.integers(1, 6)), int(rng.integers(1, 12)))][
        rng.integers(2)]
    return dict(dtype=dtype, wkind=wkind, d=d, lead=lead, res=bool(rng.integers(4) > 0),
                strided=bool(rng.integers(3) == 0), saved_h=bool(rng.integers(2)),
                gh=bool(rng.integers(2)), dres=bool(rng.integers(4) == 0), seed=1000 + i)


CASES = [_case(i) for i in range(64)]


def _tensor(rng, shape, dtype, strided):
    """A device tensor of `shape`; strided ones are a slice of a wider last dimension."""
    if not strided:
        return P.to_device(P.gaussian(rng, shape), dtype)
    wide = P.to_device(P.gaussian(rng, shape[:-1] + (shape[-1] + 24,)), dtype)
    return wide[..., 3:3 + shape[-1]]


@pytest.mark.parametrize("c", CASES, ids=[f"{i}" for i in range(len(CASES))])
def test_random_case_matches_oracle(c):
    dtype, d = c["dtype"], c["d"]
    shape = c["lead"] + (d,)
    print(f"sweep {c}", flush=True)
    rng = np.random.default_rng(c["seed"])
    x = _tensor(rng, shape, dtype, c["strided"])
    res = _tensor(rng, shape, dtype, c["strided"]) if c["res"] else None
    w = None
    if c["wkind"] != "none":
        w = P.to_device(P.weight_vec(rng, d), dtype if c["wkind"] == "same" else torch.float32)
    eps = 1e-5

    y, h, inv = vk.fused_rmsnorm_residual_forward(x, res, w, eps)
    x32 = P.upcast(x)
    r32 = P.upcast(res) if res is not None else None
    w32 = P.upcast(w) if w is not None else None
    ry, rh, rinv = ora.fused_rmsnorm_residual_forward(x32, r32, w32, eps)
    if dtype == torch.float32:
        assert np.array_equal(P.upcast(h), rh)
        assert P.rel_err(P.upcast(y), ry) <= P.FP32_REL_TOL
    else:
        P.assert_within_ulp(h, rh, 0, "h")
        P.assert_within_ulp(y, ry, 1, "y")
    assert P.rel_err(P.upcast(inv), rinv) <= P.FP32_REL_TOL
    if res is None:
        assert h is x

    g = _tensor(rng, shape, dtype, c["strided"])
    gh = _tensor(rng, shape, dtype, False) if c["gh"] else None
    inv32 = P.upcast(inv)
    h32 = P.upcast(h)
    if c["saved_h"]:
        saved, xhat = h, h32 * inv32
    else:
        # the reference's normed_input: xhat in the working dtype
        saved = (h.float() * inv).to(dtype)
        xhat = P.upcast(saved)
    dres = torch.empty(shape, device="cuda", dtype=dtype) if c["dres"] else None
    dx, dw = vk.fused_rmsnorm_residual_backward(g, saved, w, inv, saved_is_h=c["saved_h"],
                                                dresidual_out=dres, grad_h=gh)
    g32 = P.upcast(g)
    gw = g32 * w32 if w32 is not None else g32
    if gh is not None:
        rdx, rdw = ora.backward_with_residual_grad(g32, xhat, w32, inv32, P.upcast(gh))
    else:
        rdx, rdw = ora.fused_rmsnorm_residual_backward(g32, xhat, w32, inv32)
    if dtype == torch.float32:
        scale = P.dx_scale(gw, xhat, inv32) + (np.abs(P.upcast(gh)) if gh is not None else 0.0)
        err = np.abs(P.upcast(dx).astype(np.float64) - rdx) / (scale + 1e-30)
        assert float(np.max(err)) <= P.FP32_REL_TOL
    else:
        P.dx_check(dx, rdx, gw, xhat, inv32, "dx",
                   grad_h=P.upcast(gh) if gh is not None else None)
    if dres is not None:
        assert torch.equal(dres, dx)
    if w is None:
        assert dw is None
    else:
        P.assert_dweight(P.upcast(dw), rdw.reshape(-1))
