"""Rows that are not 16-byte multiples (hidden sizes such as 4100 bf16).  Rows of 8n + 4
two-byte elements whose streams start on 8-byte boundaries take the register-resident kernels
(whole chunks in 8-byte halves, the last 4 elements a half chunk); the others take the generic
kernels: each row's 16-byte-aligned middle moves in 16-byte accesses and its head and tail
element by element, and the backward sums its dweight columns in LDS, where a column moves
between threads from row to row.  Checked against the oracle with tests/_parity.py's tolerances: contiguous
tensors (every row through the aligned middle), tensors of different row strides (rows whose
streams disagree inside a 16-byte line take the element-wise path, so one workgroup mixes both),
rows at the LDS limit and past it, and bitwise repeatability of dx and dweight."""

import numpy as np
import pytest
import torch

from oracle import fused_rmsnorm as ora
from tests import _parity as P
from velograd_amd import kernels as vk

pytestmark = pytest.mark.gpu

BF16, F16, F32 = torch.bfloat16, torch.float16, torch.float32

CASES = [
    # rows, dim, dtype, weight ("same", "f32", None), residual-stream gradient
    (2048, 4100, BF16, "same", False),
    (1024, 4099, F16, "f32", True),
    (1024, 4102, BF16, None, False),
    (512, 1001, F32, "same", True),
    (777, 16000, BF16, "same", False),   # LDS sums at their limit (kGenericLdsCols)
    (300, 16008, BF16, "same", True),    # past it: element-wise rows, sums in the partial row
    (64, 20002, F32, "same", False),
    # rows of 8n + 4 two-byte elements on 8-byte boundaries: the register-resident kernels over
    # the whole chunks in 8-byte halves plus a half chunk (fwd_vec_kernel X8, bwd_ring_kernel
    # kRing8), down to one whole chunk (dim 12)
    (999, 2052, F16, "f32", False),
    (4097, 1028, BF16, None, True),
    (300, 4092, BF16, "same", False),
    (64, 12, BF16, "same", True),
    (1, 4100, BF16, "same", True),
    (3, 508, F16, None, False),
]


def _dev(rng, shape, dtype, width=None):
    """A device tensor of `shape`; with `width`, the leading columns of a wider tensor (another
    row stride, so its rows sit elsewhere inside their 16-byte lines)."""
    if width is None:
        return P.to_device(P.gaussian(rng, shape), dtype)
    return P.to_device(P.gaussian(rng, shape[:-1] + (width,)), dtype)[..., :shape[-1]]


def _check(rows, d, dtype, wkind, with_gh, seed, widths=None):
    widths = widths or {}
    rng = np.random.default_rng(seed)
    shape = (rows, d)
    x = _dev(rng, shape, dtype, widths.get("x"))
    res = _dev(rng, shape, dtype, widths.get("res"))
    w = None
    if wkind is not None:
        w = P.to_device(P.weight_vec(rng, d), dtype if wkind == "same" else F32)
    y, h, inv = vk.fused_rmsnorm_residual_forward(x, res, w, 1e-5)
    w32 = P.upcast(w) if w is not None else None
    ry, rh, rinv = ora.fused_rmsnorm_residual_forward(P.upcast(x), P.upcast(res), w32, 1e-5)
    if dtype == F32:
        assert np.array_equal(P.upcast(h), rh)
        assert P.rel_err(P.upcast(y), ry) <= P.FP32_REL_TOL
    else:
        P.assert_within_ulp(h, rh, 0, "h")
        P.assert_within_ulp(y, ry, 1, "y")
    assert P.rel_err(P.upcast(inv), rinv) <= P.FP32_REL_TOL

    g = _dev(rng, shape, dtype, widths.get("g"))
    gh = _dev(rng, shape, dtype) if with_gh else None
    saved = h
    if "saved" in widths:
        saved = torch.empty(rows, widths["saved"], device="cuda", dtype=dtype)[:, :d]
        saved.copy_(h)
    dx, dw = vk.fused_rmsnorm_residual_backward(g, saved, w, inv, saved_is_h=True, grad_h=gh)
    g32, inv32 = P.upcast(g), P.upcast(inv)
    xhat = P.upcast(h) * inv32
    gw = g32 * w32 if w32 is not None else g32
    if gh is not None:
        rdx, rdw = ora.backward_with_residual_grad(g32, xhat, w32, inv32, P.upcast(gh))
    else:
        rdx, rdw = ora.fused_rmsnorm_residual_backward(g32, xhat, w32, inv32)
    if dtype == F32:
        scale = P.dx_scale(gw, xhat, inv32) + (np.abs(P.upcast(gh)) if gh is not None else 0.0)
        err = np.abs(P.upcast(dx).astype(np.float64) - rdx) / (scale + 1e-30)
        assert float(np.max(err)) <= P.FP32_REL_TOL
    else:
        P.dx_check(dx, rdx, gw, xhat, inv32, "dx",
                   grad_h=P.upcast(gh) if gh is not None else None)
    if w is None:
        assert dw is None
    else:
        P.assert_dweight(P.upcast(dw), rdw.reshape(-1))
        acc = np.einsum("rd,rd->d", g32.astype(np.float64), xhat.astype(np.float64))
        P.assert_dweight(P.upcast(dw), acc, "dweight vs float64")
    # the same call again: bitwise the same dx and dweight
    dx2, dw2 = vk.fused_rmsnorm_residual_backward(g, saved, w, inv, saved_is_h=True, grad_h=gh)
    assert torch.equal(dx, dx2)
    if w is not None:
        assert torch.equal(dw, dw2)


@pytest.mark.parametrize("rows,d,dtype,wkind,with_gh", CASES,
                         ids=[f"{r}x{d}-{str(t).split('.')[-1]}" for r, d, t, _, _ in CASES])
def test_unaligned_rows_match_oracle(rows, d, dtype, wkind, with_gh):
    print(f"generic rows {rows}x{d} {dtype} w={wkind} grad_h={with_gh}", flush=True)
    _check(rows, d, dtype, wkind, with_gh, seed=rows * 7 + d)


@pytest.mark.parametrize("widths", [{"res": 4104}, {"saved": 4104, "g": 4103}, {"x": 4101}],
                         ids=["res-wider", "saved-g-wider", "x-wider"])
def test_streams_of_different_row_strides(widths):
    """Streams whose rows start at different places inside a 16-byte line: those rows go element
    by element, the others through the aligned middle, in the same workgroups."""
    print(f"generic rows 1500x4100 widths {widths}", flush=True)
    _check(1500, 4100, BF16, "same", True, seed=4100, widths=widths)


def test_rows_of_8_byte_alignment_without_residual():
    """The module form (no residual: y only, h is x) over rows of 8-byte alignment."""
    print("8-byte rows without a residual, 2000x4100 bf16", flush=True)
    rng = np.random.default_rng(41)
    x = P.to_device(P.gaussian(rng, (2000, 4100)), BF16)
    w = P.to_device(P.weight_vec(rng, 4100), BF16)
    y, h, inv = vk.fused_rmsnorm_residual_forward(x, None, w, 1e-5)
    ry, _, rinv = ora.fused_rmsnorm_residual_forward(P.upcast(x), None, P.upcast(w), 1e-5)
    P.assert_within_ulp(y, ry, 1, "y")
    assert P.rel_err(P.upcast(inv), rinv) <= P.FP32_REL_TOL
