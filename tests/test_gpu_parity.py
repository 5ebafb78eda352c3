"""GPU parity: the HIP kernels (through the C ABI, via velograd_amd.kernels) against the pinned
CPU oracle on the same seeded inputs, on every benchmark configuration (A-E) and on the edge cases the
reference's semantics define.  Tolerances are stated in tests/_parity.py."""

import json
import os

import numpy as np
import pytest
import torch

from oracle import fused_rmsnorm as ora
from tests import _parity as P
from velograd_amd import kernels as vk

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "rmsnorm_residual_golden.json")
with open(GOLDEN) as _f:
    CASES = json.load(_f)["cases"]


def _say(msg):
    print(msg, flush=True)


def _dev(a, dtype=torch.float32):
    return None if a is None else P.to_device(np.asarray(a, np.float32), dtype)


# ---------------------------------------------------------------------------------------------
# Golden vectors (exact truth) through the device path in fp32.
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_golden_vectors_fp32(case):
    _say(f"golden {case['name']}")
    x, res, w = _dev(case["x"]), _dev(case["residual"]), _dev(case["weight"])
    y, h, inv = vk.fused_rmsnorm_residual_forward(x, res, w, case["eps"])
    assert P.rel_err(P.upcast(y), case["expect_y"]) <= P.FP32_REL_TOL
    assert P.rel_err(P.upcast(h), case["expect_h"]) <= 1e-7
    assert P.rel_err(P.upcast(inv).reshape(-1), case["expect_inv_rms"]) <= P.FP32_REL_TOL
    g = _dev(case["grad_y"])
    dx, dw = vk.fused_rmsnorm_residual_backward(g, h * inv, w, inv)
    exp = np.asarray(case["expect_dx"])
    scale = np.max(np.abs(exp), axis=-1, keepdims=True) + 1e-6
    assert np.max(np.abs(P.upcast(dx) - exp) / scale) <= 1e-5
    if case["expect_dweight"] is None:
        assert dw is None
    else:
        assert P.rel_err(P.upcast(dw), case["expect_dweight"]) <= 1e-5
    # same case with h saved instead of xhat
    dx2, dw2 = vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True)
    assert torch.equal(dx, dx2)
    assert (dw is None and dw2 is None) or torch.equal(dw, dw2)


def test_reference_wrapper_call_of_test_exhaustive():
    """The reference suite's only call on this path (tests/test_exhaustive.py:116-123):
    fused_rmsnorm_residual(randn(4,16), randn(4,16), randn(16), eps=1e-5), there checked for its
    shape only; here with NumPy inputs (a float32 ndarray comes back, computed on the GPU) and
    against the oracle's values."""
    rng = np.random.default_rng(116)
    x, res, w = (P.gaussian(rng, s) for s in ((4, 16), (4, 16), (16,)))
    out = vk.fused_rmsnorm_residual(x, res, w, eps=1e-5)
    assert isinstance(out, np.ndarray) and out.dtype == np.float32 and out.shape == (4, 16)
    assert P.rel_err(out, ora.fused_rmsnorm_residual(x, res, w, eps=1e-5)) <= P.FP32_REL_TOL
    # lists are accepted as the wrapper's np.asarray accepts them (kernels/__init__.py:21-27)
    out_l = vk.fused_rmsnorm_residual(x.tolist(), res.tolist(), w.tolist(), eps=1e-5)
    assert np.array_equal(out_l, out)


def test_known_answer_of_reference_rust_test():
    x = torch.tensor([[1.0, 2.0, 3.0, 4.0]], device="cuda")
    y = vk.fused_rmsnorm_residual(x, None, torch.ones(4, device="cuda"), eps=1e-5)
    assert abs(float(y[0, 0]) - 0.365148) < 1e-3


# ---------------------------------------------------------------------------------------------
# Benchmark configurations A-E (shapes, dtypes, input distributions and eps of the headline
# benchmark and its companions).
# ---------------------------------------------------------------------------------------------
def test_config_a_fp32_forward():
    """[4,128,768] fp32, x,res ~ N(0,1), weight 1+0.1N(0,1), eps 1e-6, seed 0."""
    _say("config A")
    rng = np.random.default_rng(0)
    x = P.gaussian(rng, (4, 128, 768))
    res = P.gaussian(rng, (4, 128, 768))
    w = P.weight_vec(rng, 768)
    y, h, inv = vk.fused_rmsnorm_residual_forward(_dev(x), _dev(res), _dev(w), 1e-6)
    ry, rh, rinv = ora.fused_rmsnorm_residual_forward(x, res, w, 1e-6)
    assert y.shape == (4, 128, 768) and inv.shape == (4, 128, 1) and inv.dtype == torch.float32
    assert np.array_equal(P.upcast(h), rh)  # one fp32 add on both sides
    assert P.rel_err(P.upcast(y), ry) <= P.FP32_REL_TOL
    assert P.rel_err(P.upcast(inv), rinv) <= P.FP32_REL_TOL
    # the wrapper with array-like inputs: reference wrapper semantics, float32 ndarray out
    yw = vk.fused_rmsnorm_residual(x, res, w, eps=1e-6)
    assert isinstance(yw, np.ndarray) and yw.dtype == np.float32
    assert P.rel_err(yw, ora.fused_rmsnorm_residual(x, res, w, eps=1e-6)) <= P.FP32_REL_TOL


def _bf16_forward_check(rows, d, eps, seed, std=1.0, outliers=False, dtype=torch.bfloat16):
    rng = np.random.default_rng(seed)
    x = P.gaussian(rng, (rows, d), std)
    res = P.gaussian(rng, (rows, d), std)
    if outliers:
        x = P.with_outliers(rng, x)
        res = P.with_outliers(rng, res)
    w = P.weight_vec(rng, d)
    xd, rd, wd = P.to_device(x, dtype), P.to_device(res, dtype), P.to_device(w, dtype)
    y, h, inv = vk.fused_rmsnorm_residual_forward(xd, rd, wd, eps)
    ry, rh, rinv = ora.fused_rmsnorm_residual_forward(P.upcast(xd), P.upcast(rd), P.upcast(wd), eps)
    P.assert_within_ulp(h, rh, 0, "h")
    P.assert_within_ulp(y, ry, 1, "y")
    assert P.rel_err(P.upcast(inv), rinv) <= P.FP32_REL_TOL
    return xd, rd, wd, y, h, inv


def test_config_b_bf16_forward():
    """8192 x 4096 bf16, eps 1e-5."""
    _say("config B")
    _bf16_forward_check(8192, 4096, 1e-5, seed=0)


def _backward_check(g, h, w, inv, what):
    """Backward parity given identical stored h (bf16), inv_rms and g on both sides."""
    dx, dw = vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True)
    g32, h32, w32, r32 = P.upcast(g), P.upcast(h), P.upcast(w), P.upcast(inv)
    xhat = h32 * r32
    rdx, rdw = ora.fused_rmsnorm_residual_backward(g32, xhat, w32, r32)
    n_floor = P.dx_check(dx, rdx, g32 * w32, xhat, r32, what + " dx")
    _say(f"{what}: dx elements needing the cancellation floor: {n_floor} of {rdx.size}")
    P.assert_dweight(P.upcast(dw), rdw, what + " dweight vs fp32 oracle")
    truth = np.einsum("rd,rd->d", g32.astype(np.float64), xhat.astype(np.float64))
    P.assert_dweight(P.upcast(dw), truth, what + " dweight vs float64")
    return dx, dw, xhat


def test_config_c_bf16_forward_backward():
    """16384 x 4096 bf16 fwd + bwd, eps 1e-5; dx, dresidual, fp32 dweight."""
    _say("config C")
    xd, rd, wd, y, h, inv = _bf16_forward_check(16384, 4096, 1e-5, seed=0)
    g = P.to_device(P.gaussian(np.random.default_rng(1), (16384, 4096)), torch.bfloat16)
    dx, dw, _ = _backward_check(g, h, wd, inv, "config C")
    assert dw.dtype == torch.float32 and dw.shape == (4096,)
    # normed_input (xhat) form gets the same answer from the same xhat bits
    xhat_b = (h.float() * inv).to(torch.bfloat16)
    dx2, dw2 = vk.fused_rmsnorm_residual_backward(g, xhat_b, wd, inv)
    rdx2, rdw2 = ora.fused_rmsnorm_residual_backward(P.upcast(g), P.upcast(xhat_b), P.upcast(wd),
                                                     P.upcast(inv))
    P.assert_dweight(P.upcast(dw2), rdw2, "config C xhat-form dweight")
    P.dx_check(dx2, rdx2, P.upcast(g) * P.upcast(wd), P.upcast(xhat_b), P.upcast(inv),
               "config C xhat-form dx")
    # dresidual buffer receives the same values
    dres = torch.empty_like(g)
    dx3, _ = vk.fused_rmsnorm_residual_backward(g, h, wd, inv, saved_is_h=True,
                                                dresidual_out=dres)
    assert torch.equal(dx3, dx) and torch.equal(dres, dx)


def test_config_d_bf16_outliers_all_rows():
    """32768 x 8192 bf16, x,res ~ N(0, std 2) with 0.1% entries x50, full size on the GPU and
    checked on every row against the oracle, in chunks of 4096 rows (rows are independent), and
    dweight over all rows against a float64 sum.  Inputs as every configuration's: NumPy
    default_rng(0) in fp32 (x, res, their outliers: exactly 0.1% of the entries, distinct and
    uniformly chosen, independently per tensor; then weight and grad_y), cast to bf16 with
    torch's round to nearest even."""
    _say("config D")
    rows, d = 32768, 8192
    rng = np.random.default_rng(0)
    x = P.with_outliers(rng, P.gaussian(rng, (rows, d), 2.0), inplace=True)
    res = P.with_outliers(rng, P.gaussian(rng, (rows, d), 2.0), inplace=True)
    x, res = P.to_device(x, torch.bfloat16), P.to_device(res, torch.bfloat16)
    w = P.to_device(P.weight_vec(rng, d), torch.bfloat16)
    g = P.to_device(P.gaussian(rng, (rows, d)), torch.bfloat16)
    y, h, inv = vk.fused_rmsnorm_residual_forward(x, res, w, 1e-5)
    dx, dw = vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True)
    ws = P.upcast(w)
    acc = np.zeros(d, np.float64)
    n_floor = 0
    for r0 in range(0, rows, 4096):
        sl = slice(r0, r0 + 4096)
        ry, rh, rinv = ora.fused_rmsnorm_residual_forward(P.upcast(x[sl]), P.upcast(res[sl]), ws,
                                                          1e-5)
        P.assert_within_ulp(h[sl], rh, 0, f"D h rows {r0}+")
        P.assert_within_ulp(y[sl], ry, 1, f"D y rows {r0}+")
        assert P.rel_err(P.upcast(inv[sl]), rinv) <= P.FP32_REL_TOL
        del ry, rh, rinv
        g32, h32, r32 = P.upcast(g[sl]), P.upcast(h[sl]), P.upcast(inv[sl])
        xhat = h32 * r32
        rdx, _ = ora.fused_rmsnorm_residual_backward(g32, xhat, ws, r32)
        n_floor += P.dx_check(dx[sl], rdx, g32 * ws, xhat, r32, f"D dx rows {r0}+")
        # dweight: the oracle's sum (fused.py:65) in float64
        acc += np.einsum("rd,rd->d", g32.astype(np.float64), xhat.astype(np.float64))
        del g32, h32, r32, xhat, rdx
    P.assert_dweight(P.upcast(dw), acc, "D dweight vs float64")
    print(f"config D: every row checked; {n_floor} dx elements needed the operand-scaled floor",
          flush=True)


@pytest.mark.parametrize("d", [5120, 7168])
@pytest.mark.parametrize("t", [1, 7, 64, 257])
def test_config_e_decode_shapes(t, d):
    _say(f"config E t={t} d={d}")
    _bf16_forward_check(t, d, 1e-6, seed=t * 100003 + d)


# ---------------------------------------------------------------------------------------------
# Semantics and edge cases.
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d", [1, 13, 64, 100, 768, 4096, 4104, 20000, 40000])
def test_dims_and_dtypes_forward_backward(dtype, d):
    """Vector path (d % chunk == 0, fits in registers) and generic path (ragged d, huge d)."""
    _say(f"dims d={d} {dtype}")
    rows = 37
    rng = np.random.default_rng(d)
    x = P.to_device(P.gaussian(rng, (rows, d)), dtype)
    res = P.to_device(P.gaussian(rng, (rows, d)), dtype)
    w = P.to_device(P.weight_vec(rng, d), dtype)
    g = P.to_device(P.gaussian(rng, (rows, d)), dtype)
    y, h, inv = vk.fused_rmsnorm_residual_forward(x, res, w, 1e-5)
    ry, rh, rinv = ora.fused_rmsnorm_residual_forward(P.upcast(x), P.upcast(res), P.upcast(w),
                                                      1e-5)
    if dtype == torch.float32:
        assert np.array_equal(P.upcast(h), rh)
        assert P.rel_err(P.upcast(y), ry) <= P.FP32_REL_TOL
    else:
        P.assert_within_ulp(h, rh, 0, "h")
        P.assert_within_ulp(y, ry, 1, "y")
    assert P.rel_err(P.upcast(inv), rinv) <= P.FP32_REL_TOL
    dx, dw = vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True)
    g32, h32, r32, w32 = P.upcast(g), P.upcast(h), P.upcast(inv), P.upcast(w)
    xhat = h32 * r32
    rdx, rdw = ora.fused_rmsnorm_residual_backward(g32, xhat, w32, r32)
    if dtype == torch.float32:
        P.assert_dx_fp32(dx, rdx, g32 * w32, xhat, r32)
    else:
        P.dx_check(dx, rdx, g32 * w32, xhat, r32)
    P.assert_dweight(P.upcast(dw), rdw)


def test_fp32_weight_with_bf16_activations():
    rng = np.random.default_rng(11)
    x = P.to_device(P.gaussian(rng, (64, 4096)), torch.bfloat16)
    w32 = P.to_device(P.weight_vec(rng, 4096), torch.float32)
    y, h, inv = vk.fused_rmsnorm_residual_forward(x, None, w32, 1e-5)
    ry, _, _ = ora.fused_rmsnorm_residual_forward(P.upcast(x), None, P.upcast(w32), 1e-5)
    P.assert_within_ulp(y, ry, 1, "y")
    g = P.to_device(P.gaussian(rng, (64, 4096)), torch.bfloat16)
    dx, dw = vk.fused_rmsnorm_residual_backward(g, h, w32, inv, saved_is_h=True)
    _, rdw = ora.backward_from_h(P.upcast(g), P.upcast(h), P.upcast(w32), P.upcast(inv))
    P.assert_dweight(P.upcast(dw), rdw)


def test_residual_none_returns_x_itself_and_weight_none():
    x = torch.randn(8, 256, device="cuda", dtype=torch.bfloat16)
    y, h, inv = vk.fused_rmsnorm_residual_forward(x)
    assert h is x
    ry, _, _ = ora.fused_rmsnorm_residual_forward(P.upcast(x), None, None, 1e-6)
    P.assert_within_ulp(y, ry, 1, "y")
    dx, dw = vk.fused_rmsnorm_residual_backward(torch.ones_like(x), h, None, inv, saved_is_h=True)
    assert dw is None


def test_leading_dims_weight_1xd_and_strided_rows():
    base = torch.randn(6, 5, 320, device="cuda")
    x = base[..., :256]  # row stride 320: strided view, no copy in the kernel call
    res = torch.randn(6, 5, 256, device="cuda")
    w = torch.randn(1, 256, device="cuda")
    y, h, inv = vk.fused_rmsnorm_residual_forward(x, res, w, 1e-5)
    assert y.shape == (6, 5, 256) and inv.shape == (6, 5, 1)
    ry, _, rinv = ora.fused_rmsnorm_residual_forward(P.upcast(x), P.upcast(res), P.upcast(w), 1e-5)
    assert P.rel_err(P.upcast(y), ry) <= P.FP32_REL_TOL


def test_misaligned_pointers_take_the_generic_path():
    base = torch.randn(33 * 4096 + 1, device="cuda", dtype=torch.bfloat16)
    x = base[1:].view(33, 4096)  # 2-byte offset: not 16-byte aligned
    res = torch.randn(33, 4096, device="cuda", dtype=torch.bfloat16)
    w = torch.randn(4096, device="cuda", dtype=torch.bfloat16)
    y, h, _ = vk.fused_rmsnorm_residual_forward(x, res, w, 1e-5)
    ry, rh, _ = ora.fused_rmsnorm_residual_forward(P.upcast(x), P.upcast(res), P.upcast(w), 1e-5)
    P.assert_within_ulp(h, rh, 0, "h")
    P.assert_within_ulp(y, ry, 1, "y")


def test_broadcast_residual_row():
    x = torch.randn(10, 128, device="cuda")
    res = torch.randn(128, device="cuda")
    y, h, _ = vk.fused_rmsnorm_residual_forward(x, res)
    ry, rh, _ = ora.fused_rmsnorm_residual_forward(P.upcast(x), P.upcast(res), None, 1e-6)
    assert np.array_equal(P.upcast(h), rh) and P.rel_err(P.upcast(y), ry) <= P.FP32_REL_TOL


def test_one_dimensional_inputs():
    """A single row given as a 1-D vector, as NumPy's axis=-1 reductions allow (fused.py:41-42,
    59-65): y and h shaped like x, inv_rms of shape (1,), dx like grad_y, dweight [D]; the
    array-like wrapper returns a 1-D float32 ndarray."""
    rng = np.random.default_rng(31)
    for d, dtype in ((4096, torch.bfloat16), (1000, torch.float32), (7, torch.float32)):
        x32, r32, g32 = (P.gaussian(rng, (d,)) for _ in range(3))
        w32 = P.weight_vec(rng, d)
        x, r, w, g = (P.to_device(a, dtype) for a in (x32, r32, w32, g32))
        y, h, inv = vk.fused_rmsnorm_residual_forward(x, r, w, 1e-5)
        assert y.shape == (d,) and h.shape == (d,) and inv.shape == (1,)
        ry, rh, rinv = ora.fused_rmsnorm_residual_forward(P.upcast(x), P.upcast(r), P.upcast(w),
                                                          1e-5)
        assert rinv.shape == (1,)
        if dtype == torch.float32:
            assert np.array_equal(P.upcast(h), rh)
            assert P.rel_err(P.upcast(y), ry) <= P.FP32_REL_TOL
        else:
            P.assert_within_ulp(h, rh, 0, f"1-D h d={d}")
            P.assert_within_ulp(y, ry, 1, f"1-D y d={d}")
        assert P.rel_err(P.upcast(inv), rinv) <= P.FP32_REL_TOL
        dx, dw = vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True)
        assert dx.shape == (d,) and dw.shape == (d,) and dw.dtype == torch.float32
        g2, w2 = P.upcast(g).reshape(1, d), P.upcast(w)
        xhat = P.upcast(h).reshape(1, d) * P.upcast(inv).reshape(1, 1)
        rdx, rdw = ora.fused_rmsnorm_residual_backward(g2, xhat, w2, P.upcast(inv).reshape(1, 1))
        if dtype == torch.float32:
            P.assert_dx_fp32(dx.view(1, d), rdx, g2 * w2, xhat, P.upcast(inv).reshape(1, 1))
        else:
            P.dx_check(dx.view(1, d), rdx, g2 * w2, xhat, P.upcast(inv).reshape(1, 1),
                       f"1-D dx d={d}")
        P.assert_dweight(P.upcast(dw), rdw, f"1-D dweight d={d}")
    out = vk.fused_rmsnorm_residual(x32, r32, w32, eps=1e-5)
    assert isinstance(out, np.ndarray) and out.shape == (7,) and out.dtype == np.float32
    assert P.rel_err(out, ora.fused_rmsnorm_residual(x32, r32, w32, eps=1e-5)) <= P.FP32_REL_TOL


def test_empty_inputs():
    x = torch.empty(0, 4096, device="cuda", dtype=torch.bfloat16)
    w = torch.ones(4096, device="cuda", dtype=torch.bfloat16)
    y, h, inv = vk.fused_rmsnorm_residual_forward(x, x.clone(), w)
    assert y.shape == (0, 4096) and inv.shape == (0, 1)
    dx, dw = vk.fused_rmsnorm_residual_backward(x, x.clone(), w, inv)
    assert dx.shape == (0, 4096) and torch.equal(dw, torch.zeros(4096, device="cuda"))
    z = torch.empty(3, 0, device="cuda")
    y, h, inv = vk.fused_rmsnorm_residual_forward(z, z.clone())
    assert y.shape == (3, 0) and torch.isnan(inv).all()


def test_nan_and_inf_propagate_per_row():
    x = torch.ones(4, 1024, device="cuda")
    x[1, 10] = float("nan")
    x[2, 3] = float("inf")
    y, h, inv = vk.fused_rmsnorm_residual_forward(x, torch.zeros_like(x), None, 1e-6)
    assert torch.isfinite(y[0]).all() and torch.isfinite(y[3]).all()
    assert torch.isnan(y[1]).all() and torch.isnan(inv[1]).all()
    assert float(inv[2]) == 0.0


def test_zero_and_constant_rows_closed_form():
    x = torch.zeros(3, 2048, device="cuda")
    x[1] = 0.75
    y, _, inv = vk.fused_rmsnorm_residual_forward(x, None, None, 1e-6)
    e32 = np.float32(1e-6)
    assert float(inv[0]) == float(np.float32(1.0) / np.sqrt(e32))
    assert torch.all(y[0] == 0)
    exp = np.float32(1.0) / np.sqrt(np.float32(0.5625) + e32)
    assert float(inv[1]) == float(exp)


def test_dweight_bitwise_deterministic():
    rng = np.random.default_rng(5)
    g = P.to_device(P.gaussian(rng, (4096, 4096)), torch.bfloat16)
    h = P.to_device(P.gaussian(rng, (4096, 4096)), torch.bfloat16)
    w = P.to_device(P.weight_vec(rng, 4096), torch.bfloat16)
    inv = torch.rand(4096, 1, device="cuda") + 0.5
    outs = [vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True) for _ in range(3)]
    for dx, dw in outs[1:]:
        assert torch.equal(dx, outs[0][0]) and torch.equal(dw, outs[0][1])


def test_outputs_stay_inside_their_buffers():
    """Canaries around y/h/inv_rms written through the C ABI directly."""
    from velograd_amd import _lib
    lib = _lib.load()
    rows, d, pad = 19, 4096, 4096
    x = torch.randn(rows, d, device="cuda", dtype=torch.bfloat16)
    res = torch.randn(rows, d, device="cuda", dtype=torch.bfloat16)
    ybuf = torch.full((rows * d + 2 * pad,), 7.0, device="cuda", dtype=torch.bfloat16)
    hbuf = torch.full_like(ybuf, 7.0)
    ibuf = torch.full((rows + 2 * 64,), 7.0, device="cuda")
    y = ybuf[pad:pad + rows * d]
    h = hbuf[pad:pad + rows * d]
    inv = ibuf[64:64 + rows]
    rc = lib.velograd_rmsnorm_residual_fwd(
        x.data_ptr(), res.data_ptr(), None, y.data_ptr(), h.data_ptr(), inv.data_ptr(),
        rows, d, d, d, d, d, _lib.DTYPE_BF16, _lib.DTYPE_BF16, 1e-5,
        torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "fwd")
    torch.cuda.synchronize()
    for buf, n in ((ybuf, pad), (hbuf, pad), (ibuf, 64)):
        assert torch.all(buf[:n] == 7.0) and torch.all(buf[-n:] == 7.0)
    ry, rh, _ = ora.fused_rmsnorm_residual_forward(P.upcast(x), P.upcast(res), None, 1e-5)
    P.assert_within_ulp(h.view(rows, d), rh, 0, "h")
    P.assert_within_ulp(y.view(rows, d), ry, 1, "y")


def test_workspace_too_small_is_rejected():
    from velograd_amd import _lib
    lib = _lib.load()
    g = torch.randn(64, 512, device="cuda")
    dx = torch.empty_like(g)
    dw = torch.empty(512, device="cuda")
    w = torch.ones(512, device="cuda")
    inv = torch.ones(64, device="cuda")
    # The query covers every plan the backward may pick (dtype and alignment are unknown to it),
    # so it is at least one partial row of dim floats; a buffer smaller than that one row is
    # too small for any plan.
    need = vk.bwd_workspace_bytes(64, 512)
    assert need >= 512 * 4
    small = 512 * 4 - 16
    ws = torch.empty(small, dtype=torch.uint8, device="cuda")
    rc = lib.velograd_rmsnorm_residual_bwd(
        g.data_ptr(), g.data_ptr(), 1, w.data_ptr(), inv.data_ptr(), None, dx.data_ptr(), None,
        dw.data_ptr(), ws.data_ptr(), small, 64, 512, 512, 512, 512, 512, 512,
        _lib.DTYPE_F32, _lib.DTYPE_F32, torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.ERR_WORKSPACE_TOO_SMALL
    assert "needed" in _lib.last_error()
    with pytest.raises(ValueError):
        _lib.check(rc, "bwd")


def test_dtype_mismatch_raises():
    x = torch.randn(4, 64, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(TypeError):
        vk.fused_rmsnorm_residual_forward(x, x.float())
    with pytest.raises(TypeError):
        vk.fused_rmsnorm_residual_forward(x.double())


# ---------------------------------------------------------------------------------------------
# Residual-stream gradient (grad_h) fused into the backward.
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype,rows,d", [(torch.bfloat16, 16384, 4096),
                                          (torch.bfloat16, 300, 4104),
                                          (torch.float16, 64, 768),
                                          (torch.float32, 37, 13)])
def test_backward_with_residual_stream_gradient(dtype, rows, d):
    _say(f"grad_h {dtype} {rows}x{d}")
    rng = np.random.default_rng(rows + d)
    h = P.to_device(P.gaussian(rng, (rows, d)), dtype)
    g = P.to_device(P.gaussian(rng, (rows, d)), dtype)
    gh = P.to_device(P.gaussian(rng, (rows, d)), dtype)
    w = P.to_device(P.weight_vec(rng, d), dtype)
    _, _, inv = vk.fused_rmsnorm_residual_forward(h, None, w, 1e-5)
    dx, dw = vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True, grad_h=gh)
    g32, h32, w32, r32, gh32 = (P.upcast(t) for t in (g, h, w, inv, gh))
    xhat = h32 * r32
    rdx, rdw = ora.backward_with_residual_grad(g32, xhat, w32, r32, gh32)
    if dtype == torch.float32:
        scale = P.dx_scale(g32 * w32, xhat, r32) + np.abs(gh32)
        assert np.max(np.abs(P.upcast(dx) - rdx) / scale) <= P.FP32_REL_TOL
    else:
        P.dx_check(dx, rdx, g32 * w32, xhat, r32, "dx+grad_h", grad_h=gh32)
    P.assert_dweight(P.upcast(dw), rdw)
    # the same dweight as without grad_h, bit for bit
    _, dw0 = vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True)
    assert torch.equal(dw, dw0)


def test_residual_stream_gradient_accumulates_in_place():
    """dx may be grad_h itself: the C ABI reads each element before writing it."""
    from velograd_amd import _lib
    lib = _lib.load()
    rows, d = 1024, 4096
    rng = np.random.default_rng(3)
    h = P.to_device(P.gaussian(rng, (rows, d)), torch.bfloat16)
    g = P.to_device(P.gaussian(rng, (rows, d)), torch.bfloat16)
    gh = P.to_device(P.gaussian(rng, (rows, d)), torch.bfloat16)
    w = P.to_device(P.weight_vec(rng, d), torch.bfloat16)
    _, _, inv = vk.fused_rmsnorm_residual_forward(h, None, w, 1e-5)
    ref, _ = vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True, grad_h=gh)
    acc = gh.clone()
    inv1 = inv.reshape(rows).contiguous()
    rc = lib.velograd_rmsnorm_residual_bwd(
        g.data_ptr(), h.data_ptr(), 1, w.data_ptr(), inv1.data_ptr(), acc.data_ptr(),
        acc.data_ptr(), None, None, None, 0, rows, d, d, d, d, d, d,
        _lib.DTYPE_BF16, _lib.DTYPE_BF16, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "bwd in place")
    assert torch.equal(acc, ref)
