"""Pins the CPU oracle (oracle/fused_rmsnorm.py) before anything is compared with it.

Each check is independent of the oracle's own formula: exact golden vectors (finite differences
for the backward), the reference's known answers and gradcheck rule, torch's rms_norm and
autograd, closed forms and invariants.  The mutation tests plant plausible mistakes in copies of
the oracle and show the checks above catch them.
"""

import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import fused_rmsnorm as ora
from tests._parity import FP32_REL_TOL, rel_err

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "rmsnorm_residual_golden.json")


def load_cases():
    with open(GOLDEN) as f:
        return json.load(f)["cases"]


CASES = load_cases()


def _arr(v, dtype=np.float32):
    return None if v is None else np.asarray(v, dtype=dtype)


def run_oracle(case, dtype=np.float32, fwd=ora.fused_rmsnorm_residual_forward,
               bwd=ora.fused_rmsnorm_residual_backward):
    x, res, w = _arr(case["x"], dtype), _arr(case["residual"], dtype), _arr(case["weight"], dtype)
    # The golden values add eps rounded to float32, as NumPy does for a float32 array.
    y, h, inv = fwd(x, res, w, float(np.float32(case["eps"])))
    out = {"y": y, "h": h, "inv": inv}
    if case.get("grad_y") is not None:
        g = _arr(case["grad_y"], dtype)
        dx, dw = bwd(g, h * inv, w, inv)
        out["dx"], out["dw"] = dx, dw
    return out


def golden_mismatches(case, out, tol=FP32_REL_TOL):
    """Names of the outputs that disagree with the golden values (empty list = all agree)."""
    bad = []
    if rel_err(out["y"], case["expect_y"]) > tol:
        bad.append("y")
    if rel_err(out["h"], case["expect_h"]) > 1e-7:
        bad.append("h")
    if rel_err(np.asarray(out["inv"]).reshape(-1), case["expect_inv_rms"]) > tol:
        bad.append("inv_rms")
    if "dx" in out:
        exp = np.asarray(case["expect_dx"], dtype=np.float64)
        # Row-normwise: dx is a difference, so judge it against its row's scale.
        scale = np.max(np.abs(exp), axis=-1, keepdims=True) + 1e-6
        if np.max(np.abs(np.asarray(out["dx"], np.float64) - exp) / scale) > 1e-5:
            bad.append("dx")
        if case["expect_dweight"] is None:
            if out["dw"] is not None:
                bad.append("dweight")
        elif rel_err(out["dw"], case["expect_dweight"]) > 1e-5:
            bad.append("dweight")
    return bad


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_oracle_matches_golden_fp32(case):
    assert golden_mismatches(case, run_oracle(case)) == []


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_oracle_matches_golden_fp64(case):
    out = run_oracle(case, np.float64)
    assert golden_mismatches(case, out, tol=1e-12) == []


def test_reference_rust_known_answer():
    # tests/core_engine_tests.rs:243-247: x=[1,2,3,4], gamma=1, eps=1e-5 -> |y0 - 0.365148| < 1e-3
    x = np.array([1.0, 2.0, 3.0, 4.0], dtype=np.float32)
    y, _, _ = ora.fused_rmsnorm_residual_forward(x, None, np.ones(4, np.float32), 1e-5)
    assert abs(y[0] - 0.365148) < 1e-3
    assert abs(y[0] - 0.3651481282381126) < 1e-6
    half = x / 2
    y2, h2, _ = ora.fused_rmsnorm_residual_forward(half, half, np.ones(4, np.float32), 1e-5)
    assert np.array_equal(h2, x) and np.array_equal(y2, y)


@pytest.mark.parametrize("row", [[1.2, 0.5, -1.0, 2.0], [1.1, -0.5, 0.8, 1.9]],
                         ids=["beast_121", "omnibus_125"])
def test_reference_gradcheck_rule(row):
    """python/velograd/autograd.py:55-128 rule (eps=1e-4, atol=1e-3, rtol=1e-2), L = sum(y)."""
    x = np.array([row], dtype=np.float64)
    w = np.ones(4)
    eps = 1e-6
    _, h, inv = ora.fused_rmsnorm_residual_forward(x, None, w, eps)
    analytic, _ = ora.fused_rmsnorm_residual_backward(np.ones_like(x), h * inv, w, inv)
    for j in range(4):
        xp, xm = x.copy(), x.copy()
        xp[0, j] += 1e-4
        xm[0, j] -= 1e-4
        num = (ora.fused_rmsnorm_residual_forward(xp, None, w, eps)[0].sum()
               - ora.fused_rmsnorm_residual_forward(xm, None, w, eps)[0].sum()) / 2e-4
        assert abs(analytic[0, j] - num) <= 1e-3 + 1e-2 * abs(num)


def test_forward_matches_torch_rms_norm():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((6, 257))
    res = rng.standard_normal((6, 257))
    w = 1 + 0.1 * rng.standard_normal(257)
    for eps in (1e-6, 1e-5, 0.5):
        y, h, _ = ora.fused_rmsnorm_residual_forward(x, res, w, eps)
        ref = torch.nn.functional.rms_norm(torch.from_numpy(x + res), (257,),
                                           torch.from_numpy(w), eps).numpy()
        assert np.max(np.abs(y - ref)) < 1e-12
        assert np.array_equal(h, x + res)


def test_backward_matches_torch_autograd():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 96))
    res = rng.standard_normal((5, 96))
    w = 1 + 0.1 * rng.standard_normal(96)
    g = rng.standard_normal((5, 96))
    eps = 1e-5
    tx = torch.tensor(x, requires_grad=True)
    tr = torch.tensor(res, requires_grad=True)
    tw = torch.tensor(w, requires_grad=True)
    y = torch.nn.functional.rms_norm(tx + tr, (96,), tw, eps)
    y.backward(torch.from_numpy(g))
    _, h, inv = ora.fused_rmsnorm_residual_forward(x, res, w, eps)
    dx, dw = ora.fused_rmsnorm_residual_backward(g, h * inv, w, inv)
    assert np.max(np.abs(dx - tx.grad.numpy())) < 1e-12
    assert np.max(np.abs(dx - tr.grad.numpy())) < 1e-12  # dresidual == dx
    assert np.max(np.abs(dw - tw.grad.numpy())) < 1e-12


def test_residual_stream_gradient_matches_torch_autograd():
    """L = sum(g*y) + sum(gh*h) with h = x + res: dL/dx = dL/dres = norm backward + gh."""
    rng = np.random.default_rng(4)
    x, res, g, gh = (rng.standard_normal((4, 80)) for _ in range(4))
    w = 1 + 0.1 * rng.standard_normal(80)
    eps = 1e-5
    tx = torch.tensor(x, requires_grad=True)
    tr = torch.tensor(res, requires_grad=True)
    tw = torch.tensor(w, requires_grad=True)
    th = tx + tr
    y = torch.nn.functional.rms_norm(th, (80,), tw, eps)
    ((y * torch.from_numpy(g)).sum() + (th * torch.from_numpy(gh)).sum()).backward()
    _, h, inv = ora.fused_rmsnorm_residual_forward(x, res, w, eps)
    dx, dw = ora.backward_with_residual_grad(g, h * inv, w, inv, gh)
    assert np.max(np.abs(dx - tx.grad.numpy())) < 1e-12
    assert np.max(np.abs(dx - tr.grad.numpy())) < 1e-12
    assert np.max(np.abs(dw - tw.grad.numpy())) < 1e-12
    # zero residual-stream gradient is the plain backward, bit for bit
    z = ora.backward_with_residual_grad(g, h * inv, w, inv, np.zeros_like(gh))
    p = ora.fused_rmsnorm_residual_backward(g, h * inv, w, inv)
    assert np.array_equal(z[0], p[0]) and np.array_equal(z[1], p[1])


def test_backward_from_h_equals_xhat_form():
    rng = np.random.default_rng(2)
    h = rng.standard_normal((3, 40)).astype(np.float32)
    g = rng.standard_normal((3, 40)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(40)).astype(np.float32)
    _, _, inv = ora.fused_rmsnorm_residual_forward(h, None, w, 1e-5)
    a = ora.backward_from_h(g, h, w, inv)
    b = ora.fused_rmsnorm_residual_backward(g, h * inv, w, inv)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_closed_forms():
    d = 64
    w = np.linspace(0.5, 1.5, d)
    for c in (0.0, 0.75, -3.0):
        x = np.full((1, d), c)
        y, _, inv = ora.fused_rmsnorm_residual_forward(x, None, w, 1e-6)
        assert inv[0, 0] == pytest.approx((c * c + 1e-6) ** -0.5, rel=1e-14)
        assert np.allclose(y[0], c * w * inv[0, 0], rtol=1e-14, atol=0)
    # zero row in fp32: inv_rms = float32(eps)^-1/2, y = 0 exactly
    y, _, inv = ora.fused_rmsnorm_residual_forward(np.zeros((2, 8), np.float32), None,
                                                   np.ones(8, np.float32), 1e-6)
    assert np.all(y == 0) and inv[0, 0] == np.float32(1.0) / np.sqrt(np.float32(1e-6))


def test_invariants():
    rng = np.random.default_rng(3)
    h = rng.standard_normal((4, 128))
    w = 1 + 0.1 * rng.standard_normal(128)
    g = rng.standard_normal((4, 128))
    # scale invariance at eps = 0
    y1, _, _ = ora.fused_rmsnorm_residual_forward(h, None, w, 0.0)
    y2, _, _ = ora.fused_rmsnorm_residual_forward(h * 37.5, None, w, 0.0)
    assert np.max(np.abs(y1 - y2)) < 1e-12
    # With r = (ms + eps)^-1/2 and m = mean(gw*xhat):
    #   sum_j dh_j h_j = r*(sum gw*h - m*sum xhat*h) = D*m*(1 - r^2*ms) = sum(gw*xhat)*eps/(ms+eps)
    # which is 0 at eps = 0 (the output is invariant to scaling h).
    for eps in (0.0, 1e-2, 1.0):
        _, _, inv = ora.fused_rmsnorm_residual_forward(h, None, w, eps)
        xhat = h * inv
        dx, _ = ora.fused_rmsnorm_residual_backward(g, xhat, w, inv)
        ms = np.mean(h * h, axis=-1, keepdims=True)
        lhs = np.sum(dx * h, axis=-1, keepdims=True)
        rhs = np.sum(g * w * xhat, axis=-1, keepdims=True) * eps / (ms + eps)
        assert np.max(np.abs(lhs - rhs)) < 1e-10


def test_nan_inf_propagate_per_row():
    x = np.ones((3, 16), np.float32)
    x[1, 4] = np.nan
    x[2, 7] = np.inf
    y, _, inv = ora.fused_rmsnorm_residual_forward(x, None, None, 1e-6)
    assert np.all(np.isfinite(y[0])) and np.all(np.isnan(y[1])) and np.isnan(inv[1, 0])
    assert inv[2, 0] == 0.0  # 1/sqrt(inf)


def test_wrapper_casts_to_float32_and_returns_y():
    x = [[1.0, 2.0, 3.0, 4.0]]
    out = ora.fused_rmsnorm_residual(x, None, [1, 1, 1, 1], eps=1e-5)
    assert out.dtype == np.float32 and out.shape == (1, 4)
    assert abs(out[0, 0] - 0.365148) < 1e-3


# ---------------------------------------------------------------------------------------------
# Planted mistakes: each mutated oracle must fail at least one of the pins above.
# ---------------------------------------------------------------------------------------------
def _bwd_drop_mean_term(g, xh, w, inv):
    gw = g * w if w is not None else g
    return inv * gw, (np.sum(g * xh, axis=tuple(range(xh.ndim - 1))) if w is not None else None)


def _bwd_wrong_sign(g, xh, w, inv):
    gw = g * w if w is not None else g
    m = np.mean(gw * xh, axis=-1, keepdims=True)
    return inv * (gw + xh * m), (np.sum(g * xh, axis=tuple(range(xh.ndim - 1)))
                                 if w is not None else None)


def _bwd_mean_over_rows(g, xh, w, inv):
    gw = g * w if w is not None else g
    m = np.mean(gw * xh, axis=0, keepdims=True)
    return inv * (gw - xh * m), (np.sum(g * xh, axis=tuple(range(xh.ndim - 1)))
                                 if w is not None else None)


def _bwd_dweight_uses_gw(g, xh, w, inv):
    dx, _ = ora.fused_rmsnorm_residual_backward(g, xh, w, inv)
    return dx, (np.sum(g * (w if w is not None else 1) * xh, axis=tuple(range(xh.ndim - 1)))
                if w is not None else None)


def _fwd_no_eps(x, res, w, eps):
    return ora.fused_rmsnorm_residual_forward(x, res, w, 0.0)


def _fwd_sum_not_mean(x, res, w, eps):
    h = x if res is None else x + res
    inv = 1.0 / np.sqrt(np.sum(h ** 2, axis=-1, keepdims=True) + eps)
    y = h * inv
    return (y * w if w is not None else y), h, inv


@pytest.mark.parametrize("fwd,bwd,saved", [
    (ora.fused_rmsnorm_residual_forward, _bwd_drop_mean_term, "xhat"),
    (ora.fused_rmsnorm_residual_forward, _bwd_wrong_sign, "xhat"),
    (ora.fused_rmsnorm_residual_forward, _bwd_mean_over_rows, "xhat"),
    (ora.fused_rmsnorm_residual_forward, _bwd_dweight_uses_gw, "xhat"),
    (ora.fused_rmsnorm_residual_forward, ora.fused_rmsnorm_residual_backward, "y"),
    (ora.fused_rmsnorm_residual_forward, ora.fused_rmsnorm_residual_backward, "h"),
    (_fwd_no_eps, ora.fused_rmsnorm_residual_backward, "xhat"),
    (_fwd_sum_not_mean, ora.fused_rmsnorm_residual_backward, "xhat"),
], ids=["drop_mean_term", "wrong_sign", "mean_over_rows", "dweight_uses_gw",
        "normed_input_is_y", "normed_input_is_h", "no_eps", "sum_not_mean"])
def test_planted_mistakes_are_caught(fwd, bwd, saved):
    caught = 0
    for case in CASES:
        dtype = np.float64
        x, res, w = _arr(case["x"], dtype), _arr(case["residual"], dtype), _arr(case["weight"], dtype)
        y, h, inv = fwd(x, res, w, case["eps"])
        out = {"y": y, "h": h, "inv": inv}
        g = _arr(case["grad_y"], dtype)
        sv = {"xhat": h * inv, "y": y, "h": h}[saved]
        out["dx"], out["dw"] = bwd(g, sv, w, inv)
        if golden_mismatches(case, out, tol=1e-9):
            caught += 1
    assert caught > 0, "the golden vectors did not detect the planted mistake"


def test_golden_file_is_regenerable():
    """The committed fixture equals what tests/golden/make_golden.py writes (first case)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "make_golden", os.path.join(os.path.dirname(__file__), "golden", "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    c = mg.make_case("kat_rust_direct", [[1.0, 2.0, 3.0, 4.0]], None, [1.0] * 4, [[1.0] * 4],
                     1e-5, "tests/core_engine_tests.rs:243-247")
    ref = CASES[0]
    for k in ("expect_y", "expect_inv_rms", "expect_dx", "expect_dweight"):
        assert np.allclose(c[k], ref[k], rtol=1e-15, atol=0), k
    assert math.isclose(c["expect_y"][0][0], 0.3651481282381126, rel_tol=1e-15)
