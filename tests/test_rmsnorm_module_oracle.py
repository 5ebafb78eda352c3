"""Pins the oracle of the reference's module `velograd.nn.RMSNorm` (python/velograd/nn.py:338-383):
residual-free, mean square floored at 1e-12 before eps, Python floats.

The checks do not retype the oracle's formula: the reference test's own ground-truth loop, the
Rust known answer, torch's rms_norm and autograd where the floor is inactive, closed forms where
it is active, Python's max on NaN and Inf, and the reference's gradcheck rule.  Planted mistakes
(floor ignored, floor added instead of taken as a maximum, a NaN-propagating maximum) are shown
to fail them."""

import math

import numpy as np
import pytest
import torch

from oracle import fused_rmsnorm as ora

FLOOR = ora.MODULE_MIN_MEAN_SQ


def _forward_failures(fwd):
    """Names of the checks `fwd(x, weight, eps)` -> (y, inv_rms) fails (empty = all pass)."""
    with np.errstate(all="ignore"):  # inf * 0 and 1 / 0 are part of the cases
        return _run_forward_checks(fwd)


def _run_forward_checks(fwd):
    bad = []
    # the reference test's ground truth, tests/test_velograd_v41_enterprise_verification.py:221-229
    rng = np.random.default_rng(0)
    m, n = 4, 16
    c = rng.standard_normal((m, n)) * 3
    y, _ = fwd(c, np.ones(n), 1e-6)
    for i in range(m):
        row = [float(v) for v in c[i]]
        mean_sq = sum(v * v for v in row) / float(n)
        inv = 1.0 / math.sqrt(mean_sq + 1e-6)
        if max(abs(row[j] * inv - y[i, j]) for j in range(n)) > 1e-12:
            bad.append("reference ground truth")
            break
    # tests/core_engine_tests.rs:243-247: x=[1,2,3,4], gamma=1, eps=1e-5 -> y0 = 0.365148
    y, _ = fwd(np.array([[1.0, 2.0, 3.0, 4.0]]), np.ones(4), 1e-5)
    if abs(y[0, 0] - 0.3651481282381126) > 1e-9:
        bad.append("rust known answer")
    # zero row, eps = 0: the floor alone sets inv_rms = 1/sqrt(1e-12) = 1e6, y = 0
    y, inv = fwd(np.zeros((1, 8)), np.ones(8), 0.0)
    if not (abs(inv[0, 0] / 1e6 - 1) < 1e-14 and np.all(y == 0)):
        bad.append("zero row eps=0")
    # zero row at the module's default eps: 1/sqrt(1e-12 + 1e-6), not 1/sqrt(1e-6) = 1000
    _, inv = fwd(np.zeros((1, 8)), np.ones(8), 1e-6)
    if abs(inv[0, 0] / (1.0 / math.sqrt(1e-12 + 1e-6)) - 1) > 1e-15:
        bad.append("zero row eps=1e-6")
    # constant rows either side of the floor, eps = 0: below it inv_rms = 1e6, above it 1/c
    for cst, want_inv in ((1e-8, 1e6), (0.999e-6, 1e6), (1.001e-6, 1 / 1.001e-6), (2e-6, 5e5)):
        y, inv = fwd(np.full((1, 8), cst), np.ones(8), 0.0)
        if abs(inv[0, 0] / want_inv - 1) > 1e-12 or abs(y[0, 0] / (cst * want_inv) - 1) > 1e-12:
            bad.append(f"constant row {cst}")
    # a NaN element: Python's max(1e-12, nan) is 1e-12, so the other elements stay finite
    y, inv = fwd(np.array([[1.0, np.nan, 3.0, 4.0]]), np.ones(4), 1e-6)
    if not (np.isfinite(inv[0, 0]) and abs(inv[0, 0] * math.sqrt(1e-12 + 1e-6) - 1) < 1e-15
            and np.isnan(y[0, 1]) and np.all(np.isfinite(y[0, [0, 2, 3]]))):
        bad.append("nan row")
    # an infinite element: mean_sq = inf, inv_rms = 0, inf * 0 = nan, the rest 0
    y, inv = fwd(np.array([[1.0, np.inf, 2.0, 3.0]]), np.ones(4), 1e-6)
    if not (inv[0, 0] == 0 and np.isnan(y[0, 1]) and np.all(y[0, [0, 2, 3]] == 0)):
        bad.append("inf row")
    return bad


def test_python_max_semantics_the_oracle_mirrors():
    # nn.py:349 uses the builtin max with the floor first
    assert max(1e-12, float("nan")) == 1e-12
    assert max(1e-12, float("inf")) == float("inf")
    assert max(1e-12, 0.0) == 1e-12 and max(1e-12, 2e-12) == 2e-12


def test_module_forward_passes_every_check():
    assert _forward_failures(lambda x, w, eps: ora.rmsnorm_module_forward(x, w, eps)) == []


def test_module_forward_matches_torch_where_the_floor_is_inactive():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((12, 300)) * np.exp2(rng.integers(-16, 16, (12, 1)))
    w = 1 + 0.1 * rng.standard_normal(300)
    for eps in (1e-6, 1e-5, 0.0):
        y, inv = ora.rmsnorm_module_forward(x, w, eps)
        ref = torch.nn.functional.rms_norm(torch.from_numpy(x), (300,), torch.from_numpy(w),
                                           eps).numpy()
        assert np.max(np.abs(y - ref) / (np.abs(ref) + 1e-300)) < 1e-12
        assert np.all(np.mean(x ** 2, -1) > FLOOR)


def test_module_forward_zero_min_is_the_fused_forward():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((5, 64))
    x[0] = 0.0
    w = 1 + 0.1 * rng.standard_normal(64)
    y, inv = ora.rmsnorm_module_forward(x, w, 1e-6, min_mean_sq=0.0)
    fy, _, finv = ora.fused_rmsnorm_residual_forward(x, None, w, 1e-6)
    assert np.max(np.abs(y - fy)) < 1e-14 and np.max(np.abs(inv / finv - 1)) < 1e-15


def test_module_backward_gradcheck_rule_on_the_reference_input():
    """tests/test_velograd_beast.py:117-122 (nn.RMSNorm(dim=4), x = [[1.2, 0.5, -1.0, 2.0]])
    under python/velograd/autograd.py:55-128's rule (eps=1e-4, atol=1e-3, rtol=1e-2), L = sum(y);
    and dweight by finite differences in the weight."""
    x = np.array([[1.2, 0.5, -1.0, 2.0]])
    for w in (np.ones(4), np.array([0.9, 1.1, 1.3, -0.7])):
        y, inv = ora.rmsnorm_module_forward(x, w)
        dx, dw = ora.rmsnorm_module_backward(np.ones_like(x), x, w, inv)
        for j in range(4):
            e = np.zeros_like(x)
            e[0, j] = 1e-4
            num = (ora.rmsnorm_module_forward(x + e, w)[0].sum()
                   - ora.rmsnorm_module_forward(x - e, w)[0].sum()) / 2e-4
            assert abs(dx[0, j] - num) <= 1e-3 + 1e-2 * abs(num)
            ew = np.zeros(4)
            ew[j] = 1e-4
            numw = (ora.rmsnorm_module_forward(x, w + ew)[0].sum()
                    - ora.rmsnorm_module_forward(x, w - ew)[0].sum()) / 2e-4
            assert abs(dw[j] - numw) <= 1e-3 + 1e-2 * abs(numw)


def test_module_backward_matches_torch_autograd():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 7, 96))
    w = 1 + 0.1 * rng.standard_normal(96)
    g = rng.standard_normal((3, 7, 96))
    eps = 1e-6
    _, inv = ora.rmsnorm_module_forward(x, w, eps)
    dx, dw = ora.rmsnorm_module_backward(g, x, w, inv)
    xt = torch.from_numpy(x).requires_grad_()
    wt = torch.from_numpy(w).requires_grad_()
    torch.nn.functional.rms_norm(xt, (96,), wt, eps).backward(torch.from_numpy(g))
    assert np.max(np.abs(dx - xt.grad.numpy())) < 1e-12
    assert np.max(np.abs(dw - wt.grad.numpy()) / (np.abs(wt.grad.numpy()) + 1)) < 1e-12


def test_module_backward_is_the_fused_backward_with_xhat():
    """The device path runs the module's backward as the fused backward with x as h."""
    rng = np.random.default_rng(4)
    x = rng.standard_normal((9, 40))
    x[0] = 1e-9  # a floored row: both forms use the saved inv_rms the same way
    w = 1 + 0.1 * rng.standard_normal(40)
    g = rng.standard_normal((9, 40))
    _, inv = ora.rmsnorm_module_forward(x, w)
    dx, dw = ora.rmsnorm_module_backward(g, x, w, inv)
    fdx, fdw = ora.backward_from_h(g, x, w, inv)
    scale = np.max(np.abs(dx), axis=-1, keepdims=True)
    assert np.max(np.abs(dx - fdx) / scale) < 1e-13
    assert np.max(np.abs(dw - fdw) / (np.abs(fdw) + 1)) < 1e-13


# ---------------------------------------------------------------------------------------------
# Planted mistakes in copies of the forward
# ---------------------------------------------------------------------------------------------
def _no_floor(x, w, eps):
    return ora.rmsnorm_module_forward(x, w, eps, min_mean_sq=0.0)


def _floor_added(x, w, eps):
    x = np.asarray(x, np.float64)
    ms = np.mean(x ** 2, -1, keepdims=True) + FLOOR
    inv = 1.0 / np.sqrt(ms + eps)
    return x * inv * w, inv


def _nan_propagating_max(x, w, eps):
    x = np.asarray(x, np.float64)
    ms = np.maximum(np.mean(x ** 2, -1, keepdims=True), FLOOR)
    inv = 1.0 / np.sqrt(ms + eps)
    return x * inv * w, inv


@pytest.mark.parametrize("mistake,caught_by", [
    (_no_floor, "zero row eps=0"),
    (_floor_added, "constant row 2e-06"),
    (_nan_propagating_max, "nan row"),
])
def test_planted_mistakes_are_caught(mistake, caught_by):
    assert caught_by in _forward_failures(mistake)
