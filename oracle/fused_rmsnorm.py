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
