"""Autograd and module wrappers that put the fused kernels on a model's training path.

The reference's models call a pure-Python `nn.RMSNorm` (python/velograd/nn.py:328-389, used by
models/llama.py:44-56) followed by a separate residual add, and its fused kernel wrapper has no
gradient function (python/velograd/kernels/__init__.py:30-31).  Here:

* `FusedRMSNormResidualFunction` — forward `(y, h) = fused(x, residual, weight, eps)` saving
  `(h, inv_rms)`; backward runs the fused backward once, adding the gradient that reaches `h`
  from its other consumer (the next residual add) in the same pass, and returns
  dx = dresidual and dweight.
* `RMSNormFunction` / `RMSNorm(dim, eps=1e-6)` — the reference module's constructor and call
  (`nn.py:330-355`): mean(x^2) floored at 1e-12 (`nn.py:349`), inv_rms = 1/sqrt(mean_sq + eps),
  y = x * inv_rms * weight with weight initialised to ones; its backward is the reference's
  analytic one (`nn.py:357-383`), the fused backward with the saved input as h.
* `FusedAddRMSNorm(dim, eps=1e-6)` — `(y, h) = module(x, residual)` for pre-norm blocks: the
  reference model's `h = x + attn_out; ffn_norm(h)` (`models/llama.py:52-54`) in one pass, with
  the module's floor on the mean square.
* `FusedRoPEFunction` / `apply_rope(q, k, head_dim, theta)` — the fused RoPE kernel with its
  inverse-rotation backward.
* `RMSNormRoPEFunction` / `rms_norm_rope` / `RMSNormRoPE` — the model's `attention_norm`
  then `apply_rotary_emb` (`models/llama.py:48-49`) as one forward pass.
* `RotaryEmbFunction` / `apply_rotary_emb(x, base)` — the reference model's RoPE
  (`functional.py:287-345`, interleaved pairs over the whole last axis, positions on axis -2)
  on the same kernel, with its inverse-rotation backward.

All computation runs in the HIP kernels; there is no CPU path.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import kernels as _k

__all__ = ["FusedRMSNormResidualFunction", "fused_add_rmsnorm", "RMSNormFunction", "rms_norm",
           "RMSNorm", "FusedAddRMSNorm", "FusedRoPEFunction", "apply_rope",
           "RotaryEmbFunction", "apply_rotary_emb", "RMSNormRoPEFunction", "rms_norm_rope",
           "RMSNormRoPE"]

# nn.py:349: mean_sq = max(1e-12, sum(x ** 2 for x in row) / dim)
REFERENCE_MIN_MEAN_SQ = 1e-12


class FusedRMSNormResidualFunction(torch.autograd.Function):
    """(y, h) = fused RMSNorm + residual; differentiable in x, residual and weight."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, residual: Optional[torch.Tensor],
                weight: Optional[torch.Tensor], eps: float, min_mean_sq: float = 0.0):
        y, h, inv_rms = _k.fused_rmsnorm_residual_forward(x, residual, weight, eps,
                                                          min_mean_sq=min_mean_sq)
        if residual is None:
            h = x.view_as(x)  # a distinct output object that aliases x (fused.py:39)
        ctx.save_for_backward(h, weight, inv_rms)
        ctx.has_residual = residual is not None
        return y, h

    @staticmethod
    def backward(ctx, grad_y: Optional[torch.Tensor], grad_h: Optional[torch.Tensor]):
        h, weight, inv_rms = ctx.saved_tensors
        if grad_y is None:
            grad_y = torch.zeros_like(h)
        if grad_h is not None and grad_h.dtype != h.dtype:
            grad_h = grad_h.to(h.dtype)
        dx, dweight = _k.fused_rmsnorm_residual_backward(
            grad_y.contiguous(), h, weight, inv_rms, saved_is_h=True,
            grad_h=None if grad_h is None else grad_h.contiguous())
        need_x, need_res, need_w = ctx.needs_input_grad[:3]
        if dweight is not None and weight is not None and dweight.dtype != weight.dtype:
            dweight = dweight.to(weight.dtype)
        return (dx if need_x else None,
                dx if (need_res and ctx.has_residual) else None,
                dweight.view_as(weight) if (need_w and dweight is not None) else None,
                None, None)


def fused_add_rmsnorm(x: torch.Tensor, residual: Optional[torch.Tensor] = None,
                      weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
                      min_mean_sq: float = 0.0) -> Tuple[torch.Tensor, torch.Tensor]:
    """Differentiable `(y, h)`: h = x + residual, y = RMSNorm(h) * weight.  The statistic is
    fused.py's (min_mean_sq = 0) unless a floor on mean(h^2) is given (the reference module's
    is 1e-12, nn.py:349)."""
    return FusedRMSNormResidualFunction.apply(x, residual, weight, eps, min_mean_sq)


class RMSNormFunction(torch.autograd.Function):
    """y = RMSNorm(x) * weight as the reference module computes it (nn.py:338-355, mean square
    floored at `min_mean_sq`); differentiable in x and weight with the module's analytic
    backward (nn.py:357-383): gw = g * w, dx = inv_rms * (gw - xhat * mean(gw * xhat)),
    dweight = sum over rows of g * xhat, xhat = x * inv_rms.  Like the reference, the backward
    treats inv_rms as 1/sqrt(mean(x^2) + eps) also where the floor applied."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, weight: Optional[torch.Tensor], eps: float,
                min_mean_sq: float):
        y, inv_rms = _k.rmsnorm_forward(x, weight, eps, min_mean_sq)
        ctx.save_for_backward(x, weight, inv_rms)
        return y

    @staticmethod
    def backward(ctx, grad_y: torch.Tensor):
        x, weight, inv_rms = ctx.saved_tensors
        need_x, need_w, _, _ = ctx.needs_input_grad
        dx, dweight = _k.fused_rmsnorm_residual_backward(
            grad_y.contiguous(), x, weight, inv_rms, saved_is_h=True)
        if dweight is not None and weight is not None and dweight.dtype != weight.dtype:
            dweight = dweight.to(weight.dtype)
        return (dx if need_x else None,
                dweight.view_as(weight) if (need_w and dweight is not None) else None,
                None, None)


def rms_norm(x: torch.Tensor, weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
             min_mean_sq: float = REFERENCE_MIN_MEAN_SQ) -> torch.Tensor:
    """Differentiable RMSNorm with the reference module's semantics (nn.py:338-383)."""
    return RMSNormFunction.apply(x, weight, eps, min_mean_sq)


class RMSNorm(torch.nn.Module):
    """Drop-in for the reference's `velograd.nn.RMSNorm(dim, eps=1e-6)` (nn.py:328-389): the
    mean square is floored at 1e-12 before eps, as the reference's forward does (nn.py:349)."""

    def __init__(self, dim: int, eps: float = 1e-6, device=None, dtype=None):
        super().__init__()
        self.dim = dim
        self.eps = eps
        self.weight = torch.nn.Parameter(torch.ones(dim, device=device, dtype=dtype))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return rms_norm(x, self.weight, self.eps, REFERENCE_MIN_MEAN_SQ)

    def extra_repr(self) -> str:
        return f"{self.dim}, eps={self.eps}"


class FusedAddRMSNorm(torch.nn.Module):
    """Pre-norm block helper: `(y, h) = module(x, residual)` with h = x + residual and y the
    reference module's RMSNorm of h, in one pass: the reference's model computes
    `h = x + attn_out; ffn_norm(h)` (models/llama.py:52-54) with `ffn_norm` an `nn.RMSNorm`, so
    the mean square is floored at `min_mean_sq` (1e-12, nn.py:349) unless told otherwise."""

    def __init__(self, dim: int, eps: float = 1e-6, device=None, dtype=None,
                 min_mean_sq: float = REFERENCE_MIN_MEAN_SQ):
        super().__init__()
        self.dim = dim
        self.eps = eps
        self.min_mean_sq = min_mean_sq
        self.weight = torch.nn.Parameter(torch.ones(dim, device=device, dtype=dtype))

    def forward(self, x: torch.Tensor,
                residual: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        return fused_add_rmsnorm(x, residual, self.weight, self.eps, self.min_mean_sq)

    def extra_repr(self) -> str:
        return f"{self.dim}, eps={self.eps}, min_mean_sq={self.min_mean_sq}"


class FusedRoPEFunction(torch.autograd.Function):
    """Differentiable fused RoPE of one tensor (fused.py:72-130 semantics); the backward is the
    inverse rotation of the incoming gradient, in one kernel launch."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, head_dim: Optional[int], theta: float):
        ctx.head_dim, ctx.theta = head_dim, theta
        return _k.fused_rope_forward(x, None, head_dim=head_dim, theta=theta)[0]

    @staticmethod
    def backward(ctx, grad: torch.Tensor):
        gx = _k.fused_rope_backward(grad, None, head_dim=ctx.head_dim, theta=ctx.theta)[0]
        return gx, None, None


def apply_rope(q: torch.Tensor, k: Optional[torch.Tensor] = None,
               head_dim: Optional[int] = None, theta: float = 10000.0):
    """Differentiable `(q_rot, k_rot)`; k_rot is None without k."""
    q_rot = FusedRoPEFunction.apply(q, head_dim, theta)
    k_rot = FusedRoPEFunction.apply(k, head_dim, theta) if k is not None else None
    return q_rot, k_rot


class RMSNormRoPEFunction(torch.autograd.Function):
    """`F.apply_rotary_emb(attention_norm(x))` of the reference's model (models/llama.py:48-49)
    in one forward pass; the backward rotates grad_y back and runs the RMSNorm backward with the
    saved x in one pass as well (nn.py:357-383, functional.py:316-345 chained)."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, weight: Optional[torch.Tensor], eps: float, base: float,
                min_mean_sq: float):
        y, h, inv_rms = _k.rmsnorm_rope_forward(x, weight, eps, base, None, min_mean_sq)
        ctx.save_for_backward(h, weight, inv_rms)
        ctx.base = base
        return y

    @staticmethod
    def backward(ctx, grad_y: torch.Tensor):
        h, weight, inv_rms = ctx.saved_tensors
        dx, dweight = _k.rmsnorm_rope_backward(grad_y, h, weight, inv_rms, ctx.base)
        need_x, need_w = ctx.needs_input_grad[:2]
        if dweight is not None and weight is not None and dweight.dtype != weight.dtype:
            dweight = dweight.to(weight.dtype)
        return (dx if need_x else None,
                dweight.view_as(weight) if (need_w and dweight is not None) else None,
                None, None, None)


def rms_norm_rope(x: torch.Tensor, weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
                  base: float = 10000.0,
                  min_mean_sq: float = REFERENCE_MIN_MEAN_SQ) -> torch.Tensor:
    """Differentiable `apply_rotary_emb(RMSNorm(x))` with the reference's semantics, fused."""
    return RMSNormRoPEFunction.apply(x, weight, eps, base, min_mean_sq)


class RMSNormRoPE(torch.nn.Module):
    """The reference block's `attention_norm` followed by `F.apply_rotary_emb`
    (models/llama.py:44,48-49) as one module: weight [dim] initialised to ones (nn.py:334)."""

    def __init__(self, dim: int, eps: float = 1e-6, base: float = 10000.0, device=None,
                 dtype=None):
        super().__init__()
        self.dim = dim
        self.eps = eps
        self.base = base
        self.weight = torch.nn.Parameter(torch.ones(dim, device=device, dtype=dtype))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return rms_norm_rope(x, self.weight, self.eps, self.base, REFERENCE_MIN_MEAN_SQ)

    def extra_repr(self) -> str:
        return f"{self.dim}, eps={self.eps}, base={self.base}"


class RotaryEmbFunction(torch.autograd.Function):
    """The reference's differentiable `apply_rotary_emb` (functional.py:287-345): forward and
    backward (the inverse rotation, functional.py:316-345) are one kernel launch each."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, base: float):
        ctx.base = base
        return _k.fused_rope_interleaved(x, base)

    @staticmethod
    def backward(ctx, grad: torch.Tensor):
        return _k.fused_rope_interleaved(grad.contiguous(), ctx.base, inverse=True), None


def apply_rotary_emb(x: torch.Tensor, base: float = 10000.0) -> torch.Tensor:
    """Drop-in for `velograd.functional.apply_rotary_emb(x, base=10000.0)`
    (functional.py:287): interleaved-pair RoPE over x's last axis, positions along axis -2."""
    return RotaryEmbFunction.apply(x, base)
