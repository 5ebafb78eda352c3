"""Autograd integration (velograd_amd.nn) on the GPU against torch autograd of the same math on
the CPU in float64, and against the oracle for reduced precision."""

import numpy as np
import pytest
import torch

from oracle import fused_rmsnorm as ora
from tests import _parity as P
from velograd_amd import nn as vnn

pytestmark = pytest.mark.gpu


def _torch_reference(x, res, w, gy, gh, eps):
    """float64 CPU autograd of y = rms_norm(x + res) * w; loss = sum(gy*y) + sum(gh*h)."""
    tx = x.detach().double().cpu().requires_grad_(True)
    tr = res.detach().double().cpu().requires_grad_(True) if res is not None else None
    tw = w.detach().double().cpu().requires_grad_(True)
    th = tx + tr if tr is not None else tx
    y = torch.nn.functional.rms_norm(th, (th.shape[-1],), tw, eps)
    loss = (y * gy.double().cpu()).sum()
    if gh is not None:
        loss = loss + (th * gh.double().cpu()).sum()
    loss.backward()
    return y.detach(), tx.grad, (tr.grad if tr is not None else None), tw.grad


@pytest.mark.parametrize("with_res,with_gh", [(True, True), (True, False), (False, True)])
def test_fused_add_rmsnorm_grads_fp32(with_res, with_gh):
    torch.manual_seed(0)
    shape, d, eps = (3, 50, 256), 256, 1e-5
    x = torch.randn(shape, device="cuda", requires_grad=True)
    res = torch.randn(shape, device="cuda", requires_grad=True) if with_res else None
    w = (1 + 0.1 * torch.randn(d, device="cuda")).requires_grad_(True)
    gy = torch.randn(shape, device="cuda")
    gh = torch.randn(shape, device="cuda") if with_gh else None
    y, h = vnn.fused_add_rmsnorm(x, res, w, eps)
    loss = (y * gy).sum() + ((h * gh).sum() if with_gh else 0.0)
    loss.backward()
    ry, rdx, rdres, rdw = _torch_reference(x, res, w, gy, gh, eps)
    scale = lambda t: float(t.abs().max()) + 1e-6  # noqa: E731
    assert float((y.detach().double().cpu() - ry).abs().max()) <= 1e-5 * scale(ry)
    assert float((x.grad.double().cpu() - rdx).abs().max()) <= 2e-5 * scale(rdx)
    if with_res:
        assert torch.equal(x.grad, res.grad)
        assert float((res.grad.double().cpu() - rdres).abs().max()) <= 2e-5 * scale(rdres)
    assert float((w.grad.double().cpu() - rdw).abs().max()) <= 1e-4 * scale(rdw)


def test_fused_add_rmsnorm_module_bf16_matches_oracle():
    torch.manual_seed(1)
    rows, d, eps = 2048, 4096, 1e-5
    mod = vnn.FusedAddRMSNorm(d, eps, device="cuda", dtype=torch.bfloat16)
    with torch.no_grad():
        mod.weight.copy_(1 + 0.1 * torch.randn(d, device="cuda"))
    x = torch.randn(rows, d, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    res = torch.randn(rows, d, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    gy = torch.randn(rows, d, device="cuda", dtype=torch.bfloat16)
    gh = torch.randn(rows, d, device="cuda", dtype=torch.bfloat16)
    y, h = mod(x, res)
    torch.autograd.backward([y, h], [gy, gh])
    assert mod.weight.grad.dtype == torch.bfloat16 and x.grad.dtype == torch.bfloat16
    x32, r32, w32 = P.upcast(x), P.upcast(res), P.upcast(mod.weight)
    ry, rh, _ = ora.fused_rmsnorm_residual_forward(x32, r32, w32, eps)
    P.assert_within_ulp(y, ry, 1, "y")
    P.assert_within_ulp(h, rh, 0, "h")
    # The backward sees the stored bf16 h and the inv_rms the forward saved (deterministic:
    # the plain kernel call on the same inputs returns the same bits); so does the oracle.
    from velograd_amd import kernels as vk
    _, _, inv = vk.fused_rmsnorm_residual_forward(x.detach(), res.detach(), mod.weight.detach(),
                                                  eps)
    h32, inv32 = P.upcast(h), P.upcast(inv)
    xhat = h32 * inv32
    g32, gh32 = P.upcast(gy), P.upcast(gh)
    rdx, rdw = ora.backward_with_residual_grad(g32, xhat, w32, inv32, gh32)
    P.dx_check(x.grad, rdx, g32 * w32, xhat, inv32, "dx", grad_h=gh32)
    assert torch.equal(x.grad, res.grad)
    # dweight tolerance (1e-3 of max(|b|, rms b)) plus the rounding of the fp32 dweight to the
    # bf16 parameter's gradient (half an ulp, 2^-9 relative; 2^-8 allows for either side).
    got = P.upcast(mod.weight.grad).astype(np.float64)
    ref = rdw.astype(np.float64)
    tol = P.DWEIGHT_REL_TOL * np.maximum(np.abs(ref), np.sqrt(np.mean(ref * ref))) + \
        2.0 ** -8 * np.abs(ref)
    assert np.all(np.abs(got - ref) <= tol)


def test_rmsnorm_module_forward_backward():
    torch.manual_seed(2)
    d = 768
    mod = vnn.RMSNorm(d).cuda()
    assert torch.equal(mod.weight.detach().cpu(), torch.ones(d))
    x = torch.randn(4, 128, d, device="cuda", requires_grad=True)
    y = mod(x)
    gy = torch.randn_like(y)
    y.backward(gy)
    ry, rdx, _, rdw = _torch_reference(x, None, mod.weight, gy, None, 1e-6)
    assert float((y.detach().double().cpu() - ry).abs().max()) <= 1e-5 * float(ry.abs().max())
    assert float((x.grad.double().cpu() - rdx).abs().max()) <= 2e-5 * float(rdx.abs().max())
    assert float((mod.weight.grad.double().cpu() - rdw).abs().max()) <= 1e-4 * float(
        rdw.abs().max())
    # the reference module's known answer (Rust test constants, eps 1e-5 there)
    m2 = vnn.RMSNorm(4, eps=1e-5).cuda()
    out = m2(torch.tensor([[1.0, 2.0, 3.0, 4.0]], device="cuda")).detach()
    assert abs(float(out[0, 0]) - 0.365148) < 1e-3


def test_two_stacked_prenorm_blocks_chain_gradients():
    """h of block 1 is the residual of block 2: its gradient arrives through grad_h."""
    torch.manual_seed(3)
    d = 512
    n1, n2 = vnn.FusedAddRMSNorm(d).cuda(), vnn.FusedAddRMSNorm(d).cuda()
    lin = torch.nn.Linear(d, d).cuda()
    x0 = torch.randn(64, d, device="cuda", requires_grad=True)
    r0 = torch.randn(64, d, device="cuda", requires_grad=True)
    y1, h1 = n1(x0, r0)
    y2, h2 = n2(lin(y1), h1)
    (y2.square().sum() + h2.sum()).backward()
    # same graph with torch ops in float64 on the CPU
    X0, R0 = x0.detach().double().cpu().requires_grad_(True), r0.detach().double().cpu().requires_grad_(True)
    W1 = n1.weight.detach().double().cpu().requires_grad_(True)
    W2 = n2.weight.detach().double().cpu().requires_grad_(True)
    LW, LB = lin.weight.detach().double().cpu(), lin.bias.detach().double().cpu()
    H1 = X0 + R0
    Y1 = torch.nn.functional.rms_norm(H1, (d,), W1, 1e-6)
    H2 = Y1 @ LW.T + LB + H1
    Y2 = torch.nn.functional.rms_norm(H2, (d,), W2, 1e-6)
    (Y2.square().sum() + H2.sum()).backward()
    for got, ref in ((x0.grad, X0.grad), (r0.grad, R0.grad), (n1.weight.grad, W1.grad),
                     (n2.weight.grad, W2.grad)):
        err = float((got.double().cpu() - ref).abs().max())
        assert err <= 1e-4 * float(ref.abs().max()), err


def test_apply_rope_gradients_match_torch_autograd():
    """apply_rope's backward (the inverse rotation) against float64 CPU autograd of the same
    rotate-half formula (fused.py:113-121) on the exact angles."""
    torch.manual_seed(4)
    q = torch.randn(2, 64, 4, 32, device="cuda", requires_grad=True)
    k = torch.randn(2, 64, 2, 32, device="cuda", requires_grad=True)
    gq, gk = torch.randn_like(q), torch.randn_like(k)
    q_rot, k_rot = vnn.apply_rope(q, k)
    ((q_rot * gq).sum() + (k_rot * gk).sum()).backward()

    def ref(x):
        xd = x.detach().double().cpu().requires_grad_(True)
        ang = torch.from_numpy(P.rope_angles(x.shape[1], 32, 10000.0))[None, :, None, :]
        x1, x2 = xd[..., :16], xd[..., 16:]
        return xd, torch.cat([x1 * ang.cos() - x2 * ang.sin(), x1 * ang.sin() + x2 * ang.cos()], -1)

    (qd, qr), (kd, kr) = ref(q), ref(k)
    ((qr * gq.double().cpu()).sum() + (kr * gk.double().cpu()).sum()).backward()
    for got, want in ((q.grad, qd.grad), (k.grad, kd.grad)):
        assert float((got.double().cpu() - want).abs().max()) <= 1e-5 * float(want.abs().max())
