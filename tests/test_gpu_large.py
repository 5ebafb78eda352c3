"""Tensors of more than 2^31 elements (64-bit offsets in every kernel): 262147 x 8192 bf16, 4.3 GB
per tensor.  The rows next to the 2^31-element boundary and the last row are checked against
the oracle at the usual tolerances; the full-size dweight against a float64 column sum computed
by torch on the device in row blocks.  Peak device memory about 40 GB of the 288 GB."""

import numpy as np
import pytest
import torch

from oracle import fused_rmsnorm as ora
from tests import _parity as P
from velograd_amd import kernels as vk

pytestmark = pytest.mark.gpu

ROWS, D = 262147, 8192                  # 2,147,508,224 elements > 2^31
CHECK_ROWS = [0, 1, 262143, 262144, 262145, ROWS - 1]   # 2^31 / 8192 = 262144


def _say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def big():
    assert ROWS * D > 2 ** 31
    gen = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(ROWS, D, device="cuda", dtype=torch.bfloat16, generator=gen)
    res = torch.randn(ROWS, D, device="cuda", dtype=torch.bfloat16, generator=gen)
    w = (1 + 0.1 * torch.randn(D, device="cuda", generator=gen)).to(torch.bfloat16)
    yield x, res, w
    del x, res
    torch.cuda.empty_cache()


def _rows(t):
    return t[CHECK_ROWS].float().cpu().numpy()


def test_forward_backward_beyond_2_pow_31_elements(big):
    x, res, w = big
    _say(f"large fwd/bwd {ROWS}x{D} bf16")
    y, h, inv = vk.fused_rmsnorm_residual_forward(x, res, w, 1e-5)
    w32 = P.upcast(w)
    ry, rh, rinv = ora.fused_rmsnorm_residual_forward(_rows(x), _rows(res), w32, 1e-5)
    P.assert_within_ulp(y[CHECK_ROWS], ry, 1, "y")
    P.assert_within_ulp(h[CHECK_ROWS], rh, 0, "h")
    assert P.rel_err(_rows(inv), rinv) <= P.FP32_REL_TOL
    del y

    gen = torch.Generator(device="cuda").manual_seed(1)
    g = torch.randn(ROWS, D, device="cuda", dtype=torch.bfloat16, generator=gen)
    dx, dw = vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True)
    g32, h32, inv32 = _rows(g), _rows(h), _rows(inv)
    rdx, _ = ora.backward_from_h(g32, h32, w32, inv32)
    P.dx_check(dx[CHECK_ROWS], rdx, g32 * w32, h32 * inv32, inv32, "dx")
    # dweight = sum over all rows of g * h * inv_rms, float64, 16384-row blocks
    ref = torch.zeros(D, dtype=torch.float64, device="cuda")
    for r0 in range(0, ROWS, 16384):
        sl = slice(r0, min(ROWS, r0 + 16384))
        ref += (g[sl].double() * (h[sl].double() * inv[sl].double())).sum(0)
    P.assert_dweight(dw.double().cpu().numpy(), ref.cpu().numpy())
    torch.cuda.synchronize()


def test_dim_4096_beyond_2_pow_31_elements(big):
    """The same tensors as 524294 rows of 4096: the forward that stores h after the row
    reduction (rows of 512 threads) and the ring backward with two row groups per workgroup,
    checked on the rows either side of the 2^31-element boundary (row 524288) and the last row,
    and dweight over all rows against a float64 sum."""
    x, res, w8 = big
    rows, d = ROWS * D // 4096, 4096
    check = [0, 1, 524287, 524288, 524289, rows - 1]
    _say(f"large fwd/bwd {rows}x{d} bf16")
    x4, r4 = x.view(rows, d), res.view(rows, d)
    w = w8[:d].contiguous()
    y, h, inv = vk.fused_rmsnorm_residual_forward(x4, r4, w, 1e-5)
    w32 = P.upcast(w)
    xs, rs = x4[check].float().cpu().numpy(), r4[check].float().cpu().numpy()
    ry, rh, rinv = ora.fused_rmsnorm_residual_forward(xs, rs, w32, 1e-5)
    P.assert_within_ulp(y[check], ry, 1, "y")
    P.assert_within_ulp(h[check], rh, 0, "h")
    assert P.rel_err(inv[check].float().cpu().numpy(), rinv) <= P.FP32_REL_TOL
    del y

    gen = torch.Generator(device="cuda").manual_seed(3)
    g = torch.randn(rows, d, device="cuda", dtype=torch.bfloat16, generator=gen)
    dx, dw = vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True)
    g32 = g[check].float().cpu().numpy()
    h32 = h[check].float().cpu().numpy()
    inv32 = inv[check].float().cpu().numpy()
    rdx, _ = ora.backward_from_h(g32, h32, w32, inv32)
    P.dx_check(dx[check], rdx, g32 * w32, h32 * inv32, inv32, "dx")
    ref = torch.zeros(d, dtype=torch.float64, device="cuda")
    for r0 in range(0, rows, 32768):
        sl = slice(r0, min(rows, r0 + 32768))
        ref += (g[sl].double() * (h[sl].double() * inv[sl].double())).sum(0)
    P.assert_dweight(dw.double().cpu().numpy(), ref.cpu().numpy())
    torch.cuda.synchronize()


def _check_norm_rope_backward_large(x3, w, check, seed):
    """The one-pass norm + RoPE backward over x3 = [1, rows, dim] (one sequence): dx on the `check`
    rows against the oracle composition at their positions (the rotation's inverse, then the
    module backward, both float64), the full dweight against a float64 sum of (rotated-back g) *
    xhat computed by torch on the device in row blocks, with the angles pos * base^(-2i/dim) in
    float64 (functional.py:302-303, 316-345)."""
    rows, d = x3.shape[1], x3.shape[2]
    _, h, inv = vk.rmsnorm_rope_forward(x3, w, 1e-6, 10000.0)
    gen = torch.Generator(device="cuda").manual_seed(seed)
    g = torch.randn(1, rows, d, device="cuda", dtype=torch.bfloat16, generator=gen)
    dx, dw = vk.rmsnorm_rope_backward(g, h, w, inv, 10000.0)
    pos = np.array(check)
    g64 = g[0, check].double().cpu().numpy()
    h64 = h[0, check].double().cpu().numpy()
    r64 = inv[0, check].double().cpu().numpy()
    w64 = P.upcast(w).astype(np.float64)
    gn = ora.apply_rotary_emb(g64, 10000.0, inverse=True, positions=pos)
    rdx, _ = ora.rmsnorm_module_backward(gn, h64, w64, r64)
    # angles in double: 16 float32 ulps of the pair at any position, plus 2^-18 for the float32
    # rotation recurrence of the backward walks, which evaluate the rotation afresh every 16 rows
    # however long the walk
    dg = np.repeat((P.ROPE_ANGLE_ULPS * 2.0 ** -24 + 2.0 ** -18)
                   * (np.abs(g64[:, 0::2]) + np.abs(g64[:, 1::2])), 2, axis=1)
    xhat = h64 * r64
    tol = r64 * (np.abs(w64) * dg + np.abs(xhat) * np.mean(np.abs(w64 * xhat) * dg, axis=-1,
                                                           keepdims=True))
    tol += P.DX_FLOOR * P.dx_scale(gn * w64, xhat, r64) + 2.0 ** -8 * np.abs(rdx)
    err = np.abs(dx[0, check].double().cpu().numpy() - rdx)
    assert np.all(err <= tol), float((err - tol).max())
    del dx
    ref = torch.zeros(d, dtype=torch.float64, device="cuda")
    inv_freq = 10000.0 ** (-torch.arange(0, d, 2, dtype=torch.float64, device="cuda") / d)
    step = (1 << 27) // d
    for r0 in range(0, rows, step):
        r1 = min(rows, r0 + step)
        ang = torch.arange(r0, r1, dtype=torch.float64, device="cuda")[:, None] * inv_freq
        c, sn = torch.cos(ang), torch.sin(ang)
        gb = g[0, r0:r1].double()
        gn = torch.empty_like(gb)
        gn[:, 0::2] = gb[:, 0::2] * c + gb[:, 1::2] * sn
        gn[:, 1::2] = gb[:, 1::2] * c - gb[:, 0::2] * sn
        ref += (gn * (h[0, r0:r1].double() * inv[0, r0:r1].double())).sum(0)
    P.assert_dweight(dw.double().cpu().numpy(), ref.cpu().numpy())
    del g
    torch.cuda.synchronize()


def test_norm_rope_backward_beyond_2_pow_31_elements(big):
    """One sequence of 262147 positions at dim 8192: its walks cross the sequence end away from
    their first position, so bwd_vec_kernel's re-evaluating walk runs."""
    x, _, w = big
    _say(f"large norm+rope backward {ROWS}x{D} bf16")
    _check_norm_rope_backward_large(x.view(1, ROWS, D), w, CHECK_ROWS, 2)


@pytest.mark.parametrize("rows,d", [(262400, 8192), (524544, 4096)])
def test_norm_rope_ring_backward_beyond_2_pow_31_elements(rows, d):
    """The ring kernel (two chunks per thread at dim 8192, one at 4096) over one sequence whose
    length is a multiple of its 256 slots, past 2^31 elements: rows either side of the boundary
    (2^31 / dim) and the last rows."""
    assert rows * d > 2 ** 31
    _say(f"large norm+rope ring backward {rows}x{d} bf16")
    gen = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(1, rows, d, device="cuda", dtype=torch.bfloat16, generator=gen)
    w = (1 + 0.1 * torch.randn(d, device="cuda", generator=gen)).to(torch.bfloat16)
    b = 2 ** 31 // d
    _check_norm_rope_backward_large(x, w, [0, 1, b - 1, b, b + 1, rows - 1], 6)
    del x
    torch.cuda.empty_cache()


def test_quantised_forwards_beyond_2_pow_31_bytes(big):
    x, res, w = big
    w32 = P.upcast(w)
    x32, r32 = _rows(x), _rows(res)
    _say(f"large fp8 {ROWS}x{D}")
    y8, ys, _, inv = vk.fused_rmsnorm_residual_forward_fp8(x, res, w, 1e-5)
    gi = _rows(inv)
    codes, scales, _, _ = ora.fused_rmsnorm_residual_forward_fp8(x32, r32, w32, 1e-5, inv_rms=gi)
    assert np.array_equal(y8[CHECK_ROWS].view(torch.uint8).cpu().numpy(), codes)
    assert np.array_equal(_rows(ys), scales)
    del y8, ys
    _say(f"large mxfp8 {ROWS}x{D}")
    yq, sc, _, inv = vk.fused_rmsnorm_residual_forward_mx(x, res, w, 1e-5, fmt="e4m3")
    gi = _rows(inv)
    codes, scales, _, _ = ora.fused_rmsnorm_residual_forward_mx(x32, r32, w32, 1e-5, fmt="e4m3",
                                                                inv_rms=gi)
    assert np.array_equal(yq[CHECK_ROWS].view(torch.uint8).cpu().numpy(), codes)
    assert np.array_equal(sc[CHECK_ROWS].view(torch.uint8).cpu().numpy(), scales)
    torch.cuda.synchronize()


def test_rope_beyond_2_pow_31_elements():
    seq, heads, hd = 65537, 256, 128     # 2,147,516,416 elements
    _say(f"large rope [1, {seq}, {heads}, {hd}]")
    gen = torch.Generator(device="cuda").manual_seed(2)
    q = torch.randn(1, seq, heads, hd, device="cuda", dtype=torch.bfloat16, generator=gen)
    out, _ = vk.fused_rope_forward(q, theta=10000.0)
    pos = [0, 1, 65535, 65536, seq - 1]  # 2^31 / (256 * 128) = 65536
    got = out[0, pos].double().cpu().numpy()
    xs = q[0, pos].double().cpu().numpy()
    # float64 truth and the float32 tolerance of tests/_parity.py at each position's angles,
    # plus half a bf16 ulp for the output rounding
    half = hd // 2
    ang = np.asarray(pos, np.float64)[:, None] * 10000.0 ** (-2.0 * np.arange(half) / hd)
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    x1, x2 = xs[..., :half], xs[..., half:]
    want = np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], axis=-1)
    b = (P.ROPE_ANGLE_ULPS * 2.0 ** -24 * np.maximum(np.abs(ang), 1.0)[:, None, :] + 2.0 ** -21) \
        * (np.abs(x1) + np.abs(x2))
    tol = np.concatenate([b, b], axis=-1) + 2.0 ** -8 * 1.01 * np.abs(want)
    assert np.all(np.abs(got - want) <= tol)
    del q, out
    torch.cuda.synchronize()


def test_interleaved_rope_beyond_2_pow_31_elements():
    """The interleaved pairing's 16-byte tiles with element offsets past 2^31 (position 262144
    of a [262145, 8192] sequence starts at element 2^31; 262145 leaves a two-position last tile)."""
    seq, d = 262145, 8192
    _say(f"large interleaved rope [{seq}, {d}]")
    gen = torch.Generator(device="cuda").manual_seed(4)
    x = torch.randn(seq, d, device="cuda", dtype=torch.bfloat16, generator=gen)
    out = vk.fused_rope_interleaved(x, 500000.0)
    pos = [0, 1, 2, 3, 262141, 262142, 262143, 262144]
    got = out[pos].double().cpu().numpy()
    xs = x[pos].double().cpu().numpy()
    want = ora.apply_rotary_emb(xs, 500000.0, positions=pos)
    mag = np.abs(xs[:, 0::2]) + np.abs(xs[:, 1::2])
    b = (P.ROPE_ANGLE_ULPS * 2.0 ** -24 + 2.0 ** -21) * np.repeat(mag, 2, axis=1)
    tol = b + 2.0 ** -8 * 1.01 * np.abs(want)
    assert np.all(np.abs(got - want) <= tol)
    del x, out
    torch.cuda.synchronize()
