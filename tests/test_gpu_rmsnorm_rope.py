"""The reference model's attention-branch input in one pass, `F.apply_rotary_emb(attention_norm(x))`
(models/llama.py:48-49), through velograd_rmsnorm_rope_fwd, against the composition of the two
pinned oracles: rmsnorm_module_forward (nn.py:338-355, float64, 1e-12 floor) then apply_rotary_emb
(functional.py:287-315, float64).  Tolerance per rotated element: 16 float32 ulps of the normalised
pair (the fused kernels form the angles in double, so the bound does not grow with the
position), a float32 term for the norm, and for bf16/fp16 outputs 2^-17 of the pair for the
forward walk's float32 rotation recurrence (at most 31 steps of about 3 float32 ulps from an
exact value; fp32 outputs keep it in double) plus half an output ulp (half the subnormal spacing
for fp16 outputs below 2^-14); inv_rms |a-b|/(|b|+1e-6) <= 1e-5; h bit-exact.  The one-pass backward
(velograd_rmsnorm_rope_bwd) is checked against the composition of the inverse rotation and the
module backward, with the bound stated above its test.  The autograd module is checked against
torch float64 autograd of rms_norm and the complex-number rotation."""

import numpy as np
import pytest
import torch

from oracle import fused_rmsnorm as ora
from tests import _parity as P
from velograd_amd import kernels as vk
from velograd_amd import nn as vnn

pytestmark = pytest.mark.gpu

ROUNDING = {torch.float32: 0.0, torch.bfloat16: 2.0 ** -8 * 1.01, torch.float16: 2.0 ** -11 * 1.01}
# The forward walk's float32 rotation recurrence (16-bit outputs): at most 31 steps of about
# 3 float32 ulps of the pair each from an exact value (2^-17.5); fp32 outputs keep it in double.
RECURRENCE = {torch.float32: 0.0, torch.bfloat16: 2.0 ** -17, torch.float16: 2.0 ** -17}
# Half the spacing of the output dtype's subnormals: below 2^-14 an fp16 output rounds to a
# multiple of 2^-24, so its rounding error is up to 2^-25 whatever its relative size.
SUBNORMAL_HALF = {torch.float32: 0.0, torch.bfloat16: 2.0 ** -134, torch.float16: 2.0 ** -25}


def _bound(n: np.ndarray, base: float, recurrence: float = 0.0) -> np.ndarray:
    """RoPE tolerance for pairs (n_2i, n_2i+1), plus a float32 term for the norm.  The fused
    kernels form every angle pos * freq in double and reduce it exactly before a float32
    sincospi, so the bound does not grow with the position: 16 float32 ulps of the pair, plus
    `recurrence` of the pair for a float32 rotation recurrence."""
    mag = np.abs(n[..., 0::2]) + np.abs(n[..., 1::2])
    b = (P.ROPE_ANGLE_ULPS * 2.0 ** -24 + 2.0 ** -21 + 2.0 ** -20 + recurrence) * mag
    out = np.empty_like(n)
    out[..., 0::2] = b
    out[..., 1::2] = b
    return out


CASES = [(torch.bfloat16, (2, 64, 4096), True), (torch.bfloat16, (1, 128, 8192), False),
         (torch.float32, (3, 33, 1000), True), (torch.float16, (2, 50, 256), False),
         (torch.bfloat16, (3, 5, 6), True), (torch.float32, (4, 2, 3, 40), False),
         # the 16-bit kernel's walks over rows b, b + G, ... (G = rows / W workgroups, W = 32
         # rows for row groups over 256 threads and at least 16384 rows, else 16): no sequence
         # end (W = 32, G = 512, seq 16384), returning to the walk's first position every 4 rows
         # (seq 2048 a multiple of G = 512) and on every row (W = 16, G = 128 a multiple of seq
         # 64), angles evaluated afresh where a walk crosses a sequence end (W = 16, G = 938, seq
         # 3000; W = 32, G = 563), and 640-thread rows returning every 16 rows (W = 32, G = 512)
         (torch.bfloat16, (1, 16384, 4096), False), (torch.float16, (8, 2048, 4096), True),
         (torch.bfloat16, (32, 64, 1024), True), (torch.bfloat16, (5, 3000, 4096), False),
         (torch.bfloat16, (6, 3000, 4096), False), (torch.bfloat16, (2, 8192, 5120), True),
         # rows of more than 1024 chunks: the one-shot rows with each pair's rotation evaluated
         # directly (two to four chunks per thread)
         (torch.bfloat16, (2, 64, 16384), True), (torch.float32, (3, 16, 6144), False),
         (torch.float16, (1, 40, 12288), True)]


@pytest.mark.parametrize("dtype,shape,with_res", CASES,
                         ids=[f"{str(c[0]).split('.')[-1]}-{'x'.join(map(str, c[1]))}-{c[2]}"
                              for c in CASES])
@pytest.mark.parametrize("base", [10000.0, 500000.0])
def test_fused_norm_rope_matches_the_oracle_composition(dtype, shape, with_res, base):
    print(f"rmsnorm_rope {dtype} {shape} res={with_res} base={base}", flush=True)
    rng = np.random.default_rng(shape[-1] + len(shape))
    xs = P.gaussian(rng, shape)
    xs.reshape(-1, shape[-1])[0] = 0.0              # a floored row (mean square 0)
    x = P.to_device(xs, dtype)
    r = P.to_device(P.gaussian(rng, shape), dtype) if with_res else None
    w = P.to_device(P.weight_vec(rng, shape[-1]), dtype)
    y, h, inv = vk.rmsnorm_rope_forward(x, w, 1e-6, base, residual=r)
    assert y.dtype == dtype and y.shape == x.shape and inv.shape == x.shape[:-1] + (1,)
    h32 = P.upcast(x) + (P.upcast(r) if with_res else 0.0)
    if with_res:
        if dtype == torch.float32:
            assert np.array_equal(P.upcast(h), h32)
        else:
            P.assert_within_ulp(h, h32, 0, "h")
    else:
        assert h is x
    n, rinv = ora.rmsnorm_module_forward(h32.astype(np.float64), P.upcast(w).astype(np.float64),
                                         1e-6)
    want = ora.apply_rotary_emb(n, base)
    assert P.rel_err(P.upcast(inv), rinv) <= P.FP32_REL_TOL
    tol = (_bound(n, base, RECURRENCE[dtype]) + ROUNDING[dtype] * np.abs(want)
           + SUBNORMAL_HALF[dtype])
    err = np.abs(P.upcast(y).astype(np.float64) - want)
    assert np.all(err <= tol), float((err - tol).max())


def test_fused_equals_the_two_pass_path_up_to_the_intermediate_rounding():
    """fp32: the fused pass and rmsnorm_forward + fused_rope_interleaved agree closely (the
    two-pass path rounds the normalised rows once more and evaluates every angle afresh).
    The row statistic is the same fp32 sum of squares taken in another order (the module-form
    norm without a residual reads two 16-byte chunks per thread, the fused pass one), so the
    two inv_rms agree to a couple of ulps rather than bit for bit."""
    torch.manual_seed(0)
    x = torch.randn(2, 256, 1024, device="cuda")
    w = 1 + 0.1 * torch.randn(1024, device="cuda")
    y, _, inv = vk.rmsnorm_rope_forward(x, w, 1e-6, 10000.0)
    n, inv2 = vk.rmsnorm_forward(x, w, 1e-6)
    y2 = vk.fused_rope_interleaved(n, 10000.0)
    assert P.rel_err(P.upcast(inv), P.upcast(inv2)) <= 2.0 ** -21
    assert float((y - y2).abs().max()) < 2e-4


def test_module_autograd_matches_torch_float64():
    rng = np.random.default_rng(5)
    b, s, d = 2, 40, 512
    x32 = P.gaussian(rng, (b, s, d))
    mod = vnn.RMSNormRoPE(d, eps=1e-6, base=10000.0).cuda()
    with torch.no_grad():
        mod.weight.copy_(torch.from_numpy(P.weight_vec(rng, d)))
    x = torch.from_numpy(x32).cuda().requires_grad_(True)
    y = mod(x)
    g = torch.from_numpy(P.gaussian(rng, (b, s, d))).cuda()
    y.backward(g)

    t = torch.from_numpy(x32.astype(np.float64)).requires_grad_(True)
    tw = mod.weight.detach().double().cpu().requires_grad_(True)
    n = torch.nn.functional.rms_norm(t, (d,), tw, 1e-6)
    z = torch.view_as_complex(n.reshape(b, s, d // 2, 2))
    inv_freq = 10000.0 ** (-torch.arange(0, d, 2, dtype=torch.float64) / d)
    ang = torch.arange(s, dtype=torch.float64)[:, None] * inv_freq[None, :]
    ref = torch.view_as_real(z * torch.polar(torch.ones_like(ang), ang)).reshape(b, s, d)
    ref.backward(g.double().cpu())
    assert float((y.detach().double().cpu() - ref.detach()).abs().max()) < 1e-4
    assert float((x.grad.double().cpu() - t.grad).abs().max()) < 1e-3 * float(t.grad.abs().max())
    rw = tw.grad
    assert float((mod.weight.grad.double().cpu() - rw).abs().max()) < 1e-3 * float(rw.abs().max())


def test_errors():
    x = torch.zeros(2, 4, 7, device="cuda")
    with pytest.raises(ValueError):
        vk.rmsnorm_rope_forward(x)                                  # odd dim
    with pytest.raises(ValueError):
        vk.rmsnorm_rope_forward(torch.zeros(8, device="cuda"))     # no seq axis
    with pytest.raises(ValueError):
        vk.rmsnorm_rope_forward(torch.zeros(2, 4, 8, device="cuda"), base=0.0)
    with pytest.raises(TypeError):
        vk.rmsnorm_rope_forward(np.zeros((2, 4, 8), np.float32))


# ---------------------------------------------------------------------------------------------
# The backward in one pass (velograd_rmsnorm_rope_bwd): grad_y rotated back in registers, then
# the norm's backward.  Truth is the composition of the two pinned float64 oracles: the inverse
# interleaved rotation (functional.py:316-345) then the module backward (nn.py:357-383) with the
# device's h and inv_rms.  Bound: 16 float32 ulps of each gradient pair (angles in double), plus
# 2^-18 of the pair for the float32 rotation recurrence of the backward walks (bwd_vec_kernel's
# and bwd_rope_ring_kernel's, each re-evaluated directly every 16 rows and at sequence ends, so
# at most 15 steps of about 3 float32 ulps each, whatever the walk's length),
# propagated through dx = r (w g - xhat mean(w g xhat)) and dweight = sum g xhat; on top of it
# the usual dx rule (1 ulp or the operand-scaled floor) and the dweight rule (1e-3).
# ---------------------------------------------------------------------------------------------
def _rope_grad_bound(g: np.ndarray, base: float) -> np.ndarray:
    mag = np.abs(g[..., 0::2]) + np.abs(g[..., 1::2])
    b = (P.ROPE_ANGLE_ULPS * 2.0 ** -24 + 2.0 ** -18) * mag
    out = np.empty_like(g)
    out[..., 0::2] = b
    out[..., 1::2] = b
    return out


def _check_rope_backward(dx, dw, g, h, w, inv, base, what, g_round=0.0, positions=None):
    """`g_round`: relative rounding of the rotated-back gradient before the norm's backward
    (the two-pass path stores it in the activation dtype; the fused pass keeps it in fp32).
    `positions`: the rows' positions when the tensors are a slice of rows (dw is then None)."""
    d = g.shape[-1]
    g64, h64 = P.upcast(g).astype(np.float64), P.upcast(h).astype(np.float64)
    r = P.upcast(inv).astype(np.float64)
    w64 = np.ones(d) if w is None else P.upcast(w).astype(np.float64).reshape(-1)
    gn = ora.apply_rotary_emb(g64, base, inverse=True, positions=positions)
    tdx, tdw = ora.rmsnorm_module_backward(gn, h64, None if w is None else w64, r)
    xhat = h64 * r
    dg = _rope_grad_bound(g64, base) + g_round * np.abs(gn)
    ddx = r * (np.abs(w64) * dg + np.abs(xhat) * np.mean(np.abs(w64 * xhat) * dg, axis=-1,
                                                           keepdims=True))
    gw = gn * w64
    scale = P.dx_scale(gw.reshape(-1, d), xhat.reshape(-1, d), r.reshape(-1, 1)).reshape(gn.shape)
    half_ulp = {torch.float32: 0.0, torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}[dx.dtype]
    err = np.abs(P.upcast(dx).astype(np.float64) - tdx)
    tol = ddx + P.DX_FLOOR * scale + half_ulp * np.abs(tdx) + 1e-6 * scale + SUBNORMAL_HALF[dx.dtype]
    assert np.all(err <= tol), f"{what}: dx over its bound by {float((err - tol).max()):.3e}"
    if positions is not None:
        return
    if w is not None:
        ddw = np.sum((np.abs(xhat) * dg).reshape(-1, d), axis=0)
        got = dw.detach().cpu().numpy().astype(np.float64)
        sc = np.maximum(np.abs(tdw), np.sqrt(np.mean(tdw * tdw)))
        assert np.all(np.abs(got - tdw) <= ddw + P.DWEIGHT_REL_TOL * sc), f"{what}: dweight"
    else:
        assert dw is None


BWD_CASES = [(torch.bfloat16, (2, 64, 4096), True), (torch.bfloat16, (1, 128, 8192), True),
             (torch.float32, (3, 33, 1000), True), (torch.float16, (2, 50, 256), False),
             (torch.bfloat16, (3, 5, 6), True), (torch.float32, (4, 2, 3, 40), True),
             (torch.bfloat16, (1, 16384, 4096), True), (torch.bfloat16, (8, 2048, 4096), True),
             # the ring kernel (bwd_rope_ring_kernel, one 512-thread workgroup per CU): fp32
             # with two row groups per workgroup and a 32-row walk; fp16 with eight row groups
             # and no weight, one or two rows per slot; four row groups, a partial last
             # iteration and a return to the walk's first position on every row; two row groups
             # returning on every second row; 384-thread workgroups, two per CU.  Then a shape
             # whose walks cross sequence ends at other positions: bwd_vec_kernel's walk
             (torch.float32, (4, 4096, 1024), True), (torch.float16, (3, 1000, 512), False),
             (torch.bfloat16, (257, 64, 1024), True), (torch.bfloat16, (8, 1024, 2048), True),
             (torch.bfloat16, (2, 1024, 3072), True),
             # two chunks per thread (rows of 513 to 1024 chunks): 320-, 384-, 448- and
             # 512-thread row groups, fp32, fp16 and bf16; then the same widths where walks cross
             # sequence ends
             # elsewhere (bwd_vec_kernel)
             (torch.bfloat16, (2, 1024, 5120), True), (torch.bfloat16, (4, 512, 7168), False),
             (torch.float32, (2, 1024, 2560), True), (torch.float32, (1, 4096, 4096), True),
             (torch.float16, (2, 512, 6144), True),
             (torch.bfloat16, (6, 1000, 4096), True), (torch.bfloat16, (3, 1000, 8192), True),
             # wider rows: bwd_vec_kernel's walk with three chunks per thread (1280 and 1536
             # chunks); then rows no walk plan fits, bwd_vec_kernel with each pair's rotation
             # evaluated where g is decoded: 1540 chunks as two per thread in 832-thread rows,
             # 2048 chunks as four per thread in 512-thread rows
             (torch.bfloat16, (1, 300, 10240), False), (torch.bfloat16, (2, 256, 12288), True),
             (torch.bfloat16, (1, 64, 12320), True), (torch.bfloat16, (1, 64, 16384), True)]


@pytest.mark.parametrize("dtype,shape,with_w", BWD_CASES,
                         ids=[f"{str(c[0]).split('.')[-1]}-{'x'.join(map(str, c[1]))}-w{c[2]}"
                              for c in BWD_CASES])
@pytest.mark.parametrize("base", [10000.0, 500000.0])
def test_fused_backward_matches_the_oracle_composition(dtype, shape, with_w, base):
    print(f"rmsnorm_rope backward {dtype} {shape} w={with_w} base={base}", flush=True)
    rng = np.random.default_rng(shape[-1] * 3 + len(shape))
    x = P.to_device(P.gaussian(rng, shape), dtype)
    w = P.to_device(P.weight_vec(rng, shape[-1]), dtype) if with_w else None
    g = P.to_device(P.gaussian(rng, shape), dtype)
    _, h, inv = vk.rmsnorm_rope_forward(x, w, 1e-6, base)
    dx, dw = vk.rmsnorm_rope_backward(g, h, w, inv, base)
    torch.cuda.synchronize()
    _check_rope_backward(dx, dw, g, h, w, inv, base, f"{dtype} {shape}")
    # the two-pass path it replaces lands in the same bound (and the two agree closely)
    g_back = vk.fused_rope_interleaved(g, base, inverse=True)
    dx2, dw2 = vk.fused_rmsnorm_residual_backward(g_back, h, w, inv, saved_is_h=True)
    g_round = {torch.float32: 0.0, torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}[dtype]
    _check_rope_backward(dx2, dw2, g, h, w, inv, base, f"two-pass {dtype} {shape}", g_round)


def test_fused_backward_long_fp32_walk():
    """fp32, one sequence of 131072 positions at dim 4096: the ring kernel with two chunks per
    thread (512-thread row groups, one per CU), so each of the 256 slots walks 512 rows of one
    sequence with no position wrap. The rotation state is re-evaluated every 16 rows, so the last
    rows of the walks (and the middle ones) keep the same 2^-18 recurrence bound as short
    walks."""
    seq, d, base = 131072, 4096, 500000.0
    print(f"rmsnorm_rope backward fp32 long walk: seq={seq} dim={d}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(11)
    x = torch.randn(1, seq, d, device="cuda", generator=gen)
    g = torch.randn(1, seq, d, device="cuda", generator=gen)
    w = 1.0 + 0.1 * torch.randn(d, device="cuda", generator=gen)
    _, h, inv = vk.rmsnorm_rope_forward(x, w, 1e-6, base)
    dx, _ = vk.rmsnorm_rope_backward(g, h, w, inv, base)
    torch.cuda.synchronize()
    del x
    for lo, hi in ((0, 256), (seq // 2 - 256, seq // 2 + 256), (seq - 512, seq)):
        sl = slice(lo, hi)
        _check_rope_backward(dx[:, sl], None, g[:, sl], h[:, sl], w, inv[:, sl], base,
                             f"fp32 long walk rows {lo}..{hi}",
                             positions=np.arange(lo, hi))


@pytest.mark.parametrize("dtype,seq,d", [(torch.bfloat16, 131072, 4096),
                                         (torch.float32, 65536, 2048)])
def test_fused_backward_long_ring_walk(dtype, seq, d):
    """The ring kernel (rows of 512 chunks: bf16 dim 4096, fp32 dim 2048) over one sequence of
    seq positions: each of its 256 slots (one workgroup per CU) walks seq / 256 rows (512, 256)
    with no position wrap, re-evaluating its rotations every 16 rows; rows at the start, middle
    and end of the walks keep the 2^-18 recurrence bound."""
    base = 500000.0
    print(f"rmsnorm_rope backward ring long walk: {dtype} seq={seq} dim={d}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(13)
    x = torch.randn(1, seq, d, device="cuda", generator=gen).to(dtype)
    g = torch.randn(1, seq, d, device="cuda", generator=gen).to(dtype)
    w = (1.0 + 0.1 * torch.randn(d, device="cuda", generator=gen)).to(dtype)
    _, h, inv = vk.rmsnorm_rope_forward(x, w, 1e-6, base)
    dx, _ = vk.rmsnorm_rope_backward(g, h, w, inv, base)
    torch.cuda.synchronize()
    del x
    for lo, hi in ((0, 1024), (seq // 2 - 512, seq // 2 + 512), (seq - 1024, seq)):
        sl = slice(lo, hi)
        _check_rope_backward(dx[:, sl], None, g[:, sl], h[:, sl], w, inv[:, sl], base,
                             f"{dtype} ring long walk rows {lo}..{hi}",
                             positions=np.arange(lo, hi))


def test_fused_backward_is_deterministic():
    rng = np.random.default_rng(9)
    x = P.to_device(P.gaussian(rng, (4, 1024, 4096)), torch.bfloat16)
    w = P.to_device(P.weight_vec(rng, 4096), torch.bfloat16)
    g = P.to_device(P.gaussian(rng, (4, 1024, 4096)), torch.bfloat16)
    _, h, inv = vk.rmsnorm_rope_forward(x, w, 1e-6, 10000.0)
    outs = [vk.rmsnorm_rope_backward(g, h, w, inv, 10000.0) for _ in range(3)]
    for dx, dw in outs[1:]:
        assert torch.equal(dx, outs[0][0]) and torch.equal(dw, outs[0][1])


def test_fused_forward_is_bitwise_repeatable_on_any_stream():
    """The forward at the headline shape, with and without a residual, gives bit-identical y,
    h and inv_rms on every call: on the current stream and on a side stream, interleaved with
    calls on other buffers."""
    rng = np.random.default_rng(21)
    x = P.to_device(P.gaussian(rng, (8, 2048, 4096)), torch.bfloat16)
    r = P.to_device(P.gaussian(rng, (8, 2048, 4096)), torch.bfloat16)
    x2 = P.to_device(P.gaussian(rng, (8, 2048, 4096)), torch.bfloat16)
    w = P.to_device(P.weight_vec(rng, 4096), torch.bfloat16)
    ref = vk.rmsnorm_rope_forward(x, w, 1e-5, 10000.0)
    ref_r = vk.rmsnorm_rope_forward(x, w, 1e-5, 10000.0, residual=r)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    outs = []
    with torch.cuda.stream(side):
        for _ in range(2):
            outs.append((vk.rmsnorm_rope_forward(x, w, 1e-5, 10000.0), ref))
            vk.rmsnorm_rope_forward(x2, w, 1e-5, 10000.0, residual=r)
            outs.append((vk.rmsnorm_rope_forward(x, w, 1e-5, 10000.0, residual=r), ref_r))
    torch.cuda.current_stream().wait_stream(side)
    outs.append((vk.rmsnorm_rope_forward(x, w, 1e-5, 10000.0), ref))
    torch.cuda.synchronize()
    for got, want in outs:
        assert torch.equal(got[0], want[0]), "y"
        assert torch.equal(got[2], want[2]), "inv_rms"
        if want[1] is not None:
            assert torch.equal(got[1], want[1]), "h"


def test_every_output_row_is_written_on_every_call():
    """Each forward writes every row of y and inv_rms on every call: outputs NaN-filled before
    each of 8 calls (4 on the current stream, 4 on a side stream) at the headline shape, for the
    fused norm + RoPE (one 64-byte inv_rms block per workgroup) and the plain forward (one float
    per workgroup), each call equal to the first bit for bit."""
    from velograd_amd import _lib
    lib = _lib.load()
    rows, d = 16384, 4096
    rng = np.random.default_rng(5)
    x = P.to_device(P.gaussian(rng, (rows, d)), torch.bfloat16)
    r = P.to_device(P.gaussian(rng, (rows, d)), torch.bfloat16)
    w = P.to_device(P.weight_vec(rng, d), torch.bfloat16)
    y = torch.empty_like(x)
    h = torch.empty_like(x)
    inv = torch.empty(rows, device="cuda")
    bf = _lib.DTYPE_BF16
    side = torch.cuda.Stream()

    def rope(res, sp):
        return lib.velograd_rmsnorm_rope_fwd(
            x.data_ptr(), r.data_ptr() if res else None, w.data_ptr(), y.data_ptr(),
            h.data_ptr() if res else None, inv.data_ptr(), rows, d, d, d, d, d, 2048, bf, bf,
            1e-5, 1e-12, 10000.0, sp)

    def plain(res, sp):
        return lib.velograd_rmsnorm_residual_fwd(
            x.data_ptr(), r.data_ptr() if res else None, w.data_ptr(), y.data_ptr(),
            h.data_ptr() if res else None, inv.data_ptr(), rows, d, d, d, d, d, bf, bf, 1e-5, sp)

    for name, fn in (("rmsnorm_rope_fwd", rope), ("rmsnorm_residual_fwd", plain)):
        for res in (False, True):
            first = None
            for call in range(8):
                stream = side if call % 2 else torch.cuda.current_stream()
                stream.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(stream):
                    y.fill_(float("nan"))
                    inv.fill_(float("nan"))
                    _lib.check(fn(res, stream.cuda_stream), name)
                torch.cuda.current_stream().wait_stream(stream)
                torch.cuda.synchronize()
                what = f"{name} res={res} call {call}"
                assert not bool(inv.isnan().any()), f"{what}: inv_rms rows left unwritten"
                assert not bool(y.isnan().any()), f"{what}: y rows left unwritten"
                if first is None:
                    first = (y.clone(), inv.clone())
                else:
                    assert torch.equal(y, first[0]) and torch.equal(inv, first[1]), what


def test_backward_errors():
    g = torch.zeros(2, 4, 8, device="cuda")
    inv = torch.ones(2, 4, 1, device="cuda")
    with pytest.raises(ValueError):
        vk.rmsnorm_rope_backward(torch.zeros(2, 4, 7, device="cuda"),
                                 torch.zeros(2, 4, 7, device="cuda"), None, inv)   # odd dim
    with pytest.raises(ValueError):
        vk.rmsnorm_rope_backward(g, g[:, :2], None, inv)                           # h shape
    with pytest.raises(ValueError):
        vk.rmsnorm_rope_backward(g, g, None, inv[:, :2])                           # inv_rms rows
    with pytest.raises(ValueError):
        vk.rmsnorm_rope_backward(g, g, None, inv, base=-1.0)                       # base
    with pytest.raises(TypeError):
        vk.rmsnorm_rope_backward(np.zeros((2, 4, 8), np.float32), g, None, inv)


_FORWARD_NV_CHILD = r'''
import sys
sys.path.insert(0, sys.argv[1])
import torch
from tests.test_gpu_rmsnorm_rope import test_fused_norm_rope_matches_the_oracle_composition as t
dt = {"bf16": torch.bfloat16, "fp32": torch.float32}[sys.argv[2]]
shape = tuple(int(v) for v in sys.argv[3].split("x"))
for with_res in (False, True):
    for base in (10000.0, 500000.0):
        t(dt, shape, with_res, base)
print("forward-nv ok", flush=True)
'''


@pytest.mark.parametrize("nv,dtype,shape", [(3, "bf16", "1x64x12288"), (4, "bf16", "1x64x16384"),
                                            (4, "fp32", "2x16x8192")])
def test_fused_forward_three_and_four_chunks_per_thread(nv, dtype, shape):
    """The one-shot rows with each pair's rotation evaluated directly at three and four chunks
    per thread (512-thread rows).  The default plans take two chunks per thread up to 2048
    chunks, so these layouts run only under VELOGRAD_FWD_NV, read once per process: a child
    process with it set runs the oracle comparison above on rows of 1536 and 2048 chunks."""
    import os
    import subprocess
    import sys
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print(f"child: VELOGRAD_FWD_NV={nv} rmsnorm_rope forward {dtype} {shape}", flush=True)
    env = dict(os.environ, VELOGRAD_FWD_NV=str(nv))
    out = subprocess.run([sys.executable, "-c", _FORWARD_NV_CHILD, repo, dtype, shape], env=env,
                         capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, (out.stdout[-2000:], out.stderr[-4000:])
    assert "forward-nv ok" in out.stdout
