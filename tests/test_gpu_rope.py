"""GPU parity of the fused RoPE kernel (velograd_rope) against the oracle restatement of
python/velograd/kernels/fused.py:72-130 on the same inputs.

Tolerance (tests/_parity.py, stated there): per rotated element
|got - want| <= (16 * 2^-24 * max(|angle|, 1) + 2^-21) * (|x1| + |x2|), i.e. a few float32 ulps of
the angle (NumPy's float32 power is faithful, not correctly rounded, so freq and with it the
angle may differ by ulps) plus a few ulps of the operands; reduced-precision outputs may also
differ by their own rounding (half an ulp: 2^-8 relative for bf16, 2^-11 for fp16).  Elements past
head_dim are copied exactly."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import fused_rmsnorm as ora
from tests import _parity as P
from velograd_amd import _lib
from velograd_amd import kernels as vk
from velograd_amd import nn as vnn

pytestmark = pytest.mark.gpu

ROUNDING = {torch.float32: 0.0, torch.bfloat16: 2.0 ** -8 * 1.01, torch.float16: 2.0 ** -11 * 1.01}


def _say(msg):
    print(msg, flush=True)


def _check(got: torch.Tensor, x: torch.Tensor, hd: int, theta: float, inverse=False, what=""):
    x32 = P.upcast(x)
    want, _ = ora.fused_rope_forward(x32, None, head_dim=hd, theta=theta, inverse=inverse)
    xc = P.rope_canonical(x32, hd)
    P.assert_rope_close(P.rope_canonical(P.upcast(got), hd), P.rope_canonical(want, hd), xc, hd,
                        theta, extra=ROUNDING[got.dtype], what=what)


CASES = [
    # (q shape, k shape or None, head_dim, theta, dtype)
    ((512, 1024), None, 64, 10000.0, torch.float32),            # bench_vs_pytorch.py:57-59
    ((33, 64), (33, 64), None, 10000.0, torch.bfloat16),        # 2-D, one head
    ((2, 128, 8, 64), (2, 128, 2, 64), None, 10000.0, torch.bfloat16),   # GQA
    ((3, 16, 96), None, 64, 10000.0, torch.float16),            # pass-through tail, vector path
    ((1, 50, 3, 10), (1, 50, 5, 6), 6, 10000.0, torch.float32),  # scalar path (half = 3)
    ((1, 32768, 2, 64), None, None, 10000.0, torch.float32),    # long positions
    ((4096, 32, 128), (4096, 8, 128), None, 500000.0, torch.bfloat16),  # Llama-3-like
]


@pytest.mark.parametrize("qs,ks,hd,theta,dtype", CASES, ids=[str(c[0]) for c in CASES])
def test_rope_matches_oracle(qs, ks, hd, theta, dtype):
    _say(f"rope q{qs} k{ks} hd={hd} theta={theta} {dtype}")
    rng = np.random.default_rng(sum(qs))
    q = P.to_device(P.gaussian(rng, qs), dtype)
    k = P.to_device(P.gaussian(rng, ks), dtype) if ks is not None else None
    h_dim = hd or qs[-1]
    q_rot, k_rot = vk.fused_rope_forward(q, k, head_dim=hd, theta=theta)
    assert q_rot.shape == q.shape and q_rot.dtype == dtype
    _check(q_rot, q, h_dim, theta, what="q")
    if k is not None:
        assert k_rot.shape == k.shape
        _check(k_rot, k, h_dim, theta, what="k")
    else:
        assert k_rot is None


def test_rope_reference_wrapper_case_host_arrays():
    """The reference test's call (tests/test_exhaustive.py:126-128) with NumPy input: float32
    ndarray out, computed on the GPU."""
    x = P.gaussian(np.random.default_rng(1), (4, 16))
    out = vk.fused_rope(x, head_dim=8)
    assert isinstance(out, np.ndarray) and out.dtype == np.float32 and out.shape == (4, 16)
    want = ora.fused_rope(x, head_dim=8)
    P.assert_rope_close(P.rope_canonical(out, 8), P.rope_canonical(want, 8),
                        P.rope_canonical(x, 8), 8, 10000.0)
    q_rot, k_rot = vk.fused_rope(x, x * 2, head_dim=8)
    assert np.array_equal(q_rot, out)
    P.assert_rope_close(P.rope_canonical(k_rot, 8), P.rope_canonical(want * 2, 8),
                        P.rope_canonical(x * 2, 8), 8, 10000.0)


def test_rope_position_zero_exact_and_tail_copied():
    rng = np.random.default_rng(2)
    x = P.to_device(P.gaussian(rng, (2, 9, 4, 80)), torch.bfloat16)
    y, _ = vk.fused_rope_forward(x, head_dim=64)
    assert torch.equal(y[:, 0], x[:, 0])
    assert torch.equal(y[..., 64:], x[..., 64:])


def test_rope_backward_is_inverse_and_adjoint():
    _say("rope backward")
    rng = np.random.default_rng(3)
    x = P.to_device(P.gaussian(rng, (2, 300, 4, 128)), torch.float32)
    g = P.to_device(P.gaussian(rng, (2, 300, 4, 128)), torch.float32)
    y, _ = vk.fused_rope_forward(x)
    gx, _ = vk.fused_rope_backward(g)
    _check(gx, g, 128, 10000.0, inverse=True, what="backward")
    lhs = float((y.double() * g.double()).sum())
    rhs = float((x.double() * gx.double()).sum())
    assert abs(lhs - rhs) <= 1e-5 * float((x.double().abs() * gx.double().abs()).sum())
    back, _ = vk.fused_rope_backward(y)
    assert float((back - x).abs().max()) <= 1e-4


def test_rope_in_place_through_the_c_abi():
    rng = np.random.default_rng(4)
    x = P.to_device(P.gaussian(rng, (1, 64, 8, 128)), torch.bfloat16)
    want, _ = vk.fused_rope_forward(x)
    buf = x.clone()
    rc = _lib.load().velograd_rope(buf.data_ptr(), buf.data_ptr(), 1, 64, 8, 128, 128, 10000.0,
                                   0, _lib.ROPE_HALF, _lib.DTYPE_BF16,
                                   torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "velograd_rope in place")
    assert torch.equal(buf, want)


def test_rope_layout_errors():
    x = torch.zeros(4, 30, device="cuda")
    with pytest.raises(ValueError):
        vk.fused_rope_forward(x, head_dim=8)            # 30 is not a multiple of 8
    with pytest.raises(ValueError):
        vk.fused_rope_forward(x, head_dim=7)            # odd head_dim
    with pytest.raises(ValueError):
        vk.fused_rope_forward(torch.zeros(2, 5, 3, 16, device="cuda"),
                              torch.zeros(2, 6, 3, 16, device="cuda"))   # k positions differ


def test_rope_empty_and_deterministic():
    e = torch.empty(0, 8, 64, device="cuda", dtype=torch.bfloat16)
    assert vk.fused_rope_forward(e)[0].shape == e.shape
    rng = np.random.default_rng(5)
    x = P.to_device(P.gaussian(rng, (512, 16, 64)), torch.bfloat16)
    assert torch.equal(vk.fused_rope_forward(x)[0], vk.fused_rope_forward(x)[0])


# ---------------------------------------------------------------------------------------------
# Interleaved pairs: the reference model's apply_rotary_emb (functional.py:287-345)
# ---------------------------------------------------------------------------------------------
def _interleaved_bound(x: np.ndarray, base: float) -> np.ndarray:
    """Tolerance for pairs (x_2i, x_2i+1): ROPE_ANGLE_ULPS float32 ulps of the pair for cos and
    sin plus 2^-21 for the rotation's products.  It does not grow with the position: both paths
    form the angles in double (as the reference's Python floats do) and reduce them exactly
    before a float32 sincospi; the 16-byte path does so for every position of fp32 outputs and
    for the first of each 3-position tile of bf16/fp16 ones, whose next two positions advance the
    float32 rotation by a step rotation (a few float32 ulps each)."""
    x = np.abs(np.asarray(x, np.float64))
    mag = x[..., 0::2] + x[..., 1::2]
    b = (P.ROPE_ANGLE_ULPS * 2.0 ** -24 + 2.0 ** -21) * mag
    out = np.empty_like(x)
    out[..., 0::2] = b
    out[..., 1::2] = b
    return out


INTERLEAVED_CASES = [(torch.float32, (37, 64)), (torch.bfloat16, (2, 128, 4096)),
                     (torch.float16, (3, 50, 256)), (torch.bfloat16, (1, 64, 8192)),
                     (torch.bfloat16, (1, 64, 16384)),
                     (torch.float32, (3, 5, 6)), (torch.bfloat16, (2, 9, 12)),
                     (torch.float32, (2, 9, 12)), (torch.float32, (4, 2, 3, 40)),
                     # the scalar path at long positions (10 and 12 elements do not split into
                     # 16-byte chunks of whole pairs)
                     (torch.float32, (1, 32768, 10)), (torch.bfloat16, (1, 20000, 12))]


@pytest.mark.parametrize("dtype,shape", INTERLEAVED_CASES,
                         ids=[f"{str(d).split('.')[-1]}-{'x'.join(map(str, s))}"
                              for d, s in INTERLEAVED_CASES])
@pytest.mark.parametrize("base", [10000.0, 500000.0])
def test_interleaved_rope_matches_oracle(dtype, shape, base):
    _say(f"rope interleaved {dtype} {shape} base {base}")
    rng = np.random.default_rng(len(shape) + shape[-1])
    x = P.to_device(P.gaussian(rng, shape), dtype)
    x64 = P.upcast(x).astype(np.float64)
    for inverse in (False, True):
        got = vk.fused_rope_interleaved(x, base, inverse=inverse)
        assert got.dtype == dtype and got.shape == x.shape
        want = ora.apply_rotary_emb(x64, base, inverse=inverse)
        tol = _interleaved_bound(x64, base) + ROUNDING[dtype] * np.abs(want)
        err = np.abs(P.upcast(got).astype(np.float64) - want)
        assert np.all(err <= tol), (inverse, float((err - tol).max()))
    # position 0 of every leading index is the identity (bit-exact)
    assert torch.equal(vk.fused_rope_interleaved(x, base)[..., 0, :], x[..., 0, :])


def test_interleaved_rope_round_trip_and_autograd():
    rng = np.random.default_rng(9)
    x32 = P.gaussian(rng, (2, 33, 256))
    x = torch.from_numpy(x32).cuda().requires_grad_(True)
    y = vnn.apply_rotary_emb(x, 10000.0)
    g = torch.from_numpy(P.gaussian(rng, (2, 33, 256))).cuda()
    y.backward(g)
    # torch float64 autograd of the complex formulation on the CPU
    t = torch.from_numpy(x32.astype(np.float64)).requires_grad_(True)
    z = torch.view_as_complex(t.reshape(2, 33, 128, 2))
    inv_freq = 10000.0 ** (-torch.arange(0, 256, 2, dtype=torch.float64) / 256)
    ang = torch.arange(33, dtype=torch.float64)[:, None] * inv_freq[None, :]
    ref = torch.view_as_real(z * torch.polar(torch.ones_like(ang), ang)).reshape(2, 33, 256)
    ref.backward(g.double().cpu())
    assert float((y.detach().double().cpu() - ref.detach()).abs().max()) < 2e-4
    assert float((x.grad.double().cpu() - t.grad).abs().max()) < 2e-4
    back = vk.fused_rope_interleaved(y.detach(), 10000.0, inverse=True)
    assert float((back - x.detach()).abs().max()) < 1e-4


# The 16-byte interleaved path (rope_tile_kernel) through the C ABI: several heads, a rotated
# prefix of each head with the rest copied, in place, token vectors of fewer than 256 chunks and
# of a number of chunks that is not a multiple of 256, every remainder of the sequence length by
# the kernel's 3-position tiles, and bases under 1 (whose step rotations exceed one radian and are
# reduced as the tiles' first rotations are).
TILE_CASES = [
    # (dtype, outer, seq, heads, dim, rot_dim, base)
    (torch.bfloat16, 2, 49, 4, 128, 64, 10000.0),
    (torch.float16, 1, 50, 1, 4104, 4104, 10000.0),
    (torch.float32, 3, 31, 2, 48, 32, 500000.0),
    (torch.bfloat16, 1, 64, 8, 256, 256, 0.5),
    (torch.float32, 2, 65, 1, 512, 512, 0.25),
    (torch.float16, 1, 7, 3, 2048, 1024, 10000.0),
    (torch.bfloat16, 1, 3, 1, 8, 8, 10000.0),
]
_CODES = {torch.float32: _lib.DTYPE_F32, torch.float16: _lib.DTYPE_F16,
          torch.bfloat16: _lib.DTYPE_BF16}


def _heads_want(x64: np.ndarray, rot: int, base: float, inverse: bool) -> np.ndarray:
    """x64 [outer, seq, heads, dim]: each head's first `rot` elements rotated by the oracle
    (positions moved to axis -2 for it), the rest copied."""
    want = x64.copy()
    part = np.ascontiguousarray(x64[..., :rot].transpose(0, 2, 1, 3))
    want[..., :rot] = ora.apply_rotary_emb(part, base, inverse=inverse).transpose(0, 2, 1, 3)
    return want


@pytest.mark.parametrize("dtype,outer,seq,heads,dim,rot,base", TILE_CASES,
                         ids=[f"{str(c[0]).split('.')[-1]}-{c[1]}x{c[2]}x{c[3]}x{c[4]}-r{c[5]}"
                              f"-b{c[6]}" for c in TILE_CASES])
def test_interleaved_tiles_through_the_c_abi(dtype, outer, seq, heads, dim, rot, base):
    _say(f"rope interleaved tiles {dtype} [{outer}, {seq}, {heads}, {dim}] rot {rot} base {base}")
    rng = np.random.default_rng(seq * 7 + dim)
    x = P.to_device(P.gaussian(rng, (outer, seq, heads, dim)), dtype)
    x64 = P.upcast(x).astype(np.float64)
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    for inverse in (0, 1):
        out = torch.full_like(x, float("nan"))
        _lib.check(lib.velograd_rope(x.data_ptr(), out.data_ptr(), outer, seq, heads, dim, rot,
                                     base, inverse, _lib.ROPE_INTERLEAVED, _CODES[dtype], st),
                   "velograd_rope interleaved")
        want = _heads_want(x64, rot, base, bool(inverse))
        tol = _interleaved_bound(x64, base) + ROUNDING[dtype] * np.abs(want)
        tol[..., rot:] = 0.0                                    # copied exactly
        err = np.abs(P.upcast(out).astype(np.float64) - want)
        assert np.all(err <= tol), (inverse, float((err - tol).max()))
        buf = x.clone()
        _lib.check(lib.velograd_rope(buf.data_ptr(), buf.data_ptr(), outer, seq, heads, dim, rot,
                                     base, inverse, _lib.ROPE_INTERLEAVED, _CODES[dtype], st),
                   "velograd_rope interleaved in place")
        assert torch.equal(buf, out)


def test_interleaved_rope_errors():
    with pytest.raises(ValueError):
        vk.fused_rope_interleaved(torch.zeros(4, 7, device="cuda"))      # odd dim
    with pytest.raises(ValueError):
        vk.fused_rope_interleaved(torch.zeros(8, device="cuda"))         # no seq axis
    with pytest.raises(TypeError):
        vk.fused_rope_interleaved(np.zeros((4, 8), np.float32))
