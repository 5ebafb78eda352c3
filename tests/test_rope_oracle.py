"""The RoPE oracle (restatement of python/velograd/kernels/fused.py:72-130 and the wrapper
python/velograd/kernels/__init__.py:34-48) pinned against float64 truth from the exact angles,
torch's rotate-half formulation on the CPU, closed forms and invariants, the reference test's
own shape case, and planted mistakes that the pins must catch."""

import numpy as np
import pytest
import torch

from oracle import fused_rmsnorm as ora
from tests import _parity as P


def _x(shape, seed=0, std=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * std).astype(np.float32)


def _torch_rope(x: np.ndarray, head_dim: int, theta: float) -> np.ndarray:
    """rotate-half RoPE written with torch ops on a canonical [T, S, H, D] array: q * cos +
    rotate_half(q) * sin with cos, sin of float32 angles."""
    t = torch.from_numpy(x)
    half = head_dim // 2
    j = torch.arange(half, dtype=torch.float32)
    freqs = 1.0 / (theta ** (2.0 * j / head_dim))
    ang = torch.outer(torch.arange(x.shape[1], dtype=torch.float32), freqs)
    cos = torch.cat([ang.cos(), ang.cos()], -1)[None, :, None, :]
    sin = torch.cat([ang.sin(), ang.sin()], -1)[None, :, None, :]
    r = t[..., :head_dim]
    rot_half = torch.cat([-r[..., half:], r[..., :half]], -1)
    out = r * cos + rot_half * sin
    return torch.cat([out, t[..., head_dim:]], -1).numpy()


CASES = [
    # (shape, head_dim, theta) in the layouts fused.py:86-96 accepts
    ((4, 16), 8, 10000.0),                 # the reference test's case (test_exhaustive.py:126-128)
    ((512, 1024), 64, 10000.0),            # bench_vs_pytorch.py:57-59 shape
    ((33, 64), None, 10000.0),             # 2-D, one head per row
    ((2, 37, 3, 32), None, 500000.0),      # [batch, seq, heads, head_dim]
    ((3, 16, 96), 64, 10000.0),            # [seq, heads, dim] with a 32-wide pass-through
    ((1, 4096, 2, 128), None, 10000.0),    # long positions
]


@pytest.mark.parametrize("shape,hd,theta", CASES, ids=[str(c[0]) for c in CASES])
def test_oracle_against_float64_truth_and_torch(shape, hd, theta):
    x = _x(shape)
    h_dim = hd or shape[-1]
    got, none = ora.fused_rope_forward(x, None, head_dim=hd, theta=theta)
    assert none is None and got.shape == x.shape and got.dtype == np.float32
    xc = P.rope_canonical(x, h_dim)
    gc = P.rope_canonical(got, h_dim)
    P.assert_rope_close(gc, P.rope_truth(xc, h_dim, theta), xc, h_dim, theta, what="vs truth")
    P.assert_rope_close(gc, _torch_rope(xc, h_dim, theta), xc, h_dim, theta, what="vs torch")
    # past head_dim the values are copied
    assert np.array_equal(gc[..., h_dim:], xc[..., h_dim:])


def test_wrapper_matches_forward_and_casts():
    x = _x((4, 16)).astype(np.float64)
    k = _x((4, 16), seed=1)
    q_only = ora.fused_rope(x.tolist(), head_dim=8)
    assert isinstance(q_only, np.ndarray) and q_only.dtype == np.float32 and q_only.shape == (4, 16)
    q_rot, k_rot = ora.fused_rope(x, k, head_dim=8, base=10000.0)
    rq, rk = ora.fused_rope_forward(x.astype(np.float32), k, head_dim=8)
    assert np.array_equal(q_rot, rq) and np.array_equal(k_rot, rk)
    assert np.array_equal(q_only, rq)


def test_position_zero_is_identity_and_norms_are_kept():
    x = _x((1, 50, 4, 64))
    y, _ = ora.fused_rope_forward(x)
    assert np.array_equal(y[:, 0], x[:, 0])            # cos 0 = 1, sin 0 = 0 exactly
    n_in = x[..., :32].astype(np.float64) ** 2 + x[..., 32:].astype(np.float64) ** 2
    n_out = y[..., :32].astype(np.float64) ** 2 + y[..., 32:].astype(np.float64) ** 2
    assert np.allclose(n_out, n_in, rtol=1e-6, atol=1e-6)


def test_relative_position_property():
    """<rope(q)_m, rope(k)_n> depends only on m - n (the point of RoPE)."""
    rng = np.random.default_rng(3)
    qv = rng.standard_normal(64).astype(np.float32)
    kv = rng.standard_normal(64).astype(np.float32)
    s = 40
    q = np.tile(qv, (1, s, 1, 1)).reshape(1, s, 1, 64)
    k = np.tile(kv, (1, s, 1, 1)).reshape(1, s, 1, 64)
    rq, rk = ora.fused_rope_forward(q, k)
    dots = np.einsum("sd,td->st", rq[0, :, 0].astype(np.float64), rk[0, :, 0].astype(np.float64))
    for delta in (0, 1, 5, 17):
        diag = np.array([dots[m + delta, m] for m in range(s - delta)])
        assert np.ptp(diag) <= 1e-4 * (np.abs(qv) @ np.abs(kv))


def test_inverse_is_the_adjoint_and_undoes_the_rotation():
    x = _x((2, 20, 3, 48), seed=4)
    g = _x((2, 20, 3, 48), seed=5)
    y, _ = ora.fused_rope_forward(x)
    back, _ = ora.fused_rope_forward(g, inverse=True)
    lhs = float(np.sum(y.astype(np.float64) * g))
    rhs = float(np.sum(x.astype(np.float64) * back))
    assert abs(lhs - rhs) <= 1e-5 * float(np.sum(np.abs(x) * np.abs(back)))
    undo, _ = ora.fused_rope_forward(y, inverse=True)
    assert np.allclose(undo, x, atol=1e-5)
    xc = P.rope_canonical(g, 48)
    P.assert_rope_close(back, P.rope_truth(xc, 48, 10000.0, inverse=True), xc, 48, 10000.0,
                        what="inverse vs truth")


def test_k_with_other_heads_and_2d_reshape_semantics():
    q = _x((2, 30, 8, 64))
    k = _x((2, 30, 2, 64), seed=1)           # grouped-query: fewer key heads, same positions
    rq, rk = ora.fused_rope_forward(q, k)
    assert rk.shape == k.shape
    assert np.array_equal(rk, ora.fused_rope_forward(k)[0])
    # 2-D [S, H*hd] is [S, H, hd] (fused.py:88-94, 126-129)
    q2 = _x((30, 4 * 16))
    a, _ = ora.fused_rope_forward(q2, head_dim=16)
    b, _ = ora.fused_rope_forward(q2.reshape(30, 4, 16))
    assert np.array_equal(a, b.reshape(30, 64))


# Planted mistakes: each must break a pin used above.
def _interleaved(x, hd, theta):
    """GPT-J pairing (2j, 2j+1) instead of (j, j + half)."""
    y = P.rope_canonical(x, hd).astype(np.float64).copy()
    ang = P.rope_angles(y.shape[1], hd, theta)[None, :, None, :]
    a, b = y[..., 0:hd:2].copy(), y[..., 1:hd:2].copy()
    y[..., 0:hd:2] = a * np.cos(ang) - b * np.sin(ang)
    y[..., 1:hd:2] = a * np.sin(ang) + b * np.cos(ang)
    return y


def _variant(x, hd, theta, kind):
    xc = P.rope_canonical(x, hd).astype(np.float64)
    half = hd // 2
    j = np.arange(half, dtype=np.float64)
    if kind == "heads_as_positions":
        ang = np.arange(xc.shape[2])[None, None, :, None] * theta ** (-2.0 * j / hd)
    else:
        expo = (j / hd) if kind == "half_exponent" else (2.0 * j / hd)
        ang = (np.arange(xc.shape[1])[:, None] * theta ** (-expo))[None, :, None, :]
    c, s = np.cos(ang), np.sin(ang)
    if kind == "sign":
        s = -s
    if kind == "swap":
        c, s = s, c
    x1, x2 = xc[..., :half], xc[..., half:hd]
    return np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c, xc[..., hd:]], -1)


@pytest.mark.parametrize("kind", ["interleaved", "heads_as_positions", "half_exponent", "sign",
                                  "swap"])
def test_planted_mistakes_are_caught(kind):
    x = _x((2, 24, 4, 32), seed=7)
    xc = P.rope_canonical(x, 32)
    wrong = _interleaved(x, 32, 10000.0) if kind == "interleaved" else _variant(x, 32, 10000.0,
                                                                                 kind)
    with pytest.raises(AssertionError):
        P.assert_rope_close(wrong, P.rope_truth(xc, 32, 10000.0), xc, 32, 10000.0)
    with pytest.raises(AssertionError):
        P.assert_rope_close(wrong, _torch_rope(xc, 32, 10000.0), xc, 32, 10000.0)
