"""Pins the oracle of the reference model's RoPE, `apply_rotary_emb` (python/velograd/functional.py:
287-345; interleaved pairs over the last axis, positions along axis -2), before the GPU kernel is
compared with it.

Independent checks: torch's complex arithmetic (each pair as a complex number times
e^{i·pos·theta}, theta = base^(-2i/dim)) in float64; position 0 is the identity; pair norms are
kept; the inverse rotation undoes the forward and is its adjoint (the reference's backward rule,
functional.py:333-337, ops.rs:501-530); dot products depend only on the position difference.
Planted mistakes (rotate-half pairing, positions on the wrong axis, exponent i/dim instead of
2i/dim, the sign of the inverse) are shown to fail them."""

import numpy as np
import pytest
import torch

from oracle import fused_rmsnorm as ora


def _complex_truth(x: np.ndarray, base: float) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float64))
    seq, dim = t.shape[-2], t.shape[-1]
    z = torch.view_as_complex(t.reshape(*t.shape[:-1], dim // 2, 2).contiguous())
    inv_freq = base ** (-torch.arange(0, dim, 2, dtype=torch.float64) / dim)
    ang = torch.arange(seq, dtype=torch.float64)[:, None] * inv_freq[None, :]
    rot = z * torch.polar(torch.ones_like(ang), ang)
    return torch.view_as_real(rot).reshape(t.shape).numpy()


def _failures(fn):
    """Names of the checks `fn(x, base, inverse)` fails (empty = all pass)."""
    bad = []
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 37, 64))
    y = fn(x, 10000.0, False)
    if np.max(np.abs(y - _complex_truth(x, 10000.0))) > 1e-12:
        bad.append("complex truth")
    y2 = fn(x[:, :5, :10], 500.0, False)
    if np.max(np.abs(y2 - _complex_truth(x[:, :5, :10], 500.0))) > 1e-12:
        bad.append("complex truth small")
    if not np.array_equal(y[:, 0], x[:, 0]):
        bad.append("position 0")
    n_in = x[..., 0::2] ** 2 + x[..., 1::2] ** 2
    n_out = y[..., 0::2] ** 2 + y[..., 1::2] ** 2
    if np.max(np.abs(n_in - n_out)) > 1e-12:
        bad.append("pair norms")
    back = fn(y, 10000.0, True)
    if np.max(np.abs(back - x)) > 1e-12:
        bad.append("inverse")
    g = rng.standard_normal(x.shape)
    if abs(np.sum(fn(g, 10000.0, True) * x) - np.sum(g * y)) > 1e-9:
        bad.append("adjoint")
    # <R_m q, R_n k> depends on m - n only: rotate the same q, k at positions (m, n) = (5, 2)
    # and (33, 30)
    q = rng.standard_normal(64)
    k = rng.standard_normal(64)
    qs = np.tile(q, (37, 1))[None]
    ks = np.tile(k, (37, 1))[None]
    rq, rk = fn(qs, 10000.0, False)[0], fn(ks, 10000.0, False)[0]
    if abs(rq[5] @ rk[2] - rq[33] @ rk[30]) > 1e-9:
        bad.append("relative position")
    return bad


def test_oracle_passes_every_check():
    assert _failures(ora.apply_rotary_emb) == []


def test_reference_theta_formula_at_a_point():
    # functional.py:302-303 at i = 3, dim = 16, pos = 7: angle = 7 / 10000^(6/16)
    x = np.zeros((8, 16))
    x[7, 6] = 1.0                      # pair i = 3, first element
    y = ora.apply_rotary_emb(x, 10000.0)
    ang = 7.0 / (10000.0 ** (6.0 / 16.0))
    assert abs(y[7, 6] - np.cos(ang)) < 1e-15 and abs(y[7, 7] - np.sin(ang)) < 1e-15
    assert np.count_nonzero(y) == 2


def _rotate_half(x, base, inverse):
    x = np.asarray(x, np.float64)
    dim = x.shape[-1]
    h = dim // 2
    theta = 1.0 / base ** (2.0 * np.arange(h) / dim)
    ang = np.arange(x.shape[-2])[:, None] * theta
    c, s = np.cos(ang), np.sin(ang) * (-1 if inverse else 1)
    a, b = x[..., :h], x[..., h:]
    return np.concatenate([a * c - b * s, a * s + b * c], axis=-1)


def _positions_on_axis_minus3(x, base, inverse):
    x = np.asarray(x, np.float64)
    sw = np.swapaxes(x, -2, -3) if x.ndim >= 3 else x
    out = ora.apply_rotary_emb(sw, base, inverse)
    return np.swapaxes(out, -2, -3) if x.ndim >= 3 else out


def _exponent_i_over_dim(x, base, inverse):
    x = np.asarray(x, np.float64)
    dim = x.shape[-1]
    theta = 1.0 / base ** (np.arange(dim // 2) / dim)
    ang = np.arange(x.shape[-2])[:, None] * theta
    c, s = np.cos(ang), np.sin(ang) * (-1 if inverse else 1)
    out = np.empty_like(x)
    out[..., 0::2] = x[..., 0::2] * c - x[..., 1::2] * s
    out[..., 1::2] = x[..., 0::2] * s + x[..., 1::2] * c
    return out


def _inverse_not_negated(x, base, inverse):
    return ora.apply_rotary_emb(x, base, False)


@pytest.mark.parametrize("mistake,caught_by", [
    (_rotate_half, "complex truth"),
    (_positions_on_axis_minus3, "complex truth"),
    (_exponent_i_over_dim, "complex truth"),
    (_inverse_not_negated, "inverse"),
])
def test_planted_mistakes_are_caught(mistake, caught_by):
    assert caught_by in _failures(mistake)


def test_positions_argument_matches_rows_of_the_whole_sequence():
    """Rows taken out of a sequence, rotated with their own positions, equal the same rows of the
    whole sequence rotated (forward and inverse)."""
    rng = np.random.default_rng(4)
    x = rng.standard_normal((2, 300, 64))
    rows = np.array([0, 1, 7, 150, 298, 299])
    for inverse in (False, True):
        whole = ora.apply_rotary_emb(x, 500000.0, inverse=inverse)
        part = ora.apply_rotary_emb(x[:, rows], 500000.0, inverse=inverse, positions=rows)
        assert np.array_equal(part, whole[:, rows])
