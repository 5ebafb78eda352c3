"""GPU parity of the fp8 output epilogue (velograd_rmsnorm_residual_fwd_fp8) against the oracle.

Parity bar: h bit-exact; inv_rms within the fp32 tolerance; and, given the device's inv_rms
(the only value whose rounding depends on a summation order), the e4m3 codes and the per-row
scales bit-exact, since every later step (y = (h * r) * w, amax, amax / 448, 1 / scale, the
product, the e4m3 rounding) is elementwise and exactly specified.  NaN codes are compared on
the NaN property only (the sign of y * NaN is the NaN operand's)."""

import numpy as np
import pytest
import torch

from oracle import fused_rmsnorm as ora
from tests import _parity as P
from velograd_amd import kernels as vk

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _codes(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.uint8).cpu().numpy()


def _check(x, res, w, eps, label):
    yq, sc, h, inv = vk.fused_rmsnorm_residual_forward_fp8(x, res, w, eps)
    assert yq.dtype == torch.float8_e4m3fn and yq.shape == x.shape
    assert sc.dtype == torch.float32 and sc.shape == x.shape[:-1] + (1,)
    x32 = P.upcast(x)
    r32 = P.upcast(res) if res is not None else None
    w32 = P.upcast(w) if w is not None else None
    _, rh, rinv = ora.fused_rmsnorm_residual_forward(x32, r32, w32, eps)
    if res is not None and h.dtype == torch.float32:
        assert np.array_equal(P.upcast(h), rh, equal_nan=True), f"{label} h"
    elif res is not None:
        P.assert_within_ulp(h, rh, 0, f"{label} h")
    else:
        assert h is x
    gi = P.upcast(inv)
    assert np.array_equal(np.isnan(gi), np.isnan(rinv)), label
    fin = ~np.isnan(rinv)
    assert P.rel_err(gi[fin], rinv[fin]) <= P.FP32_REL_TOL, label
    codes, scale, _, _ = ora.fused_rmsnorm_residual_forward_fp8(x32, r32, w32, eps,
                                                                inv_rms=P.upcast(inv))
    got_c, got_s = _codes(yq), P.upcast(sc)
    nan_ref = (codes & 0x7F) == 0x7F
    assert np.array_equal((got_c & 0x7F) == 0x7F, nan_ref), f"{label}: NaN codes differ"
    bad = np.nonzero((got_c != codes) & ~nan_ref)
    assert bad[0].size == 0, (f"{label}: {bad[0].size} codes differ", got_c[bad][:8],
                              codes[bad][:8])
    assert np.array_equal(got_s, scale, equal_nan=True), f"{label}: scales differ"
    return yq, sc, h, inv


CASES = [
    # (dtype, rows, dim, weight dtype or None, residual?) — vector paths, multi-wave rows,
    # the generic path (dims that are not whole 16-byte chunks) and decode shapes
    (torch.bfloat16, 16384, 4096, torch.bfloat16, True),
    (torch.bfloat16, 300, 4104, torch.float32, True),
    (torch.bfloat16, 7, 5120, torch.bfloat16, True),
    (torch.bfloat16, 5, 40000, torch.bfloat16, True),
    (torch.bfloat16, 33, 100, None, True),
    (torch.float16, 64, 768, torch.float16, False),
    (torch.float32, 512, 768, torch.float32, True),
    (torch.float32, 37, 13, torch.float32, True),
    (torch.float32, 3, 20000, None, False),
]


@pytest.mark.parametrize("dtype,rows,d,wdt,with_res", CASES,
                         ids=[f"{c[0]}-{c[1]}x{c[2]}-w{c[3]}-res{c[4]}".replace("torch.", "")
                              for c in CASES])
def test_fp8_epilogue_matches_oracle(dtype, rows, d, wdt, with_res):
    _say(f"fp8 {dtype} {rows}x{d} w={wdt} res={with_res}")
    rng = np.random.default_rng(rows * 7 + d)
    x = P.to_device(P.gaussian(rng, (rows, d)), dtype)
    res = P.to_device(P.gaussian(rng, (rows, d)), dtype) if with_res else None
    w = P.to_device(P.weight_vec(rng, d), wdt) if wdt is not None else None
    yq, sc, h, inv = _check(x, res, w, 1e-5, f"{dtype} {rows}x{d}")
    # h is the plain forward's; inv_rms agrees with it to a couple of ulps (the epilogue's plan
    # takes two chunks per thread where the plain forward takes one, so the row's sum of squares
    # is added in another order); y_fp8 * scale is y to e4m3 precision
    y, h2, inv2 = vk.fused_rmsnorm_residual_forward(x, res, w, 1e-5)
    assert P.rel_err(P.upcast(inv), P.upcast(inv2)) <= 2.0 ** -21
    if with_res:
        assert torch.equal(h, h2)
    deq = yq.cpu().float() * sc.cpu()
    yf = y.cpu().float()
    # half an e4m3 ulp (2^-4 relative) plus the rounding of the reference y to its dtype
    assert float((deq - yf).abs().max()) <= float((2.0 ** -4 + 2.0 ** -8) * yf.abs().max())


def test_fp8_leading_dims_strides_and_outliers():
    _say("fp8 [4,300,1024] strided x, outliers")
    rng = np.random.default_rng(11)
    base = P.with_outliers(rng, P.gaussian(rng, (4, 300, 2048), std=2.0))
    x = P.to_device(base, torch.bfloat16)[..., :1024]          # row stride 2048
    res = P.to_device(P.gaussian(rng, (4, 300, 1024)), torch.bfloat16)
    w = P.to_device(P.weight_vec(rng, 1024), torch.bfloat16)
    _check(x, res, w, 1e-5, "strided")


def test_fp8_special_rows():
    _say("fp8 special rows")
    d = 512
    rng = np.random.default_rng(12)
    x = P.gaussian(rng, (6, d))
    res = P.gaussian(rng, (6, d))
    x[0] = 0.0
    res[0] = 0.0              # zero row: scale 0, codes +0
    x[1] = 3.0
    res[1] = 0.0              # constant row, no weight: every y equal, all codes 448
    x[2, 17] = np.nan         # NaN row: NaN scale and codes
    x[3, :] *= 1e-3           # tiny row: scale from eps-dominated statistic
    res[3, :] *= 1e-3
    x[4, 5] = 1e4             # one huge element: everything else near zero / subnormal codes
    xd = P.to_device(x, torch.bfloat16)
    rd = P.to_device(res, torch.bfloat16)
    yq, sc, _, _ = _check(xd, rd, None, 1e-5, "special")
    s = P.upcast(sc)
    c = _codes(yq)
    assert s[0, 0] == 0.0 and np.all(c[0] == 0)
    assert np.all((c[1] & 0x7F) == 0x7E)
    assert np.isnan(s[2, 0]) and np.all((c[2] & 0x7F) == 0x7F)
    assert np.all(np.isfinite(s[3:]))


def test_fp8_empty_inputs():
    x = torch.empty(0, 64, device="cuda", dtype=torch.bfloat16)
    yq, sc, h, inv = vk.fused_rmsnorm_residual_forward_fp8(x, x.clone(), None)
    assert yq.shape == (0, 64) and sc.shape == (0, 1) and inv.shape == (0, 1)


def test_fp8_deterministic():
    rng = np.random.default_rng(13)
    x = P.to_device(P.gaussian(rng, (2048, 4096)), torch.bfloat16)
    r = P.to_device(P.gaussian(rng, (2048, 4096)), torch.bfloat16)
    a = vk.fused_rmsnorm_residual_forward_fp8(x, r, None, 1e-6)
    b = vk.fused_rmsnorm_residual_forward_fp8(x, r, None, 1e-6)
    for u, v in zip(a, b):
        assert torch.equal(u.view(torch.uint8) if u.dtype == torch.float8_e4m3fn else u,
                           v.view(torch.uint8) if v.dtype == torch.float8_e4m3fn else v)


@pytest.mark.parametrize("d", [16384, 16383], ids=["vector-path", "generic-path"])
def test_fp8_encoder_on_dense_values(d):
    """The device encoder on every e4m3 value, midpoint (and its float32 neighbours), rounding
    boundary pattern and a random spread, through the product kernel: fp32 rows of ones with
    eps = 0 give inv_rms = 1 exactly, so y = weight; with 448 in the weight the scale is 1 and the
    codes are e4m3(weight) themselves."""
    from tests.test_fp8_codec import _dense_values

    v = _dense_values()
    v = v[np.abs(v) <= 448.0]
    per = d - 1
    chunks = [v[i:i + per] for i in range(0, v.size, per)]
    _say(f"fp8 dense values: {v.size} values, {len(chunks)} calls, dim {d}")
    x = torch.ones(1, d, device="cuda", dtype=torch.float32)
    for c in chunks:
        w = np.zeros(d, dtype=np.float32)
        w[:c.size] = c
        w[-1] = 448.0
        yq, sc, _, inv = vk.fused_rmsnorm_residual_forward_fp8(x, None, P.to_device(w, torch.float32),
                                                               0.0)
        assert float(inv[0, 0]) == 1.0 and float(sc[0, 0]) == 1.0
        got = _codes(yq)[0]
        want = ora.e4m3fn_encode(w)
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, (w[bad[:8]], got[bad[:8]], want[bad[:8]])
