"""GPU parity of the MX epilogue (velograd_rmsnorm_residual_fwd_mx) against the oracle.

Parity bar as for the per-row fp8 epilogue: h bit-exact, inv_rms within the fp32 tolerance,
and, given the device's inv_rms, the element codes and the E8M0 scale codes bit-exact (every
later step is elementwise or an order-independent maximum)."""

import numpy as np
import pytest
import torch

from oracle import fused_rmsnorm as ora
from tests import _parity as P
from velograd_amd import kernels as vk

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _check(x, res, w, eps, fmt, label):
    yq, sc, h, inv = vk.fused_rmsnorm_residual_forward_mx(x, res, w, eps, fmt=fmt)
    d = x.shape[-1]
    assert sc.dtype == torch.float8_e8m0fnu and sc.shape == x.shape[:-1] + (d // 32,)
    if fmt == "e4m3":
        assert yq.dtype == torch.float8_e4m3fn and yq.shape == x.shape
    else:
        assert yq.dtype == torch.float4_e2m1fn_x2 and yq.shape == x.shape[:-1] + (d // 2,)
    x32 = P.upcast(x)
    r32 = P.upcast(res) if res is not None else None
    w32 = P.upcast(w) if w is not None else None
    _, rh, rinv = ora.fused_rmsnorm_residual_forward(x32, r32, w32, eps)
    if res is not None:
        if h.dtype == torch.float32:
            assert np.array_equal(P.upcast(h), rh, equal_nan=True), label
        else:
            P.assert_within_ulp(h, rh, 0, f"{label} h")
    gi = P.upcast(inv)
    assert np.array_equal(np.isnan(gi), np.isnan(rinv)), label
    fin = ~np.isnan(rinv)
    assert P.rel_err(gi[fin], rinv[fin]) <= P.FP32_REL_TOL, label
    codes, scales, _, _ = ora.fused_rmsnorm_residual_forward_mx(x32, r32, w32, eps, fmt=fmt,
                                                                inv_rms=gi)
    got_c = yq.view(torch.uint8).cpu().numpy()
    got_s = sc.view(torch.uint8).cpu().numpy()
    bad = np.nonzero(got_s != scales)
    assert bad[0].size == 0, (f"{label}: {bad[0].size} scales differ", got_s[bad][:8],
                              scales[bad][:8])
    bad = np.nonzero(got_c != codes)
    assert bad[0].size == 0, (f"{label}: {bad[0].size} code bytes differ", got_c[bad][:8],
                              codes[bad][:8])
    return yq, sc


CASES = [
    # (dtype, rows, dim, weight dtype or None, residual?): 4 lanes per block (bf16/fp16),
    # 8 lanes per block (fp32), multi-wave rows, decode rows, the generic path
    (torch.bfloat16, 4096, 4096, torch.bfloat16, True),
    (torch.bfloat16, 7, 5120, torch.float32, True),
    (torch.float16, 64, 768, torch.float16, False),
    (torch.float32, 512, 768, torch.float32, True),
    (torch.float32, 33, 2048, None, True),
    (torch.bfloat16, 3, 40032, torch.bfloat16, True),    # past the register path: generic
]


@pytest.mark.parametrize("fmt", ["e4m3", "e2m1"])
@pytest.mark.parametrize("dtype,rows,d,wdt,with_res", CASES,
                         ids=[f"{c[0]}-{c[1]}x{c[2]}".replace("torch.", "") for c in CASES])
def test_mx_epilogue_matches_oracle(dtype, rows, d, wdt, with_res, fmt):
    _say(f"mx {fmt} {dtype} {rows}x{d}")
    rng = np.random.default_rng(rows + d)
    x = P.to_device(P.gaussian(rng, (rows, d)), dtype)
    res = P.to_device(P.gaussian(rng, (rows, d)), dtype) if with_res else None
    w = P.to_device(P.weight_vec(rng, d), wdt) if wdt is not None else None
    _check(x, res, w, 1e-5, fmt, f"{fmt} {dtype} {rows}x{d}")


@pytest.mark.parametrize("fmt", ["e4m3", "e2m1"])
def test_mx_special_blocks_and_outliers(fmt):
    _say(f"mx {fmt} special blocks")
    d = 256
    rng = np.random.default_rng(7)
    x = P.with_outliers(rng, P.gaussian(rng, (6, d), std=2.0))
    res = P.gaussian(rng, (6, d))
    x[0] = 0.0
    res[0] = 0.0                   # zero row: every block scale code 0, codes +0
    x[1, 100] = np.nan             # NaN row: every block 0xFF
    x[2, :32] *= 1e-4              # one tiny block among normal ones
    res[2, :32] *= 1e-4
    xd = P.to_device(x, torch.bfloat16)
    rd = P.to_device(res, torch.bfloat16)
    w = np.ones(d, dtype=np.float32)
    w[200] = np.inf                # an infinite weight: the block holding column 200 is 0xFF
    wd = P.to_device(w, torch.float32)
    yq, sc = _check(xd, rd, wd, 1e-5, fmt, f"{fmt} special")
    s = sc.view(torch.uint8).cpu().numpy()
    blk = 200 // 32                # 0 * inf is NaN even in the zero row
    assert np.all(np.delete(s[0], blk) == 0) and s[0, blk] == 0xFF
    assert np.all(s[1] == 0xFF) and np.all(s[2:, blk] == 0xFF)


def test_mx_strided_and_leading_dims():
    _say("mx strided")
    rng = np.random.default_rng(8)
    base = P.gaussian(rng, (2, 50, 1024))
    x = P.to_device(base, torch.bfloat16)[..., :512]       # row stride 1024
    res = P.to_device(P.gaussian(rng, (2, 50, 512)), torch.bfloat16)
    w = P.to_device(P.weight_vec(rng, 512), torch.bfloat16)
    for fmt in ("e4m3", "e2m1"):
        _check(x, res, w, 1e-6, fmt, f"strided {fmt}")


def test_mx_rejects_dims_off_the_block():
    x = torch.zeros(2, 48, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        vk.fused_rmsnorm_residual_forward_mx(x, None, None)
    with pytest.raises(ValueError):
        vk.fused_rmsnorm_residual_forward_mx(torch.zeros(2, 64, device="cuda"), fmt="e5m2")


@pytest.mark.parametrize("fmt,top", [("e4m3", 300.0), ("e2m1", 7.0)])
@pytest.mark.parametrize("d", [16384, 16416], ids=["vector-path", "generic-path"])
def test_mx_element_encoder_on_dense_values(fmt, top, d):
    """The device's element conversion on a dense set of values through the product kernel:
    fp32 rows of ones with eps = 0 give inv_rms = 1, so y = weight; every 32-element block holds
    one value `top` whose exponent makes the block factor 2^0, and 31 test values."""
    from tests.test_fp8_codec import _dense_values

    lim = 448.0 if fmt == "e4m3" else 7.5
    v = _dense_values()
    v = np.concatenate([v[np.abs(v) <= min(lim, top)],
                        np.linspace(-top, top, 20001, dtype=np.float32)])
    per_row = (d // 32) * 31
    _say(f"mx {fmt} dense values: {v.size} values, dim {d}")
    x = torch.ones(1, d, device="cuda", dtype=torch.float32)
    for i in range(0, v.size, per_row):
        chunk = v[i:i + per_row]
        w = np.zeros((d // 32, 32), dtype=np.float32)
        w[:, 0] = top
        flat = w[:, 1:].reshape(-1)
        flat[:chunk.size] = chunk
        w[:, 1:] = flat.reshape(d // 32, 31)
        w = w.reshape(-1)
        yq, sc, _, inv = vk.fused_rmsnorm_residual_forward_mx(
            x, None, P.to_device(w, torch.float32), 0.0, fmt=fmt)
        assert float(inv[0, 0]) == 1.0
        assert np.all(sc.view(torch.uint8).cpu().numpy() == 127)
        codes, _ = ora.mx_quantize_rows(w[None, :], fmt)
        got = yq.view(torch.uint8).cpu().numpy()
        bad = np.nonzero(got != codes)
        assert bad[1].size == 0, (fmt, got[bad][:8], codes[bad][:8])
