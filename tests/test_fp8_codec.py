"""fp8 E4M3 epilogue, CPU side: the oracle's codec and per-row quantiser pinned against torch's
float8_e4m3fn casts, the reference's decoder and closed-form bounds; the device code's encoder
(velograd_amd/csrc/fp8_e4m3.h, compiled here for the CPU) checked against the oracle."""

import ctypes
import os
import shutil
import subprocess

import numpy as np
import pytest
import torch

from oracle import fused_rmsnorm as ora

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)


def _torch_cast(v: np.ndarray) -> np.ndarray:
    """torch's float32 -> float8_e4m3fn cast (round to nearest even) after clamping to +-448:
    torch maps values beyond the format to NaN, the clamp gives saturation."""
    t = torch.from_numpy(np.ascontiguousarray(v, dtype=np.float32))
    return t.clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def _dense_values() -> np.ndarray:
    """Every representable value, every midpoint and its float32 neighbours, all binades with the
    rounding-boundary bit patterns, random values at several scales and the special values."""
    tab = ora._E4M3_TABLE
    mids = ((tab[1:] + tab[:-1]) / 2).astype(np.float32)
    parts = [tab.astype(np.float32), mids, np.nextafter(mids, np.float32(0)),
             np.nextafter(mids, np.float32(np.inf))]
    # normal binades 2^-12 .. 2^9, each top-3-mantissa value, dropped bits around the half point
    exps = np.arange(115, 137, dtype=np.uint32)
    top = np.arange(8, dtype=np.uint32)
    low = np.array([0, 1, 0x7FFFF, 0x80000, 0x80001, 0xFFFFF, 0x40000, 0xC0000], dtype=np.uint32)
    bits = (exps[:, None, None] << 23) | (top[None, :, None] << 20) | low[None, None, :]
    parts.append(bits.reshape(-1).view(np.float32))
    rng = np.random.default_rng(0)
    for s in (1e-4, 1e-3, 1e-2, 0.1, 1.0, 10.0, 100.0, 300.0):
        parts.append((rng.standard_normal(20000) * s).astype(np.float32))
    parts.append(np.float32([0.0, 2.0 ** -10, 3 * 2.0 ** -11, 1e-30, 1e-45, 447.9, 448.0,
                             448.1, 463.9, 464.0, 464.1, 479.0, 480.0, 500.0, 1e9, 3e38]))
    v = np.concatenate(parts)
    return np.concatenate([v, -v])


def test_decode_matches_torch_for_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(ora.e4m3fn_decode(codes), want, equal_nan=True)


def test_decode_matches_reference_decoder_values():
    # include/velograd/kernels.h:58-73: subnormal (m/8) * 2^-6, normal 2^(e-7) * (1 + m/8);
    # it returns 0 for 0x7F/0xFF where the format (and this oracle) has NaN.
    for c in range(256):
        s, e, m = c >> 7, (c >> 3) & 0xF, c & 7
        if c in (0x7F, 0xFF):
            assert np.isnan(ora.e4m3fn_decode(np.uint8(c)))
            continue
        mag = (m / 8.0) * 0.015625 if e == 0 else np.ldexp(1.0 + m / 8.0, e - 7)
        assert float(ora.e4m3fn_decode(np.uint8(c))) == (-mag if s else mag), hex(c)
    assert float(ora.e4m3fn_decode(np.uint8(0x7E))) == 448.0


def test_encode_matches_torch_cast():
    v = _dense_values()
    got, want = ora.e4m3fn_encode(v), _torch_cast(v)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, (v[bad[:5]], got[bad[:5]], want[bad[:5]])
    # the special values explicitly: saturation, signed NaN, signed zero
    sp = np.float32([np.inf, -np.inf, np.nan, -np.nan, 0.0, -0.0])
    assert list(ora.e4m3fn_encode(sp)) == [0x7E, 0xFE, 0x7F, 0xFF, 0x00, 0x80]


def test_encode_decode_round_trip_and_rounding_bound():
    codes = np.array([c for c in range(256) if c & 0x7F != 0x7F], dtype=np.uint8)
    assert np.array_equal(ora.e4m3fn_encode(ora.e4m3fn_decode(codes)), codes)
    v = _dense_values()
    v = v[np.abs(v) <= 448]
    err = np.abs(ora.e4m3fn_decode(ora.e4m3fn_encode(v)).astype(np.float64) - v)
    # half a unit in the last place: 2^-10 absolute below 2^-6, 2^-4 relative above
    bound = np.maximum(2.0 ** -10, np.exp2(np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -6))))
                       * 2.0 ** -4)
    assert np.all(err <= bound)


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_device_encoder_matches_oracle(tmp_path):
    so = tmp_path / "fp8_check.so"
    subprocess.run(["g++", "-std=c++17", "-O2", "-shared", "-fPIC", "-I",
                    os.path.join(REPO, "velograd_amd", "csrc"), os.path.join(HERE, "fp8_check.cpp"),
                    "-o", str(so)], check=True, capture_output=True, text=True)
    lib = ctypes.CDLL(str(so))
    lib.vg_e4m3_encode_n.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
    lib.vg_e4m3_quantize_n.argtypes = [ctypes.c_void_p, ctypes.c_float, ctypes.c_void_p,
                                       ctypes.c_int64]
    rng = np.random.default_rng(1)
    v = np.concatenate([_dense_values(), rng.integers(0, 2 ** 32, 2_000_000, dtype=np.uint64)
                        .astype(np.uint32).view(np.float32),
                        np.float32([np.inf, -np.inf, np.nan, -np.nan, 0.0, -0.0])])
    out = np.empty(v.shape, dtype=np.uint8)
    lib.vg_e4m3_encode_n(v.ctypes.data, out.ctypes.data, v.size)
    want = ora.e4m3fn_encode(v)
    bad = np.nonzero(out != want)[0]
    assert bad.size == 0, (v[bad[:5]], out[bad[:5]], want[bad[:5]])
    # per-element quantisation with a row scale, and the zero-scale rule
    y = (rng.standard_normal(100000) * 3).astype(np.float32)
    y[:3] = [0.0, -0.0, 1e-3]
    codes, scale = ora.quantize_rows_e4m3(y)
    lib.vg_e4m3_quantize_n(y.ctypes.data, float(scale[0]), out.ctypes.data, y.size)
    assert np.array_equal(out[:y.size], codes)
    z = np.float32([0.0, -0.0, 0.0])
    zc, zs = ora.quantize_rows_e4m3(z)
    lib.vg_e4m3_quantize_n(z.ctypes.data, 0.0, out.ctypes.data, 3)
    assert float(zs[0]) == 0.0 and list(zc) == [0x00, 0x80, 0x00] and list(out[:3]) == list(zc)


def _quantizer_pins(y, codes, scale) -> bool:
    """Closed-form facts every per-row e4m3 quantisation of y must satisfy."""
    amax = np.max(np.abs(y), axis=-1, keepdims=True)
    if not np.array_equal(scale, (amax / np.float32(448)).astype(np.float32)):
        return False
    # the row's largest element lands on +-448 (y / scale = 448 up to one rounding)
    j = np.argmax(np.abs(y), axis=-1)
    if not np.all((np.take_along_axis(codes, j[..., None], -1) & 0x7F) == 0x7E):
        return False
    # the library form of the same quantisation, torch's (y * (1 / scale)).clamp(+-448) cast
    ty = torch.from_numpy(y)
    tinv = torch.from_numpy(scale).reciprocal()
    if not np.array_equal(codes, _torch_cast((ty * tinv).numpy())):
        return False
    # dequantisation error: half an e4m3 ulp of y / scale, plus the roundings of 1 / scale and
    # of the product (2 float32 ulps), times the scale
    deq = ora.e4m3fn_decode(codes).astype(np.float64) * scale
    v = np.abs(y.astype(np.float64) / scale)
    half_ulp = np.maximum(2.0 ** -10,
                          np.exp2(np.floor(np.log2(np.maximum(v, 2.0 ** -6)))) * 2.0 ** -4)
    return bool(np.all(np.abs(deq - y) <= (half_ulp + 2.0 ** -22 * v) * scale))


def _rows(seed=2):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((64, 1000)) * rng.uniform(1e-3, 1e3, (64, 1))).astype(np.float32)


def test_quantize_rows_properties():
    y = _rows()
    codes, scale = ora.quantize_rows_e4m3(y)
    assert scale.shape == (64, 1) and scale.dtype == np.float32
    assert _quantizer_pins(y, codes, scale)
    # zero row: scale 0, signed zero codes; NaN row: NaN scale and NaN codes
    zc, zs = ora.quantize_rows_e4m3(np.float32([[0.0, -0.0, 0.0]]))
    assert zs[0, 0] == 0 and list(zc[0]) == [0x00, 0x80, 0x00]
    nc, ns = ora.quantize_rows_e4m3(np.float32([[1.0, np.nan, -2.0]]))
    # (NaN sign is not meaningful: y / NaN takes the NaN operand's sign)
    assert np.isnan(ns[0, 0]) and np.all((nc[0] & 0x7F) == 0x7F)


def test_forward_fp8_given_statistic_reproduces_forward():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((16, 256)).astype(np.float32)
    r = rng.standard_normal((16, 256)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(256)).astype(np.float32)
    y, h, inv = ora.fused_rmsnorm_residual_forward(x, r, w, 1e-5)
    codes, scale, h2, inv2 = ora.fused_rmsnorm_residual_forward_fp8(x, r, w, 1e-5)
    assert np.array_equal(h, h2) and np.array_equal(inv, inv2)
    assert (codes, scale)[0].shape == y.shape
    c3, s3 = ora.quantize_rows_e4m3(y)
    assert np.array_equal(codes, c3) and np.array_equal(scale, s3)
    # a given statistic is used as is
    c4, s4, _, inv4 = ora.fused_rmsnorm_residual_forward_fp8(x, r, w, 1e-5, inv_rms=inv * 2)
    c5, s5 = ora.quantize_rows_e4m3((h * (inv * 2)) * w)
    assert np.array_equal(c4, c5) and np.array_equal(s4, s5)


def _truncating_encode(v):
    """Planted mistake: truncation toward zero instead of round-to-nearest-even."""
    v = np.asarray(v, dtype=np.float32)
    a = np.minimum(np.abs(v).astype(np.float64), 448.0)
    code = np.searchsorted(ora._E4M3_TABLE, a, side="right") - 1
    return (code | (np.signbit(v).astype(np.int64) << 7)).astype(np.uint8)


def _fnuz_decode(codes):
    """Planted mistake: the bias-8 "fnuz" variant (MI300's fp8), not OCP e4m3fn."""
    return (ora.e4m3fn_decode(codes).astype(np.float64) / 2).astype(np.float32)


def test_planted_mistakes_are_caught():
    v = _dense_values()
    assert not np.array_equal(_truncating_encode(v), _torch_cast(v))
    codes = np.arange(0x7F, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert not np.array_equal(_fnuz_decode(codes), want)
    y = _rows(4)
    amax = np.max(np.abs(y), axis=-1, keepdims=True)
    good = (amax / np.float32(448)).astype(np.float32)
    # truncating instead of rounding
    inv = (np.float32(1) / good).astype(np.float32)
    assert _quantizer_pins(y, ora.e4m3fn_encode(y * inv), good)
    assert not _quantizer_pins(y, _truncating_encode(y * inv), good)
    # the scale of the fnuz format (largest finite 240)
    s240 = (amax / np.float32(240)).astype(np.float32)
    assert not _quantizer_pins(y, ora.e4m3fn_encode(y / s240), s240)
    # the scale from the un-weighted h although y = h * w
    w = np.random.default_rng(5).uniform(0.5, 2.0, y.shape[-1]).astype(np.float32)
    yw = y * w
    assert not _quantizer_pins(yw, ora.e4m3fn_encode(yw * inv), good)
