"""MX (OCP Microscaling) epilogue, CPU side: the oracle's E2M1 / E8M0 codecs and block
quantiser pinned against the reference's E2M1 table (include/velograd/kernels.h:47-51), torch's
float8_e8m0fnu values, exact float64 arithmetic and closed-form bounds; the device code's
helpers (velograd_amd/csrc/mx_formats.h, compiled here for the CPU) checked against the oracle."""

import ctypes
import math
import os
import shutil
import subprocess

import numpy as np
import pytest
import torch

from oracle import fused_rmsnorm as ora
from tests.test_fp8_codec import _dense_values

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)

# include/velograd/kernels.h:48-51, FP4_E2M1_TABLE, indexed by the nibble
REFERENCE_E2M1_TABLE = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                        -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]


@pytest.fixture(scope="module")
def check_lib(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    so = tmp_path_factory.mktemp("mx") / "fp8_check.so"
    subprocess.run(["g++", "-std=c++17", "-O2", "-shared", "-fPIC", "-I",
                    os.path.join(REPO, "velograd_amd", "csrc"), os.path.join(HERE, "fp8_check.cpp"),
                    "-o", str(so)], check=True, capture_output=True, text=True)
    lib = ctypes.CDLL(str(so))
    lib.vg_e2m1_encode_n.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
    lib.vg_mx_scale_n.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p,
                                  ctypes.c_void_p, ctypes.c_int64]
    return lib


def test_e2m1_decode_is_the_reference_table():
    got = ora.e2m1_decode(np.arange(16))
    for n in range(16):
        want = REFERENCE_E2M1_TABLE[n]
        assert got[n] == want and math.copysign(1, got[n]) == math.copysign(1, want), n


def test_e2m1_encode_is_the_nearest_value_with_ties_to_even():
    v = np.concatenate([_dense_values(), np.linspace(-8, 8, 100001, dtype=np.float32),
                        np.float32([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, -5.0, 7.0, 1e9])])
    codes = ora.e2m1_encode(v)
    got = np.abs(ora.e2m1_decode(codes).astype(np.float64))
    a = np.minimum(np.abs(v.astype(np.float64)), 6.0)
    dist = np.abs(got - a)
    # no other representable magnitude is closer (optimality against every table entry)
    for t in ora.E2M1_VALUES:
        assert np.all(dist <= np.abs(t - a))
    # at an exact midpoint the even code (mantissa bit 0) is chosen
    tie = np.isin(a, [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0])
    assert tie.any() and np.all((codes[tie] & 1) == 0)
    # the sign bit follows v, saturation at 6
    assert np.array_equal((codes >> 3) & 1, np.signbit(v).astype(np.uint8))
    assert np.all((codes[np.abs(v) >= 6] & 7) == 7)
    # round trip of every code
    assert np.array_equal(ora.e2m1_encode(ora.e2m1_decode(np.arange(16))), np.arange(16))


def test_e8m0_decode_matches_torch():
    codes = np.arange(255, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e8m0fnu).float().numpy().astype(np.float64)
    assert np.array_equal(ora.e8m0_decode(codes), want)
    assert np.isnan(ora.e8m0_decode(np.uint8(255)))


@pytest.mark.parametrize("fmt", ["e4m3", "e2m1"])
def test_mx_quantize_block_facts(fmt):
    rng = np.random.default_rng(1)
    y = (rng.standard_normal((16, 256)) * np.exp2(rng.integers(-30, 30, (16, 1)))).astype(np.float32)
    y[0, :32] = 0.0                                  # zero block
    y[1, 40] = np.nan                                # NaN block (block 1 of row 1)
    y[2, 64] = np.inf                                # Inf block
    codes, scales = ora.mx_quantize_rows(y, fmt)
    assert scales.shape == (16, 8) and codes.shape == (16, 256 if fmt == "e4m3" else 128)
    blocks = y.reshape(16, 8, 32).astype(np.float64)
    amax = np.max(np.abs(blocks), axis=-1)
    emax = ora.MX_EMAX[fmt]
    elem_max = 448.0 if fmt == "e4m3" else 6.0
    for r in range(16):
        for b in range(8):
            a = amax[r, b]
            if not np.isfinite(a):
                assert scales[r, b] == 0xFF
                continue
            if a == 0:
                assert scales[r, b] == 0
                continue
            s = int(scales[r, b]) - 127
            # the exact float64 exponent: 2^(s + emax) <= amax < 2^(s + emax + 1)
            assert 2.0 ** (s + emax) <= a < 2.0 ** (s + emax + 1), (r, b, a, s)
    deq = ora.mx_dequantize_rows(codes, scales, fmt).reshape(16, 8, 32)
    fin = np.isfinite(amax) & (amax > 0)
    x = 2.0 ** (scales.astype(np.float64) - 127)[..., None]
    v = np.abs(blocks) / x
    # half a unit in the last place of the element format at |v|, or the saturation gap
    if fmt == "e4m3":
        half = np.maximum(2.0 ** -10, np.exp2(np.floor(np.log2(np.maximum(v, 2.0 ** -6)))) * 2.0 ** -4)
    else:
        half = np.where(v < 2, 0.25, np.where(v < 4, 0.5, 1.0))
    bound = (np.maximum(half, v - elem_max) + 1e-12) * x
    err = np.abs(deq - blocks)
    assert np.all(err[fin] <= bound[fin])
    assert np.all(codes.reshape(16, -1)[1, (32 if fmt == "e4m3" else 16):(64 if fmt == "e4m3" else 32)] == 0)


def test_device_mx_helpers_match_oracle(check_lib):
    v = np.concatenate([_dense_values(), np.random.default_rng(2).integers(
        0, 2 ** 32, 1_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)])
    out = np.empty(v.shape, dtype=np.uint8)
    check_lib.vg_e2m1_encode_n(v.ctypes.data, out.ctypes.data, v.size)
    assert np.array_equal(out, ora.e2m1_encode(v))
    # scales: floor(log2) of normal and subnormal amax, zero, inf, NaN, both element formats
    a = np.abs(np.concatenate([v, np.float32([0.0, 1e-45, 1.1e-38, 3.4e38, np.inf, np.nan])]))
    for fmt, emax in ora.MX_EMAX.items():
        code = np.empty(a.shape, dtype=np.uint8)
        fac = np.empty(a.shape, dtype=np.float32)
        check_lib.vg_mx_scale_n(a.ctypes.data, emax, code.ctypes.data, fac.ctypes.data, a.size)
        # the oracle's scale of a block whose largest element is a
        blocks = np.zeros((a.size, 32), dtype=np.float32)
        blocks[:, 0] = a
        _, want = ora.mx_quantize_rows(blocks, fmt)
        assert np.array_equal(code, want[:, 0]), fmt
        fin = np.isfinite(a)
        assert np.array_equal(fac[fin].astype(np.float64),
                              2.0 ** (127 - code[fin].astype(np.float64))), fmt


def _ceil_scale(y, fmt):
    """Planted mistake: ceil(log2(amax)) instead of floor."""
    blocks = y.reshape(y.shape[0], -1, 32).astype(np.float64)
    amax = np.max(np.abs(blocks), axis=-1)
    return (np.ceil(np.log2(amax)) - ora.MX_EMAX[fmt] + 127).astype(np.uint8)


def test_planted_mistakes_are_caught():
    rng = np.random.default_rng(3)
    y = rng.standard_normal((8, 128)).astype(np.float32) * 5
    codes, scales = ora.mx_quantize_rows(y, "e2m1")
    # ceil instead of floor breaks the exponent bracket 2^(s+emax) <= amax < 2^(s+emax+1)
    bad = _ceil_scale(y, "e2m1")
    amax = np.max(np.abs(y.reshape(8, 4, 32)), axis=-1).astype(np.float64)
    s = bad.astype(np.float64) - 127
    assert not np.all((2.0 ** (s + 2) <= amax) & (amax < 2.0 ** (s + 3)))
    # swapped nibbles (odd element low) no longer dequantise to y within the bound
    swapped = ((codes >> 4) | (codes << 4)).astype(np.uint8)
    good = np.abs(ora.mx_dequantize_rows(codes, scales, "e2m1") - y).max()
    assert np.abs(ora.mx_dequantize_rows(swapped, scales, "e2m1") - y).max() > 4 * good
    # E2M1's emax (2) taken for E4M3 elements: every scale 2^6 too large
    c8, s8 = ora.mx_quantize_rows(y, "e4m3")
    wrong_scales = (s8.astype(np.int64) + 6).astype(np.uint8)
    assert np.abs(ora.mx_dequantize_rows(c8, wrong_scales, "e4m3") - y).max() > 10 * np.abs(
        ora.mx_dequantize_rows(c8, s8, "e4m3") - y).max()
