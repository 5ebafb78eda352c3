"""The C ABI library: it loads, exports exactly what include/velograd_kernels.h declares, and
rejects bad arguments on the host before any HIP call (no GPU needed)."""

import ctypes
import os
import re

import pytest
import torch

from velograd_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "velograd_kernels.h")


def declared_functions():
    with open(HEADER) as f:
        text = f.read()
    return re.findall(r"VELOGRAD_API\s+[\w\s\*]+?\b(velograd_\w+)\s*\(", text)


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        from velograd_amd.build import build_library
        build_library()
    return _lib.load()


def test_header_declares_the_bound_functions():
    names = declared_functions()
    assert len(names) == len(set(names))
    assert set(names) == set(_lib.SIGNATURES), (names, sorted(_lib.SIGNATURES))


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name
    # and nothing but the ABI is visible (-fvisibility=hidden)
    out = os.popen(f"nm -D --defined-only {_lib.LIB_PATH}").read()
    exported = set(re.findall(r"\b[TW] (velograd_\w+)", out))
    assert exported == set(declared_functions())


def test_version_string(lib):
    v = lib.velograd_kernels_version().decode()
    assert "gfx950" in v and "velograd_amd" in v


def _fwd(lib, **kw):
    args = dict(x=16, residual=None, weight=None, y=32, h=None, inv_rms=None, rows=4, dim=64,
                ld_x=64, ld_res=64, ld_y=64, ld_h=64, dtype=2, w_dtype=2, eps=1e-5, stream=None)
    args.update(kw)
    return lib.velograd_rmsnorm_residual_fwd(*args.values())


def _bwd(lib, **kw):
    args = dict(g=16, saved=48, saved_is_h=0, weight=None, inv_rms=80, grad_h=None, dx=32,
                dres=None, dweight=None, ws=None, ws_bytes=0, rows=4, dim=64, ld_g=64, ld_s=64,
                ld_gh=64, ld_dx=64, ld_dres=64, dtype=2, w_dtype=2, stream=None)
    args.update(kw)
    return lib.velograd_rmsnorm_residual_bwd(*args.values())


# Every case below returns before the library touches the HIP runtime (the pointers are dummies
# that are never dereferenced), so it runs on a host without a GPU.
@pytest.mark.parametrize("kw,code,msg", [
    (dict(dtype=7), _lib.ERR_UNSUPPORTED_DTYPE, "unsupported dtype"),
    (dict(dtype=0, w_dtype=2), _lib.ERR_UNSUPPORTED_DTYPE, "unsupported dtype"),
    (dict(dim=0), _lib.ERR_INVALID_ARGUMENT, "invalid shape"),
    (dict(rows=-1), _lib.ERR_INVALID_ARGUMENT, "invalid shape"),
    (dict(x=None), _lib.ERR_INVALID_ARGUMENT, "must not be NULL"),
    (dict(y=None), _lib.ERR_INVALID_ARGUMENT, "must not be NULL"),
    (dict(ld_x=63), _lib.ERR_INVALID_ARGUMENT, "row strides"),
    (dict(y=16), _lib.ERR_INVALID_ARGUMENT, "alias"),
    (dict(residual=64, h=64), _lib.ERR_INVALID_ARGUMENT, "alias"),
])
def test_fwd_argument_errors(lib, kw, code, msg):
    assert _fwd(lib, **kw) == code
    assert msg in _lib.last_error()


def test_fwd_zero_rows_is_a_no_op(lib):
    assert _fwd(lib, rows=0, x=None, y=None) == 0
    assert _lib.last_error() == ""


def _rmsnorm_fwd(lib, **kw):
    args = dict(x=16, residual=None, weight=None, y=32, h=None, inv_rms=None, rows=4, dim=64,
                ld_x=64, ld_res=64, ld_y=64, ld_h=64, dtype=2, w_dtype=2, eps=1e-6,
                min_mean_sq=1e-12, stream=None)
    args.update(kw)
    return lib.velograd_rmsnorm_fwd(*args.values())


@pytest.mark.parametrize("kw,code,msg", [
    (dict(min_mean_sq=-1e-12), _lib.ERR_INVALID_ARGUMENT, "min_mean_sq"),
    (dict(min_mean_sq=float("nan")), _lib.ERR_INVALID_ARGUMENT, "min_mean_sq"),
    (dict(min_mean_sq=float("inf")), _lib.ERR_INVALID_ARGUMENT, "min_mean_sq"),
    (dict(dtype=7), _lib.ERR_UNSUPPORTED_DTYPE, "unsupported dtype"),
    (dict(dim=0), _lib.ERR_INVALID_ARGUMENT, "invalid shape"),
    (dict(x=None), _lib.ERR_INVALID_ARGUMENT, "must not be NULL"),
    (dict(ld_y=63), _lib.ERR_INVALID_ARGUMENT, "row strides"),
    (dict(y=16), _lib.ERR_INVALID_ARGUMENT, "alias"),
    (dict(residual=48, h=48), _lib.ERR_INVALID_ARGUMENT, "alias"),
    (dict(residual=48, h=80, ld_res=32), _lib.ERR_INVALID_ARGUMENT, "row strides"),
])
def test_rmsnorm_fwd_argument_errors(lib, kw, code, msg):
    assert _rmsnorm_fwd(lib, **kw) == code
    assert msg in _lib.last_error() and "velograd_rmsnorm_fwd" in _lib.last_error()


def test_rmsnorm_fwd_zero_rows_is_a_no_op(lib):
    assert _rmsnorm_fwd(lib, rows=0, x=None, y=None) == 0
    assert _lib.last_error() == ""


def _rmsnorm_rope_fwd(lib, **kw):
    args = dict(x=16, residual=None, weight=None, y=32, h=None, inv_rms=None, rows=4, dim=64,
                ld_x=64, ld_res=64, ld_y=64, ld_h=64, seq=2, dtype=2, w_dtype=2, eps=1e-6,
                min_mean_sq=1e-12, base=10000.0, stream=None)
    args.update(kw)
    return lib.velograd_rmsnorm_rope_fwd(*args.values())


@pytest.mark.parametrize("kw,code,msg", [
    (dict(dim=63, ld_x=63, ld_y=63), _lib.ERR_INVALID_ARGUMENT, "even dim"),
    (dict(seq=0), _lib.ERR_INVALID_ARGUMENT, "seq >= 1"),
    (dict(seq=3), _lib.ERR_INVALID_ARGUMENT, "dividing rows"),
    (dict(base=0.0), _lib.ERR_INVALID_ARGUMENT, "base"),
    (dict(base=float("nan")), _lib.ERR_INVALID_ARGUMENT, "base"),
    (dict(min_mean_sq=-1.0), _lib.ERR_INVALID_ARGUMENT, "min_mean_sq"),
    (dict(y=16), _lib.ERR_INVALID_ARGUMENT, "alias"),
    (dict(dtype=7), _lib.ERR_UNSUPPORTED_DTYPE, "unsupported dtype"),
])
def test_rmsnorm_rope_fwd_argument_errors(lib, kw, code, msg):
    assert _rmsnorm_rope_fwd(lib, **kw) == code
    assert msg in _lib.last_error() and "velograd_rmsnorm_rope_fwd" in _lib.last_error()


def _fwd_fp8(lib, **kw):
    args = dict(x=16, residual=None, weight=None, y=32, y_scale=112, h=None, inv_rms=None,
                rows=4, dim=64, ld_x=64, ld_res=64, ld_y=64, ld_h=64, dtype=2, w_dtype=2,
                eps=1e-5, stream=None)
    args.update(kw)
    return lib.velograd_rmsnorm_residual_fwd_fp8(*args.values())


@pytest.mark.parametrize("kw,code,msg", [
    (dict(dtype=9), _lib.ERR_UNSUPPORTED_DTYPE, "unsupported dtype"),
    (dict(y_scale=None), _lib.ERR_INVALID_ARGUMENT, "y_scale must not be NULL"),
    (dict(dim=0), _lib.ERR_INVALID_ARGUMENT, "invalid shape"),
    (dict(y=None), _lib.ERR_INVALID_ARGUMENT, "must not be NULL"),
    (dict(ld_y=32), _lib.ERR_INVALID_ARGUMENT, "row strides"),
    (dict(y_scale=16), _lib.ERR_INVALID_ARGUMENT, "alias"),
    (dict(y_scale=32), _lib.ERR_INVALID_ARGUMENT, "alias"),
    (dict(residual=48, h=112), _lib.ERR_INVALID_ARGUMENT, "alias"),
])
def test_fwd_fp8_argument_errors(lib, kw, code, msg):
    assert _fwd_fp8(lib, **kw) == code
    assert msg in _lib.last_error() and "fwd_fp8" in _lib.last_error()


def test_fwd_fp8_zero_rows_is_a_no_op(lib):
    assert _fwd_fp8(lib, rows=0, x=None, y=None, y_scale=None) == 0
    assert _lib.last_error() == ""


@pytest.mark.parametrize("kw,code,msg", [
    (dict(dtype=5), _lib.ERR_UNSUPPORTED_DTYPE, "unsupported dtype"),
    (dict(dtype=1, w_dtype=2), _lib.ERR_UNSUPPORTED_DTYPE, "unsupported dtype"),
    (dict(dim=-3), _lib.ERR_INVALID_ARGUMENT, "invalid shape"),
    (dict(inv_rms=None), _lib.ERR_INVALID_ARGUMENT, "must not be NULL"),
    (dict(saved=None), _lib.ERR_INVALID_ARGUMENT, "must not be NULL"),
    (dict(ld_dx=1), _lib.ERR_INVALID_ARGUMENT, "row strides"),
    (dict(dx=16), _lib.ERR_INVALID_ARGUMENT, "alias"),
    (dict(dres=48), _lib.ERR_INVALID_ARGUMENT, "alias"),
    (dict(grad_h=96, dres=96), _lib.ERR_INVALID_ARGUMENT, "alias"),
    (dict(grad_h=96, ld_gh=8), _lib.ERR_INVALID_ARGUMENT, "row strides"),
    (dict(grad_h=32, ld_gh=128), _lib.ERR_INVALID_ARGUMENT, "same row stride"),
])
def test_bwd_argument_errors(lib, kw, code, msg):
    assert _bwd(lib, **kw) == code
    assert msg in _lib.last_error()


def _rmsnorm_rope_bwd(lib, **kw):
    args = dict(grad_y=16, h=32, weight=None, inv_rms=48, dx=64, dweight=None, ws=None,
                ws_bytes=0, rows=4, dim=64, ld_g=64, ld_h=64, ld_dx=64, seq=2, dtype=2,
                w_dtype=2, base=10000.0, stream=None)
    args.update(kw)
    return lib.velograd_rmsnorm_rope_bwd(*args.values())


@pytest.mark.parametrize("kw,code,msg", [
    (dict(dim=63, ld_g=63, ld_h=63, ld_dx=63), _lib.ERR_INVALID_ARGUMENT, "even dim"),
    (dict(seq=0), _lib.ERR_INVALID_ARGUMENT, "seq >= 1"),
    (dict(seq=3), _lib.ERR_INVALID_ARGUMENT, "dividing rows"),
    (dict(base=0.0), _lib.ERR_INVALID_ARGUMENT, "base"),
    (dict(base=float("inf")), _lib.ERR_INVALID_ARGUMENT, "base"),
    (dict(dtype=7), _lib.ERR_UNSUPPORTED_DTYPE, "unsupported dtype"),
    (dict(inv_rms=None), _lib.ERR_INVALID_ARGUMENT, "must not be NULL"),
    (dict(h=None), _lib.ERR_INVALID_ARGUMENT, "must not be NULL"),
    (dict(ld_dx=8), _lib.ERR_INVALID_ARGUMENT, "row strides"),
    (dict(dx=16), _lib.ERR_INVALID_ARGUMENT, "alias"),
    (dict(dx=32), _lib.ERR_INVALID_ARGUMENT, "alias"),
])
def test_rmsnorm_rope_bwd_argument_errors(lib, kw, code, msg):
    assert _rmsnorm_rope_bwd(lib, **kw) == code
    assert msg in _lib.last_error()


def test_rmsnorm_rope_bwd_zero_rows_is_a_no_op(lib):
    assert _rmsnorm_rope_bwd(lib, rows=0, grad_y=None, h=None, inv_rms=None, dx=None) == 0
    assert _lib.last_error() == ""


def test_check_maps_status_to_python_exceptions():
    with pytest.raises(TypeError):
        _lib.check(_lib.ERR_UNSUPPORTED_DTYPE, "x")
    with pytest.raises(ValueError):
        _lib.check(_lib.ERR_INVALID_ARGUMENT, "x")
    with pytest.raises(ValueError):
        _lib.check(_lib.ERR_WORKSPACE_TOO_SMALL, "x")
    with pytest.raises(RuntimeError):
        _lib.check(98, "x")  # a hipError_t
    _lib.check(0, "x")


def test_dtype_codes_match_header():
    with open(HEADER) as f:
        text = f.read()
    for name, val in (("F32", _lib.DTYPE_F32), ("F16", _lib.DTYPE_F16), ("BF16", _lib.DTYPE_BF16)):
        assert re.search(rf"#define VELOGRAD_DTYPE_{name} {val}\b", text)
    assert _lib.TORCH_DTYPE_CODES[torch.bfloat16] == _lib.DTYPE_BF16
    for name, val in (("MX_E4M3", _lib.MX_E4M3), ("MX_E2M1", _lib.MX_E2M1),
                      ("ROPE_HALF", _lib.ROPE_HALF), ("ROPE_INTERLEAVED", _lib.ROPE_INTERLEAVED)):
        assert re.search(rf"#define VELOGRAD_{name} {val}\b", text), name


def _rope(lib, **kw):
    args = dict(x=16, out=32, outer=1, seq=4, heads=2, dim=64, rot_dim=64, theta=10000.0,
                inverse=0, pairing=0, dtype=2, stream=None)
    args.update(kw)
    return lib.velograd_rope(*args.values())


@pytest.mark.parametrize("kw,code,msg", [
    (dict(dtype=3), _lib.ERR_UNSUPPORTED_DTYPE, "unsupported dtype"),
    (dict(seq=-1), _lib.ERR_INVALID_ARGUMENT, "invalid shape"),
    (dict(rot_dim=63), _lib.ERR_INVALID_ARGUMENT, "must be even"),
    (dict(rot_dim=0), _lib.ERR_INVALID_ARGUMENT, "must be even"),
    (dict(rot_dim=66), _lib.ERR_INVALID_ARGUMENT, "<= dim"),
    (dict(dim=16384, rot_dim=16384), _lib.ERR_INVALID_ARGUMENT, "needs the interleaved"),
    (dict(dim=16384, rot_dim=16384, pairing=1, x=8), _lib.ERR_INVALID_ARGUMENT,
     "needs the interleaved"),
    (dict(x=None), _lib.ERR_INVALID_ARGUMENT, "must not be NULL"),
    (dict(theta=0.0), _lib.ERR_INVALID_ARGUMENT, "theta"),
    (dict(pairing=2), _lib.ERR_INVALID_ARGUMENT, "pairing"),
    (dict(pairing=-1), _lib.ERR_INVALID_ARGUMENT, "pairing"),
    (dict(theta=float("nan")), _lib.ERR_INVALID_ARGUMENT, "theta"),
])
def test_rope_argument_errors(lib, kw, code, msg):
    # the message also shows that both translation units share the library's error state
    assert _rope(lib, **kw) == code
    assert msg in _lib.last_error() and "rope" in _lib.last_error()


def test_rope_empty_is_a_no_op(lib):
    assert _rope(lib, seq=0, x=None, out=None) == 0
    assert _lib.last_error() == ""


def _fwd_mx(lib, **kw):
    args = dict(x=16, residual=None, weight=None, y=32, scales=112, h=None, inv_rms=None,
                rows=4, dim=64, ld_x=64, ld_res=64, ld_y=64, ld_s=2, ld_h=64, dtype=2,
                w_dtype=2, fmt=0, eps=1e-5, stream=None)
    args.update(kw)
    return lib.velograd_rmsnorm_residual_fwd_mx(*args.values())


@pytest.mark.parametrize("kw,code,msg", [
    (dict(fmt=2), _lib.ERR_UNSUPPORTED_DTYPE, "unsupported mx_format"),
    (dict(dtype=9), _lib.ERR_UNSUPPORTED_DTYPE, "unsupported dtype"),
    (dict(dim=48, ld_x=48, ld_y=48, ld_h=48), _lib.ERR_INVALID_ARGUMENT, "multiple of the 32"),
    (dict(scales=None), _lib.ERR_INVALID_ARGUMENT, "scales must not be NULL"),
    (dict(ld_s=1), _lib.ERR_INVALID_ARGUMENT, "row strides"),
    (dict(fmt=1, ld_y=31), _lib.ERR_INVALID_ARGUMENT, "row strides"),
    (dict(scales=16), _lib.ERR_INVALID_ARGUMENT, "alias"),
])
def test_fwd_mx_argument_errors(lib, kw, code, msg):
    assert _fwd_mx(lib, **kw) == code
    assert msg in _lib.last_error() and "fwd_mx" in _lib.last_error()


def test_fwd_mx_e2m1_accepts_half_width_rows(lib):
    # rows = 0 returns before any launch; the e2m1 row stride is dim / 2 bytes
    assert _fwd_mx(lib, fmt=1, ld_y=32, rows=0) == 0


def test_last_error_is_per_thread(lib):
    """The error text lives in thread-local storage: a failing call on one thread does not
    overwrite what another thread reads."""
    import threading

    seen = {}

    def worker(name, kw):
        rc = _fwd(lib, **kw)
        seen[name] = (rc, _lib.last_error())

    t1 = threading.Thread(target=worker, args=("a", dict(dtype=7)))
    t1.start()
    t1.join()
    t2 = threading.Thread(target=worker, args=("b", dict(dim=0)))
    t2.start()
    t2.join()
    assert seen["a"][0] == _lib.ERR_UNSUPPORTED_DTYPE and "unsupported dtype" in seen["a"][1]
    assert seen["b"][0] == _lib.ERR_INVALID_ARGUMENT and "invalid shape" in seen["b"][1]
    # this thread's own last error is untouched by the workers
    assert _fwd(lib, rows=0, x=None, y=None) == 0 and _lib.last_error() == ""


def test_stream_probe_rejects_bad_arguments():
    """The bench's same-run ceiling probe checks its arguments before launching anything."""
    from velograd_amd.build import PROBE_LIB_PATH
    if not os.path.exists(PROBE_LIB_PATH):
        pytest.skip("stream probe not built")
    fn = ctypes.CDLL(PROBE_LIB_PATH).velograd_stream_probe
    fn.restype = ctypes.c_int32
    fn.argtypes = [ctypes.c_int32] + [ctypes.c_void_p] * 4 + [ctypes.c_int64, ctypes.c_void_p]
    p = 4096  # never dereferenced: every call below fails its argument check first
    assert fn(0, p, p, p, p, 0, None) == -1            # no vectors
    assert fn(0, None, p, p, p, 16, None) == -1        # no source
    assert fn(1, p, None, p, p, 16, None) == -1        # fwd pattern: second source missing
    assert fn(1, p, p, p, None, 16, None) == -1        # fwd pattern: second output missing
    assert fn(3, p, None, p, None, 16, None) == -1     # read-only: second source missing
    assert fn(4, p, None, p, None, 16, None) == -1     # write-only: second output missing
    assert fn(9, p, p, p, p, 16, None) == -1           # unknown pattern
