"""The pybind11 fast path of the forward (velograd_amd/csrc/torch_fastpath.cpp) against the
ctypes path to the same kernels: bitwise equal outputs, the same qualification rules (calls it
declines return [] and take the general path), the same errors, and `h is x` without residual."""

import os
import subprocess
import sys

import pytest
import torch

from velograd_amd import _lib
from velograd_amd import kernels as vk

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _fast():
    fp = _lib.fastpath()
    if fp is None:
        pytest.skip("the fast path is not built (velograd_amd.build builds it)")
    return fp


def _ctypes_forward(x, r, w, eps, min_mean_sq):
    d = x.shape[-1]
    rows = x.numel() // d
    y = torch.empty_like(x)
    h = torch.empty_like(x) if r is not None else x
    inv = torch.empty(x.shape[:-1] + (1,), device=x.device)
    code = _lib.TORCH_DTYPE_CODES[x.dtype]
    wcode = _lib.TORCH_DTYPE_CODES[w.dtype] if w is not None else code
    args = (x.data_ptr(), r.data_ptr() if r is not None else None,
            w.data_ptr() if w is not None else None, y.data_ptr(),
            h.data_ptr() if r is not None else None, inv.data_ptr(), rows, d, d, d, d, d, code,
            wcode, eps)
    st = torch.cuda.current_stream().cuda_stream
    lib = _lib.load()
    rc = (lib.velograd_rmsnorm_fwd(*args, min_mean_sq, st) if min_mean_sq > 0
          else lib.velograd_rmsnorm_residual_fwd(*args, st))
    _lib.check(rc, "forward")
    return y, h, inv


@pytest.mark.parametrize("dtype,wdt,shape,res,floor", [
    (torch.bfloat16, torch.bfloat16, (1, 5120), True, 0.0),
    (torch.bfloat16, torch.float32, (7, 7168), True, 0.0),
    (torch.float16, torch.float16, (2, 3, 1000), False, 0.0),
    (torch.float32, torch.float32, (64, 768), True, 1e-12),
    (torch.bfloat16, None, (257, 4096), False, 1e-12),
])
def test_fast_path_matches_ctypes_bitwise(dtype, wdt, shape, res, floor):
    fp = _fast()
    torch.manual_seed(0)
    x = torch.randn(shape, device="cuda").to(dtype)
    x[0] = 0
    r = torch.randn(shape, device="cuda").to(dtype) if res else None
    w = (1 + 0.1 * torch.randn(shape[-1], device="cuda")).to(wdt) if wdt is not None else None
    got = fp.forward(x, r, w, 1e-6, floor)
    assert len(got) == 3
    want = _ctypes_forward(x, r, w, 1e-6, floor)
    torch.cuda.synchronize()
    for a, b in zip(got, want):
        assert a.shape == b.shape and a.dtype == b.dtype
        assert torch.equal(a.view(torch.uint8) if a.element_size() == 1 else a, b)
    y, h, inv = vk.fused_rmsnorm_residual_forward(x, r, w, 1e-6, min_mean_sq=floor)
    assert torch.equal(y, want[0]) and torch.equal(inv, want[2])
    if r is None:
        assert h is x


def test_fast_path_declines_what_it_does_not_cover():
    fp = _fast()
    x = torch.randn(8, 256, device="cuda", dtype=torch.bfloat16)
    assert fp.forward(x.t().contiguous().t(), None, None, 1e-6, 0.0) == []          # strided
    assert fp.forward(x, x.float(), None, 1e-6, 0.0) == []                           # dtype
    assert fp.forward(x, None, torch.ones(255, device="cuda"), 1e-6, 0.0) == []      # weight
    assert fp.forward(x, None, torch.ones(256, device="cuda").half(), 1e-6, 0.0) == []
    assert fp.forward(x.cpu(), None, None, 1e-6, 0.0) == []                          # host
    assert fp.forward(x[:0], None, None, 1e-6, 0.0) == []                            # empty
    # the public API still handles such calls through the general path
    y, _, _ = vk.fused_rmsnorm_residual_forward(x.t().contiguous().t(), None, None, 1e-6)
    assert y.shape == x.shape


def test_fast_path_errors_are_python_errors():
    fp = _fast()
    x = torch.randn(4, 64, device="cuda")
    with pytest.raises(ValueError):
        fp.forward(x, None, None, 1e-6, float("nan"))


def test_ctypes_path_alone_gives_the_same_bits():
    """The whole public forward with the fast path switched off, in a child process."""
    _fast()
    code = ("import torch\nfrom velograd_amd import kernels as vk, _lib\n"
            "assert _lib.fastpath() is None\n"
            "torch.manual_seed(3)\n"
            "x = torch.randn(33, 4096, device='cuda').bfloat16()\n"
            "r = torch.randn(33, 4096, device='cuda').bfloat16()\n"
            "y, h, inv = vk.fused_rmsnorm_residual_forward(x, r, None, 1e-5)\n"
            "torch.save((y.cpu(), h.cpu(), inv.cpu()), '/tmp/vg_nofast.pt')\n")
    env = dict(os.environ, VELOGRAD_NO_FASTPATH="1", PYTHONPATH=REPO)
    subprocess.run([sys.executable, "-c", code], env=env, check=True, timeout=240)
    torch.manual_seed(3)
    x = torch.randn(33, 4096, device="cuda").bfloat16()
    r = torch.randn(33, 4096, device="cuda").bfloat16()
    y, h, inv = vk.fused_rmsnorm_residual_forward(x, r, None, 1e-5)
    yo, ho, invo = torch.load("/tmp/vg_nofast.pt", weights_only=True)
    assert torch.equal(y.cpu(), yo) and torch.equal(h.cpu(), ho) and torch.equal(inv.cpu(), invo)
