"""velograd_rmsnorm_residual_bwd_noalloc, the allocation-free backward, through the C ABI.

It runs the kernels of velograd_rmsnorm_residual_bwd with the dweight partial rows in the
library's own device scratch array, so its outputs must equal that entry point's bit for bit.
Two calls in a row, the second on a smaller input, show that what the first call left in the
scratch does not leak into the second.  Sizes beyond the scratch are refused before anything is
launched.  Graph replays of the variant equal its eager result."""

import ctypes

import numpy as np
import pytest
import torch

from velograd_amd import _lib
from velograd_amd import kernels as vk

from tests._parity import assert_dweight, gaussian, to_device, upcast, weight_vec

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
SCRATCH_BYTES = 16 << 20


def _p(t):
    return None if t is None else t.data_ptr()


def _inputs(rng, rows, dim, dtype, wdtype, saved_is_h, grad_h):
    g = to_device(gaussian(rng, (rows, dim)), dtype)
    h = to_device(gaussian(rng, (rows, dim)), dtype)
    w = to_device(weight_vec(rng, dim), wdtype)
    inv = torch.from_numpy(
        (1.0 / np.sqrt(np.mean(upcast(h).astype(np.float64) ** 2, axis=1) + 1e-5))
        .astype(np.float32)).to(DEV)
    saved = h if saved_is_h else (h.float() * inv[:, None]).to(dtype)
    gh = to_device(gaussian(rng, (rows, dim)), dtype) if grad_h else None
    return g, saved, w, inv, gh


def _run(lib, noalloc, g, saved, saved_is_h, w, inv, gh, with_dres, with_dw):
    rows, dim = g.shape
    dx = torch.empty_like(g)
    dres = torch.empty_like(g) if with_dres else None
    dw = torch.empty(dim, device=DEV, dtype=torch.float32) if with_dw else None
    code = _lib.TORCH_DTYPE_CODES[g.dtype]
    wcode = _lib.TORCH_DTYPE_CODES[w.dtype]
    stream = torch.cuda.current_stream().cuda_stream
    head = (_p(g), _p(saved), int(saved_is_h), _p(w), _p(inv), _p(gh), _p(dx), _p(dres), _p(dw))
    tail = (rows, dim, dim, dim, dim, dim, dim, code, wcode, stream)
    if noalloc:
        rc = lib.velograd_rmsnorm_residual_bwd_noalloc(*head, *tail)
    else:
        ws_bytes = vk.bwd_workspace_bytes(rows, dim, DEV)
        ws = torch.empty(max(ws_bytes, 16), device=DEV, dtype=torch.uint8)
        rc = lib.velograd_rmsnorm_residual_bwd(*head, _p(ws), ws_bytes, *tail)
    _lib.check(rc, "noalloc" if noalloc else "workspace")
    torch.cuda.synchronize()
    return dx, dres, dw


# (rows, dim, dtype, weight dtype, saved is h, grad_h, dres): the first call is the largest;
# every later one is smaller and takes another plan (one-chunk ring rows of 512 threads, 128-
# thread row groups, the element-strided ring for an odd dim).
CALLS = [
    (4096, 4096, torch.bfloat16, torch.bfloat16, True, False, True),
    (300, 1000, torch.bfloat16, torch.float32, False, True, False),
    (257, 1001, torch.float32, torch.float32, True, False, False),
]


def test_noalloc_matches_workspace_entry_point_on_calls_in_a_row():
    lib = _lib.load()
    rng = np.random.default_rng(0)
    for i, (rows, dim, dt, wdt, sih, gh, dres) in enumerate(CALLS):
        print(f"noalloc call {i}: rows={rows} dim={dim} {dt} w={wdt} saved_is_h={sih} "
              f"grad_h={gh} dres={dres}", flush=True)
        need = vk.bwd_workspace_bytes(rows, dim, DEV)
        assert 0 < need <= SCRATCH_BYTES
        g, saved, w, inv, ghv = _inputs(rng, rows, dim, dt, wdt, sih, gh)
        want = _run(lib, False, g, saved, sih, w, inv, ghv, dres, True)
        got = _run(lib, True, g, saved, sih, w, inv, ghv, dres, True)
        assert torch.equal(got[0], want[0]), f"call {i}: dx differs"
        if dres:
            assert torch.equal(got[1], want[1]), f"call {i}: dres differs"
            assert torch.equal(got[1], got[0])
        assert torch.equal(got[2], want[2]), f"call {i}: dweight differs"
        # and dweight is the sum over rows of g * xhat (float64 truth), to the parity bar
        xhat = upcast(saved).astype(np.float64)
        if sih:
            xhat = xhat * upcast(inv).astype(np.float64)[:, None]
        truth = (upcast(g).astype(np.float64) * xhat).sum(axis=0)
        assert_dweight(upcast(got[2]), truth, what=f"call {i} dweight")


def test_noalloc_without_dweight_matches():
    lib = _lib.load()
    rng = np.random.default_rng(1)
    g, saved, w, inv, _ = _inputs(rng, 512, 2048, torch.bfloat16, torch.bfloat16, True, False)
    want = _run(lib, False, g, saved, True, w, inv, None, False, False)
    got = _run(lib, True, g, saved, True, w, inv, None, False, False)
    assert torch.equal(got[0], want[0])


def test_noalloc_refuses_sizes_beyond_the_scratch():
    lib = _lib.load()
    # fp32 rows of 16384: every plan the backward can pick needs more than 16 MiB of partial
    # rows (checked on the CPU in tests/plan_check.cpp).  The buffers are real device tensors of
    # the stated shape, so a refusal that regressed would compute on valid memory and fail the
    # return-code assertion instead of touching invalid addresses.
    rows, dim = 2048, 16384
    assert vk.bwd_workspace_bytes(rows, dim, DEV) > SCRATCH_BYTES
    g = torch.zeros(rows, dim, device=DEV, dtype=torch.float32)
    h = torch.zeros_like(g)
    dx = torch.empty_like(g)
    w = torch.ones(dim, device=DEV, dtype=torch.float32)
    inv = torch.ones(rows, device=DEV, dtype=torch.float32)
    dw = torch.empty(dim, device=DEV, dtype=torch.float32)
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.velograd_rmsnorm_residual_bwd_noalloc(
        _p(g), _p(h), 1, _p(w), _p(inv), None, _p(dx), None, _p(dw), rows, dim, dim, dim, dim,
        dim, dim, _lib.DTYPE_F32, _lib.DTYPE_F32, stream)
    torch.cuda.synchronize()
    assert rc == _lib.ERR_WORKSPACE_TOO_SMALL
    msg = _lib.last_error()
    assert "fixed maximum" in msg and str(SCRATCH_BYTES) in msg, msg


def test_noalloc_graph_replays_equal_eager():
    """The variant's use case: HIP graph capture with no allocation inside the captured work.
    Each replay follows eager work on the same stream and is checked against the eager bits."""
    lib = _lib.load()
    rng = np.random.default_rng(2)
    rows, dim = 2048, 4096
    g, saved, w, inv, _ = _inputs(rng, rows, dim, torch.bfloat16, torch.bfloat16, True, False)
    want = _run(lib, True, g, saved, True, w, inv, None, False, True)
    dx = torch.empty_like(g)
    dw = torch.empty(dim, device=DEV, dtype=torch.float32)
    code = _lib.DTYPE_BF16
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            rc = lib.velograd_rmsnorm_residual_bwd_noalloc(
                _p(g), _p(saved), 1, _p(w), _p(inv), None, _p(dx), None, _p(dw), rows, dim,
                dim, dim, dim, dim, dim, code, code, ctypes.c_void_p(side.cuda_stream))
    torch.cuda.current_stream().wait_stream(side)
    _lib.check(rc, "noalloc under capture")
    for rep in range(4):
        # eager work in between: a no-alloc backward on other inputs (it rewrites the scratch),
        # then the outputs are clobbered
        other = _inputs(rng, 1024, 4096, torch.bfloat16, torch.bfloat16, True, False)
        _run(lib, True, other[0], other[1], True, other[2], other[3], None, False, True)
        dx.fill_(float("nan"))
        dw.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(dx, want[0]), f"replay {rep}: dx differs"
        assert torch.equal(dw, want[2]), f"replay {rep}: dweight differs"


_FIRST_CALL_UNDER_CAPTURE = r'''
import ctypes, sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[1])
from velograd_amd import _lib
from velograd_amd import kernels as vk
lib = _lib.load()
dev = torch.device("cuda", 0)
rows, dim = 1024, 4096
gen = torch.Generator(device=dev).manual_seed(7)
g = torch.randn(rows, dim, device=dev, generator=gen).to(torch.bfloat16)
h = torch.randn(rows, dim, device=dev, generator=gen).to(torch.bfloat16)
w = (1 + 0.1 * torch.randn(dim, device=dev, generator=gen)).to(torch.bfloat16)
inv = torch.rand(rows, device=dev, generator=gen) + 0.5
dx = torch.empty_like(g)
dw = torch.empty(dim, device=dev, dtype=torch.float32)
code = _lib.DTYPE_BF16
torch.cuda.synchronize()
side = torch.cuda.Stream()
graph = torch.cuda.CUDAGraph()
# the library's first call of the process (and so its first look-up of the scratch address)
# is made while the stream is being captured
with torch.cuda.stream(side):
    with torch.cuda.graph(graph, stream=side):
        rc = lib.velograd_rmsnorm_residual_bwd_noalloc(
            g.data_ptr(), h.data_ptr(), 1, w.data_ptr(), inv.data_ptr(), None, dx.data_ptr(),
            None, dw.data_ptr(), rows, dim, dim, dim, dim, dim, dim, code, code,
            ctypes.c_void_p(side.cuda_stream))
_lib.check(rc, "first call under capture")
want_dx, want_dw = vk.fused_rmsnorm_residual_backward(g, h, w, inv.view(rows, 1), saved_is_h=True)
for rep in range(3):
    dx.fill_(float("nan"))
    dw.fill_(float("nan"))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(dx, want_dx), f"replay {rep}: dx differs"
    assert torch.equal(dw, want_dw), f"replay {rep}: dweight differs"
print("first-call-under-capture ok", flush=True)
'''


def test_noalloc_first_call_of_the_process_under_capture():
    """A fresh process whose first library call is a no-alloc backward inside HIP graph capture
    (the scratch address is looked up there): the replays equal the workspace entry point."""
    import os
    import subprocess
    import sys
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("child: first no-alloc call under graph capture, bf16 1024 x 4096", flush=True)
    out = subprocess.run([sys.executable, "-c", _FIRST_CALL_UNDER_CAPTURE, repo],
                         capture_output=True, text=True, timeout=240)
    assert out.returncode == 0, (out.stdout[-2000:], out.stderr[-4000:])
    assert "first-call-under-capture ok" in out.stdout
