"""The ring-pipelined backward (bwd_ring_kernel, the default for rows of whole 16-byte chunks
over up to 512 threads and two chunks per thread, at most 1/8 of the lanes idle) against the
oracle, at row counts that put every pattern of its loop to work: rows fewer than the row slots
(no steady iteration), whole rings of iterations, and one or two iterations past the last whole
ring, with and without rows missing in the last one; the ring holds three rows (two with
grad_h).  Rows that leave lanes idle are checked over every dtype and both chunk counts.  Its
per-row arithmetic is that of bwd_vec_kernel, so dx must equal that kernel's bit for bit (the
child process below runs it with VELOGRAD_BWD_RING=0); dweight groups its partial sums by other
row slots, so it is held to the dweight tolerance."""

import json
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from oracle import fused_rmsnorm as ora
from tests import _parity as P
from velograd_amd import kernels as vk

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _inputs(rows, d, dtype, wdtype, seed, grad_h):
    rng = np.random.default_rng(seed)
    h = P.to_device(P.gaussian(rng, (rows, d)), dtype)
    g = P.to_device(P.gaussian(rng, (rows, d)), dtype)
    w = P.to_device(P.weight_vec(rng, d), wdtype)
    gh = P.to_device(P.gaussian(rng, (rows, d)), dtype) if grad_h else None
    _, _, inv = vk.fused_rmsnorm_residual_forward(h, None, w, 1e-5)
    return h, g, w, inv, gh


def _check_oracle(dx, dw, h, g, w, inv, gh, what):
    g32, h32, w32, r32 = (P.upcast(t) for t in (g, h, w, inv))
    xhat = h32 * r32
    if gh is None:
        rdx, rdw = ora.fused_rmsnorm_residual_backward(g32, xhat, w32, r32)
    else:
        rdx, rdw = ora.backward_with_residual_grad(g32, xhat, w32, r32, P.upcast(gh))
    if dx.dtype == torch.float32:
        scale = P.dx_scale(g32 * w32, xhat, r32) + (0.0 if gh is None else np.abs(P.upcast(gh)))
        assert np.max(np.abs(P.upcast(dx) - rdx) / scale) <= P.FP32_REL_TOL, what
    else:
        P.dx_check(dx, rdx, g32 * w32, xhat, r32, what,
                   grad_h=None if gh is None else P.upcast(gh))
    P.assert_dweight(P.upcast(dw), rdw, what)


# 256 CUs x 1 row group of 512 threads = 256 row slots at dim 4096 bf16 (512 slots of two
# 256-thread row groups when two chunks per thread are asked for); rings of 3 iterations (2 with
# grad_h): every pattern of the walk around 256, 512 and 768 rows
RING_ROWS = [1, 2, 255, 256, 257, 300, 511, 512, 513, 767, 768, 769, 1024, 1025, 1535, 1536,
             1537, 2047, 2304, 2560, 16385]


@pytest.mark.parametrize("grad_h", [False, True], ids=["ring3", "ring2-grad_h"])
@pytest.mark.parametrize("rows", RING_ROWS)
def test_ring_row_counts_match_oracle(rows, grad_h):
    print(f"ring backward rows={rows} grad_h={grad_h}", flush=True)
    h, g, w, inv, gh = _inputs(rows, 4096, torch.bfloat16, torch.bfloat16, rows, grad_h)
    dx, dw = vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True, grad_h=gh)
    torch.cuda.synchronize()
    _check_oracle(dx, dw, h, g, w, inv, gh, f"rows={rows} grad_h={grad_h}")


# (rows, dim, dtype, weight dtype, grad_h, chunks per thread of the ring's plan): one 512-thread
# row group of two chunks (dim 8192), eight row groups of one wave (dim 512), two 256-thread row
# groups of two chunks in fp32, four 128-thread row groups in fp16 with an fp32 weight
LAYOUTS = [(3000, 8192, torch.bfloat16, torch.bfloat16, False, 2),
           (2049, 512, torch.bfloat16, torch.float32, True, 1),
           (1500, 2048, torch.float32, torch.float32, False, 2),
           (999, 1024, torch.float16, torch.float32, True, 1)]

_CHILD = r"""
import json, sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[1])
from tests import _parity as P
from velograd_amd import kernels as vk
cases = json.loads(sys.argv[2])
out = {}
for i, (rows, d, dt, wdt, gh) in enumerate(cases):
    dt, wdt = getattr(torch, dt), getattr(torch, wdt)
    rng = np.random.default_rng(rows * 7 + d)
    h = P.to_device(P.gaussian(rng, (rows, d)), dt)
    g = P.to_device(P.gaussian(rng, (rows, d)), dt)
    w = P.to_device(P.weight_vec(rng, d), wdt)
    ghv = P.to_device(P.gaussian(rng, (rows, d)), dt) if gh else None
    _, _, inv = vk.fused_rmsnorm_residual_forward(h, None, w, 1e-5)
    dx, _ = vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True, grad_h=ghv)
    out[f"dx{i}"] = dx.view(torch.int16 if dx.element_size() == 2 else torch.int32).cpu().numpy()
np.savez(sys.argv[3], **out)
"""


def _bitwise_against_previous_kernel(layouts, tmp_path):
    """dx of the ring bit for bit against bwd_vec_kernel's in a child process
    (VELOGRAD_BWD_RING=0) over the same row layout (VELOGRAD_BWD_NV = the ring's chunks per
    thread), so both sum each row in the same order."""
    legacy = {}
    for nv in sorted({case[5] for case in layouts}):
        idx = [i for i, case in enumerate(layouts) if case[5] == nv]
        cases = [(r, d, str(dt).split(".")[-1], str(wdt).split(".")[-1], gh)
                 for r, d, dt, wdt, gh, _ in (layouts[i] for i in idx)]
        path = str(tmp_path / f"legacy{nv}.npz")
        env = dict(os.environ, VELOGRAD_BWD_RING="0", VELOGRAD_BWD_NV=str(nv))
        print(f"child process: the same backwards with VELOGRAD_BWD_RING=0 VELOGRAD_BWD_NV={nv}",
              flush=True)
        r = subprocess.run([sys.executable, "-c", _CHILD, REPO, json.dumps(cases), path],
                           env=env, capture_output=True, text=True, timeout=110)
        assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
        got = np.load(path)
        for k, i in enumerate(idx):
            legacy[i] = got[f"dx{k}"]
    for i, (rows, d, dt, wdt, gh, nv) in enumerate(layouts):
        print(f"ring vs previous kernel: {rows}x{d} {dt} w={wdt} grad_h={gh} nv={nv}", flush=True)
        rng = np.random.default_rng(rows * 7 + d)
        h = P.to_device(P.gaussian(rng, (rows, d)), dt)
        g = P.to_device(P.gaussian(rng, (rows, d)), dt)
        w = P.to_device(P.weight_vec(rng, d), wdt)
        ghv = P.to_device(P.gaussian(rng, (rows, d)), dt) if gh else None
        _, _, inv = vk.fused_rmsnorm_residual_forward(h, None, w, 1e-5)
        dx, dw = vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True, grad_h=ghv)
        bits = dx.view(torch.int16 if dx.element_size() == 2 else torch.int32).cpu().numpy()
        assert np.array_equal(bits, legacy[i]), f"dx differs at {rows}x{d} {dt}"
        _check_oracle(dx, dw, h, g, w, inv, ghv, f"{rows}x{d} {dt}")


def test_ring_dx_equals_the_previous_kernel_bitwise(tmp_path):
    _bitwise_against_previous_kernel(LAYOUTS, tmp_path)


_CHILD_NV2 = r"""
import json, sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[1])
from tests import _parity as P
from velograd_amd import kernels as vk
cases = json.loads(sys.argv[2])
out = {}
for i, (rows, d, dt, wdt, gh) in enumerate(cases):
    dt, wdt = getattr(torch, dt), getattr(torch, wdt)
    rng = np.random.default_rng(rows * 5 + d)
    h = P.to_device(P.gaussian(rng, (rows, d)), dt)
    g = P.to_device(P.gaussian(rng, (rows, d)), dt)
    w = P.to_device(P.weight_vec(rng, d), wdt)
    ghv = P.to_device(P.gaussian(rng, (rows, d)), dt) if gh else None
    _, _, inv = vk.fused_rmsnorm_residual_forward(h, None, w, 1e-5)
    dx, dw = vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True, grad_h=ghv)
    out[f"dx{i}"] = dx.float().cpu().numpy()
    out[f"dw{i}"] = dw.cpu().numpy()
np.savez(sys.argv[3], **out)
"""

# Two chunks per thread in row groups of 256, 128 and 64 threads (two, four and eight row groups
# a workgroup, combined in LDS), whole and with idle lanes: the layouts the planner takes when
# VELOGRAD_BWD_NV=2 asks for them (by default one chunk per thread comes first).
NV2 = [(2500, 4096, torch.bfloat16, torch.bfloat16, False),
       (1537, 4000, torch.bfloat16, torch.bfloat16, True),
       (999, 2048, torch.float16, torch.float32, False),
       (1200, 1000, torch.bfloat16, torch.bfloat16, True),
       (700, 2000, torch.float32, torch.float32, False)]


def test_ring_two_chunks_per_thread_match_oracle(tmp_path):
    cases = [(r, d, str(dt).split(".")[-1], str(wdt).split(".")[-1], gh)
             for r, d, dt, wdt, gh in NV2]
    path = str(tmp_path / "nv2.npz")
    env = dict(os.environ, VELOGRAD_BWD_NV="2")
    print("child process: ring backwards with VELOGRAD_BWD_NV=2", flush=True)
    r = subprocess.run([sys.executable, "-c", _CHILD_NV2, REPO, json.dumps(cases), path], env=env,
                       capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    got = np.load(path)
    for i, (rows, d, dt, wdt, gh) in enumerate(NV2):
        print(f"two chunks per thread: {rows}x{d} {dt} w={wdt} grad_h={gh}", flush=True)
        rng = np.random.default_rng(rows * 5 + d)
        h = P.to_device(P.gaussian(rng, (rows, d)), dt)
        g = P.to_device(P.gaussian(rng, (rows, d)), dt)
        w = P.to_device(P.weight_vec(rng, d), wdt)
        ghv = P.to_device(P.gaussian(rng, (rows, d)), dt) if gh else None
        _, _, inv = vk.fused_rmsnorm_residual_forward(h, None, w, 1e-5)
        dx = torch.from_numpy(got[f"dx{i}"]).to(dt)
        dw = torch.from_numpy(got[f"dw{i}"])
        _check_oracle(dx, dw, h, g, w, inv, ghv, f"nv2 {rows}x{d} {dt}")


# Rows of fewer 16-byte chunks than their row group's lanes hold (at most 1/8 of the slots idle):
# the idle lanes reload the row's last chunk, add nothing to the row's sum and dweight and store
# nothing.  (rows, dim, dtype, weight dtype, grad_h); the comments give idle / all chunk slots.
IDLE = [(1537, 4000, torch.bfloat16, torch.bfloat16, False, 1),  # 12/512, one row group
        (2049, 5000, torch.bfloat16, torch.bfloat16, True, 2),   # 15/640, 320 threads, 2 chunks
        (1000, 3000, torch.float16, torch.float32, False, 2),    # 9/384, two 192-thread groups
        (4097, 1000, torch.bfloat16, torch.bfloat16, True, 1),   # 3/128, four row groups
        (3001, 2000, torch.float32, torch.float32, False, 2),    # 12/512, two row groups
        (401, 1000, torch.float32, torch.float32, True, 2),      # 6/256, four row groups, more
                                                                  # row slots than rows
        (999, 456, torch.bfloat16, torch.float32, True, 1),      # 7/64, eight row groups
        (2500, 3200, torch.float16, torch.float16, False, 1),    # 48/448
        (700, 6272, torch.bfloat16, torch.bfloat16, True, 2),    # 112/896, 448 threads, 2 chunks
        (3000, 768, torch.bfloat16, torch.bfloat16, True, 1),    # 32/128: a partly idle last wave
        (1700, 1280, torch.float16, torch.float32, False, 1)]    # 32/192, two row groups


@pytest.mark.parametrize("rows,d,dt,wdt,gh,nv", IDLE,
                         ids=[f"{r}x{d}-{str(t).split('.')[-1]}" for r, d, t, _, _, _ in IDLE])
def test_ring_idle_lanes_match_oracle(rows, d, dt, wdt, gh, nv):
    print(f"ring backward with idle lanes {rows}x{d} {dt} w={wdt} grad_h={gh}", flush=True)
    h, g, w, inv, ghv = _inputs(rows, d, dt, wdt, rows + d, gh)
    dres = torch.empty_like(g)
    dx, dw = vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True, grad_h=ghv,
                                                dresidual_out=dres)
    torch.cuda.synchronize()
    _check_oracle(dx, dw, h, g, w, inv, ghv, f"{rows}x{d} {dt}")
    assert torch.equal(dres, dx)
    acc = np.einsum("rd,rd->d", P.upcast(g).astype(np.float64),
                    (P.upcast(h) * P.upcast(inv)).astype(np.float64))
    P.assert_dweight(P.upcast(dw), acc, "dweight vs float64")
    dx2, dw2 = vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True, grad_h=ghv)
    assert torch.equal(dx, dx2) and torch.equal(dw, dw2)


def test_ring_idle_lanes_dx_equals_the_previous_kernel_bitwise(tmp_path):
    _bitwise_against_previous_kernel(IDLE, tmp_path)


# Rows of 8n + 4 two-byte elements (hidden sizes such as 4100), whose rows start on 8-byte
# boundaries only: each whole chunk moves as two 8-byte halves and the row's last 4 elements form
# an extra half chunk of the row group's lane 0.  (rows, dim, dtype, weight dtype or None,
# grad_h); one chunk per thread in row groups of 512, 256 and 128 threads, one idle lane (4092).
RING8 = [(2049, 4100, torch.bfloat16, torch.bfloat16, False),
         (1537, 4100, torch.float16, torch.float32, True),
         (999, 2052, torch.bfloat16, torch.float32, False),   # two row groups a workgroup
         (4097, 1028, torch.bfloat16, torch.bfloat16, True),  # four row groups a workgroup
         (300, 4092, torch.float16, torch.float16, False),    # 511 whole chunks over 512 lanes
         (5000, 4100, torch.bfloat16, None, False),
         (1, 4100, torch.bfloat16, torch.bfloat16, True),     # one row, one workgroup
         (2, 508, torch.bfloat16, torch.bfloat16, False),     # 63 whole chunks, 64-thread rows
         (513, 508, torch.float16, torch.float32, True),      # eight row groups a workgroup
         (2000, 100, torch.bfloat16, torch.bfloat16, True)]   # 12 whole chunks, 64-thread rows


@pytest.mark.parametrize("rows,d,dt,wdt,gh", RING8,
                         ids=[f"{r}x{d}-{str(t).split('.')[-1]}" for r, d, t, _, _ in RING8])
def test_ring_rows_of_8_byte_alignment_match_oracle(rows, d, dt, wdt, gh):
    print(f"ring backward, rows of 8-byte alignment {rows}x{d} {dt} w={wdt} grad_h={gh}",
          flush=True)
    rng = np.random.default_rng(rows + d)
    h = P.to_device(P.gaussian(rng, (rows, d)), dt)
    g = P.to_device(P.gaussian(rng, (rows, d)), dt)
    w = P.to_device(P.weight_vec(rng, d), wdt) if wdt is not None else None
    ghv = P.to_device(P.gaussian(rng, (rows, d)), dt) if gh else None
    _, _, inv = vk.fused_rmsnorm_residual_forward(h, None, w, 1e-5)
    dres = torch.empty_like(g)
    dx, dw = vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True, grad_h=ghv,
                                                dresidual_out=dres)
    torch.cuda.synchronize()
    g32, h32, r32 = P.upcast(g), P.upcast(h), P.upcast(inv)
    w32 = P.upcast(w) if w is not None else None
    xhat = h32 * r32
    gw = g32 * w32 if w32 is not None else g32
    if ghv is None:
        rdx, rdw = ora.fused_rmsnorm_residual_backward(g32, xhat, w32, r32)
    else:
        rdx, rdw = ora.backward_with_residual_grad(g32, xhat, w32, r32, P.upcast(ghv))
    P.dx_check(dx, rdx, gw, xhat, r32, f"{rows}x{d}",
               grad_h=None if ghv is None else P.upcast(ghv))
    assert torch.equal(dres, dx)
    if w is None:
        assert dw is None
    else:
        P.assert_dweight(P.upcast(dw), rdw.reshape(-1), f"{rows}x{d}")
        acc = np.einsum("rd,rd->d", g32.astype(np.float64), xhat.astype(np.float64))
        P.assert_dweight(P.upcast(dw), acc, "dweight vs float64")
    dx2, dw2 = vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True, grad_h=ghv)
    assert torch.equal(dx, dx2)
    if w is not None:
        assert torch.equal(dw, dw2)


def test_ring_rows_of_8_byte_alignment_in_wider_tensors():
    """Streams of different row strides, all multiples of 8 bytes: g and dx in rows of 4104
    elements, h in rows of 4100 (through the C ABI); the rows' places inside their 16-byte lines
    then differ from stream to stream and from row to row."""
    from velograd_amd import _lib
    lib = _lib.load()
    print("ring backward, 8-byte rows in tensors of strides 4104 and 4100", flush=True)
    rows, d, wide = 1500, 4100, 4104
    rng = np.random.default_rng(4100)
    h = P.to_device(P.gaussian(rng, (rows, d)), torch.bfloat16)
    gw = P.to_device(P.gaussian(rng, (rows, wide)), torch.bfloat16)
    w = P.to_device(P.weight_vec(rng, d), torch.bfloat16)
    _, _, inv = vk.fused_rmsnorm_residual_forward(h, None, w, 1e-5)
    g = gw[:, :d].contiguous()
    ref_dx, ref_dw = vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True)
    out = torch.full((rows, wide), 7.0, device="cuda", dtype=torch.bfloat16)
    dw = torch.empty(d, device="cuda", dtype=torch.float32)
    ws_bytes = vk.bwd_workspace_bytes(rows, d, torch.device("cuda"))
    ws = torch.empty(ws_bytes, device="cuda", dtype=torch.uint8)
    inv1 = inv.reshape(rows).contiguous()
    rc = lib.velograd_rmsnorm_residual_bwd(
        gw.data_ptr(), h.data_ptr(), 1, w.data_ptr(), inv1.data_ptr(), None, out.data_ptr(), None,
        dw.data_ptr(), ws.data_ptr(), ws_bytes, rows, d, wide, d, d, wide, d,
        _lib.DTYPE_BF16, _lib.DTYPE_BF16, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "ring backward over strided 8-byte rows")
    torch.cuda.synchronize()
    assert torch.equal(out[:, :d], ref_dx) and torch.equal(dw, ref_dw)
    assert bool((out[:, d:] == 7.0).all()), "a store left its row"
    _check_oracle(ref_dx, ref_dw, h, g, w, inv, None, "strided 8-byte rows")


def test_ring_dres_and_in_place_grad_h():
    """dres gets the same bits as dx; dx may be grad_h itself (accumulation in place)."""
    from velograd_amd import _lib
    lib = _lib.load()
    rows, d = 2500, 4096
    h, g, w, inv, gh = _inputs(rows, d, torch.bfloat16, torch.bfloat16, 5, True)
    ref, _ = vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True, grad_h=gh)
    dres = torch.empty_like(g)
    dx, _ = vk.fused_rmsnorm_residual_backward(g, h, w, inv, saved_is_h=True, grad_h=gh,
                                               dresidual_out=dres)
    assert torch.equal(dx, ref) and torch.equal(dres, ref)
    acc = gh.clone()
    inv1 = inv.reshape(rows).contiguous()
    rc = lib.velograd_rmsnorm_residual_bwd(
        g.data_ptr(), h.data_ptr(), 1, w.data_ptr(), inv1.data_ptr(), acc.data_ptr(),
        acc.data_ptr(), None, None, None, 0, rows, d, d, d, d, d, d,
        _lib.DTYPE_BF16, _lib.DTYPE_BF16, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "ring backward in place")
    assert torch.equal(acc, ref)
