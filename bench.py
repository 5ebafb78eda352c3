#!/usr/bin/env python3
"""Fused RMSNorm + residual, forward + backward, bf16 16384 x 4096 on one MI355X.

One step = one forward (y, h, inv_rms from x, residual, weight) plus one backward (dx and fp32
dweight from grad_y, the saved h and inv_rms) over one batch of synthetic rows, launched through
the library's C ABI on torch's current stream.  Inputs are resident in HBM before timing starts.

MALL hygiene: MI355X's 256 MB Infinity Cache would otherwise serve repeated inputs, so the step
rotates over `--sets` independent buffer sets (768 MiB each at the default workload) and the
backward of a step works on a different set than its forward, so no input of a step was
touched by the step before it.

Output: one JSON line (the driver's contract) with
  value      = algorithmic bytes of a step / wall time of a step (GB/s, whole job, 1 GPU)
  roofline   = the forward kernel (the larger of the two): algorithmic bytes per launch over its
               mean launch time from HIP events on the launch stream, in passes run before the
               warm-up: batches of 10 back-to-back launches with events around each batch only
               (`--kernel-events` launches); per-launch events in the step sequence give the
               medians and minima.  Against 8 TB/s HBM; `traffic` comes from the committed
               rocprofv3 PMC summary when present (extra.roofline_bwd: the backward's two stages
               the same way)
  cpu_baseline = the NumPy restatement of the reference CPU path (oracle/) on the whole workload,
               on the GPU leg's own inputs, on this host, single-threaded NumPy.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import subprocess
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, AMD public spec
METRIC = "fused RMSNorm+residual fwd+bwd GB/s and % HBM peak, bf16 16384x4096"

CONFIGS = {
    # name: (rows, dim, eps, does backward)
    "A": (512, 768, 1e-6, False),
    "B": (8192, 4096, 1e-5, False),
    "C": (16384, 4096, 1e-5, True),
    "D": (32768, 8192, 1e-5, True),
    # not BASELINE configurations.  U: rows of 4100 bf16 elements (8200 bytes, not a 16-byte
    # multiple) start on 8-byte boundaries and take the register-resident kernels in 8-byte
    # halves; O (only with --config O): rows of 4095, odd, take the element-strided backward and
    # the generic forward
    "U": (16384, 4100, 1e-5, True),
    "O": (16384, 4095, 1e-5, True),
}


def fwd_bytes(rows: int, d: int, s: int) -> int:
    """Read x, residual, weight; write y, h (activation dtype) and fp32 inv_rms."""
    return 4 * rows * d * s + d * s + 4 * rows


def bwd_bytes(rows: int, d: int, s: int) -> int:
    """Read grad_y, h, weight, fp32 inv_rms; write dx (activation dtype), fp32 dweight."""
    return 3 * rows * d * s + d * s + 4 * rows + 4 * d


def bwd_grad_h_bytes(rows: int, d: int, s: int) -> int:
    """Backward with the residual-stream gradient (the training path): read grad_y, h and
    grad_h, write dx; plus weight, inv_rms and fp32 dweight."""
    return 4 * rows * d * s + d * s + 4 * rows + 4 * d


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=500)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--config", choices=sorted(CONFIGS), default="C")
    p.add_argument("--sets", type=int, default=4, help="rotating buffer sets (MALL hygiene)")
    p.add_argument("--kernel-events", type=int, default=100,
                   help="launches of each kernel timed with HIP events before the warm-up "
                        "(at least 50)")
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="CPU-baseline budget; 0 skips it")
    p.add_argument("--no-fp8", action="store_true",
                   help="skip timing the fp8 and MX-epilogue forwards (reported under extra)")
    p.add_argument("--no-other-configs", action="store_true",
                   help="skip the A/B/C/D/U summary lines (reported under extra)")
    p.add_argument("--no-decode", action="store_true",
                   help="skip the config E decode-latency table (reported under extra)")
    p.add_argument("--decode-calls", type=int, default=1000,
                   help="calls per config E shape for the back-to-back and host timings")
    p.add_argument("--no-rope", action="store_true",
                   help="skip timing the fused RoPE kernel (reported under extra)")
    p.add_argument("--no-norm-rope", action="store_true",
                   help="skip the fused versus two-pass RMSNorm + RoPE timing and the "
                        "module-form norm on its buffers")
    p.add_argument("--norm-rope-dim", type=int, default=4096,
                   help="hidden size of the interleaved RoPE and norm + RoPE legs (their rows "
                        "are the config's)")
    p.add_argument("--no-torch-baseline", action="store_true",
                   help="skip the PyTorch eager comparison and the reference benchmark's shapes")
    p.add_argument("--no-copy-ceiling", action="store_true",
                   help="skip the same-run stream-probe ceilings")
    p.add_argument("--row-scaling", action="store_true",
                   help="instead of the bench line: the forward, the backward with and without "
                        "dweight and their streaming probes over 4096..65536 rows at dim 4096 "
                        "bf16, with each kernel's fixed cost and cost per row (a markdown table)")
    p.add_argument("--probe-sweep", action="store_true",
                   help="instead of the benchmark: sweep the stream probe's shapes over the "
                        "config's tensors and print a markdown table of the byte patterns' "
                        "ceilings")
    return p.parse_args(argv)


def lscpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return platform.processor() or "unknown"


def _time_oracle_step(ora, x, res, w, g, eps: float, with_bwd: bool, budget_s: float,
                      min_runs: int = 5):
    """Median wall time of the reference CPU path (fused.py:28-66 through the oracle's NumPy
    restatement) on the given fp32 arrays: forward, then xhat = h * inv_rms and the backward.
    One untimed warm-up, then at least `min_runs` timed runs and until `budget_s` has passed."""
    def one():
        y, h, inv = ora.fused_rmsnorm_residual_forward(x, res, w, eps)
        if with_bwd:
            ora.fused_rmsnorm_residual_backward(g, h * inv, w, inv)

    one()  # warm-up
    times = []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        one()
        times.append(time.perf_counter() - t0)
        if len(times) >= min_runs and time.perf_counter() - t_start >= budget_s:
            break
    return statistics.median(times), len(times)


def cpu_baseline(rows: int, d: int, s: int, eps: float, budget_s: float, with_bwd: bool,
                 inputs):
    """The oracle (NumPy restatement of fused.py:28-66) timed on this host at the workload's
    full size, on `inputs` = (x, residual, weight, grad_y): fp32 upcasts of the GPU leg's own
    first buffer set (the same numbers the GPU computes on), copied to the host outside the
    timed region.  GB/s uses the GPU workload's algorithmic bytes (element size `s`).  A
    1024-row slice of the same arrays is timed too."""
    import numpy as np

    from oracle import fused_rmsnorm as ora

    x, res, w, g = inputs
    per_row = (fwd_bytes(rows, d, s) + (bwd_bytes(rows, d, s) if with_bwd else 0)) / rows
    med, nruns = _time_oracle_step(ora, x, res, w, g, eps, with_bwd, budget_s)
    rows_per_s = rows / med

    sample_rows = min(rows, 1024)
    smed, snruns = _time_oracle_step(ora, x[:sample_rows], res[:sample_rows], w,
                                     g[:sample_rows], eps, with_bwd, min(budget_s, 2.0))

    rng = np.random.default_rng(0)
    # the shapes of the reference's own benchmark (benchmarks/bench_vs_pytorch.py:43-72), fp32
    xb = rng.standard_normal((512, 4096), dtype=np.float32)
    wb = rng.standard_normal(4096, dtype=np.float32)
    qb = rng.standard_normal((512, 1024), dtype=np.float32)
    ref_shapes = {}
    for name, fn in (("rmsnorm_512x4096_fp32_ms", lambda: ora.fused_rmsnorm_residual(xb, None, wb, 1e-5)),
                     ("rope_512x1024_hd64_fp32_ms", lambda: ora.fused_rope(qb, head_dim=64))):
        fn()
        tt = []
        for _ in range(7):
            t0 = time.perf_counter()
            fn()
            tt.append(time.perf_counter() - t0)
        ref_shapes[name] = round(statistics.median(tt) * 1e3, 3)
    return {
        "value": round(rows_per_s * per_row / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"the whole workload: {rows} rows x {d}, fwd{'+bwd' if with_bwd else ''}, on "
                   f"fp32 upcasts of the GPU leg's own first buffer set; NumPy (single-threaded "
                   f"ufuncs); median of {nruns} runs after 1 warm-up; GB/s = the GPU workload's "
                   f"algorithmic bytes / median time"),
        "ms_median": round(med * 1e3, 3),
        "rows_per_s": round(rows_per_s, 1),
        "runs": nruns,
        "sample_1024_rows": {"ms_median": round(smed * 1e3, 3), "runs": snruns,
                             "rows_per_s": round(sample_rows / smed, 1),
                             "gbs": round(sample_rows / smed * per_row / 1e9, 4)},
        "host_cpu": lscpu_model(),
        "os_cpu_count": os.cpu_count(),
        "affinity_cpus": len(os.sched_getaffinity(0)),
        "reference_benchmark_shapes": ref_shapes,
    }


def traffic_file(config: str) -> str:
    return os.path.join(REPO, "profiles", f"pmc_traffic_config_{config}.json")


def load_traffic(config: str, which: str = "fwd"):
    """HBM bytes per launch of the forward (`which` = "fwd"), of the backward's two stages
    ("bwd") or of the backward with grad_h ("bwd_grad_h") from the committed rocprofv3 PMC
    summary of `config`, or None."""
    path = traffic_file(config)
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get(f"{which}_traffic_bytes_per_launch")


def traffic_source(config: str):
    """The file `roofline.traffic` is read from and the sha256 of its bytes (the commit that
    last changed it holds the same bytes), or None."""
    import hashlib

    path = traffic_file(config)
    if not os.path.exists(path):
        return None
    with open(path, "rb") as f:
        digest = hashlib.sha256(f.read()).hexdigest()[:16]
    return {"file": os.path.relpath(path, REPO), "sha256_16": digest}


def stream_ceilings(sets, stream_bytes: int, stream) -> dict:
    """Same-run practical ceiling: plain streaming kernels (velograd_amd/csrc/stream_probe.hip)
    with the forward's (2 reads + 2 writes) and the backward's (2 reads + 1 write) byte pattern
    over tensors of the workload's size, rotating over the same buffer sets (cold MALL); plus the
    same streams read only and written only, which show what mixing the two directions costs."""
    import ctypes

    import torch

    from velograd_amd.build import PROBE_LIB_PATH

    if not os.path.exists(PROBE_LIB_PATH):
        return {}
    lib = ctypes.CDLL(PROBE_LIB_PATH)
    fn = lib.velograd_stream_probe
    fn.restype = ctypes.c_int32
    fn.argtypes = [ctypes.c_int32] + [ctypes.c_void_p] * 4 + [ctypes.c_int64, ctypes.c_void_p]
    n16 = stream_bytes // 16
    sp = stream.cuda_stream
    out = {}
    shape = lib.velograd_stream_probe_shape
    shape.restype = ctypes.c_int32
    shape.argtypes = ([ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p,
                       ctypes.c_int64] + [ctypes.c_int32] * 5 + [ctypes.c_void_p])
    for name, pattern, nstreams, keys in (("copy", 0, 2, ("x", None, "y", None)),
                                          ("fwd_pattern", 1, 4, ("x", "res", "y", "h")),
                                          ("bwd_pattern", 2, 3, ("x", "res", "y", None)),
                                          ("read_only", 3, 2, ("x", "res", "y", None)),
                                          ("write_only", 4, 2, ("x", None, "y", "h")),
                                          ("grad_h_pattern", 5, 4, ("x", "res", "y", "h"))):
        def run(i):
            b = sets[i % len(sets)]
            ptrs = [b[k].data_ptr() if k else None for k in keys]
            rc = fn(pattern, ptrs[0], ptrs[1], ptrs[2], ptrs[3], n16, sp)
            if rc != 0:
                raise RuntimeError(f"stream probe {name} failed: {rc}")
        for i in range(len(sets)):
            run(i)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 20
        e0.record(stream)
        for i in range(reps):
            run(i)
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        out[f"ceiling_{name}_gbs"] = round(nstreams * n16 * 16 / (us * 1e-6) / 1e9, 1)
    # The backward pattern in the fastest shape the probe sweep found for it (256 threads, four
    # 16-byte vectors per thread and stream, one pass, no per-access guards;
    # profiles/stream_probe_sweep_config_C.md): no shape beat the forward pattern's bench shape.
    ptrs = [((ctypes.c_void_p * 3)(b["x"].data_ptr(), b["res"].data_ptr(), 0),
             (ctypes.c_void_p * 2)(b["y"].data_ptr(), b["h"].data_ptr())) for b in sets]

    def run_best(i):
        rd, wr = ptrs[i % len(sets)]
        rc = shape(2, 1, ctypes.cast(rd, ctypes.c_void_p), ctypes.cast(wr, ctypes.c_void_p), n16,
                   256, 4, 16, 0, 7 | 8, sp)
        if rc != 0:
            raise RuntimeError(f"stream probe best 2R1W shape failed: {rc}")
    for i in range(len(sets)):
        run_best(i)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 20
    e0.record(stream)
    for i in range(reps):
        run_best(i)
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    out["ceiling_bwd_pattern_best_shape_gbs"] = round(3 * n16 * 16 / (us * 1e-6) / 1e9, 1)
    return out


def fp8_forward_timing(lib, sets, rows: int, d: int, s: int, code: int, eps: float,
                       stream) -> dict:
    """The forward with the fp8 output epilogue (velograd_rmsnorm_residual_fwd_fp8) on the same
    rotating buffer sets: y leaves as one e4m3 byte per element (written into the first half of
    each set's y buffer) plus one fp32 scale per row."""
    import torch

    from velograd_amd import _lib

    fn = lib.velograd_rmsnorm_residual_fwd_fp8
    scales = [torch.empty(rows, device=b["x"].device, dtype=torch.float32) for b in sets]
    args = [(b["x"].data_ptr(), b["res"].data_ptr(), b["w"].data_ptr(), b["y"].data_ptr(),
             sc.data_ptr(), b["h"].data_ptr(), b["inv"].data_ptr(), rows, d, d, d, d, d, code,
             code, eps, stream.cuda_stream) for b, sc in zip(sets, scales)]
    for a in args:
        _lib.check(fn(*a), "fwd_fp8 warm-up")
    reps = 40
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    rc = 0
    for i in range(reps):
        rc |= fn(*args[i % len(args)])
    e1.record(stream)
    torch.cuda.synchronize()
    _lib.check(rc, "fwd_fp8 timed")
    us = e0.elapsed_time(e1) * 1e3 / reps
    nbytes = 3 * rows * d * s + rows * d + d * s + 8 * rows
    return {"fp8_fwd_us_mean": round(us, 2), "fp8_fwd_bytes": nbytes,
            "fp8_fwd_gbs": round(nbytes / (us * 1e-6) / 1e9, 1)}


def mx_forward_timing(lib, sets, rows: int, d: int, s: int, code: int, eps: float,
                      stream) -> dict:
    """The forward with the MX epilogues (velograd_rmsnorm_residual_fwd_mx), MXFP8 and MXFP4,
    on the same rotating buffer sets: y leaves as e4m3 bytes or e2m1 nibbles (written into each
    set's y buffer) plus one E8M0 byte per 32 elements."""
    import torch

    from velograd_amd import _lib

    fn = lib.velograd_rmsnorm_residual_fwd_mx
    scales = [torch.empty(rows, d // 32, device=b["x"].device, dtype=torch.uint8) for b in sets]
    out = {}
    for name, fmt, ybytes in (("mxfp8", _lib.MX_E4M3, d), ("mxfp4", _lib.MX_E2M1, d // 2)):
        args = [(b["x"].data_ptr(), b["res"].data_ptr(), b["w"].data_ptr(), b["y"].data_ptr(),
                 sc.data_ptr(), b["h"].data_ptr(), b["inv"].data_ptr(), rows, d, d, d, ybytes,
                 d // 32, d, code, code, fmt, eps, stream.cuda_stream)
                for b, sc in zip(sets, scales)]
        for a in args:
            _lib.check(fn(*a), f"fwd_{name} warm-up")
        reps = 40
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        rc = 0
        for i in range(reps):
            rc |= fn(*args[i % len(args)])
        e1.record(stream)
        torch.cuda.synchronize()
        _lib.check(rc, f"fwd_{name} timed")
        us = e0.elapsed_time(e1) * 1e3 / reps
        nbytes = 3 * rows * d * s + rows * ybytes + rows * (d // 32) + d * s + 4 * rows
        out.update({f"{name}_fwd_us_mean": round(us, 2), f"{name}_fwd_bytes": nbytes,
                    f"{name}_fwd_gbs": round(nbytes / (us * 1e-6) / 1e9, 1)})
    return out


def decode_latency(lib, stream, calls: int = 1000) -> list:
    """Config E: forward at decode shapes T in {1, 7, 64, 257} x D in {5120, 7168} bf16, where
    launch latency, not bandwidth, sets the time.  Per shape: device us per call back to back
    (HIP events around `calls` launches), median isolated latency (launch to completion, events
    around one launch, 200 samples), median host us per call of the C ABI (ctypes) and of the
    Python API, and device us per call when 32 calls are captured in a HIP graph and replayed."""
    import torch

    from velograd_amd import _lib
    from velograd_amd import kernels as vk

    dev = torch.device("cuda", 0)
    out = []
    fn = lib.velograd_rmsnorm_residual_fwd
    for d in (5120, 7168):
        for t in (1, 7, 64, 257):
            x = torch.randn(t, d, device=dev).to(torch.bfloat16)
            r = torch.randn(t, d, device=dev).to(torch.bfloat16)
            w = (1 + 0.1 * torch.randn(d, device=dev)).to(torch.bfloat16)
            y, h = torch.empty_like(x), torch.empty_like(x)
            inv = torch.empty(t, device=dev)
            args = (x.data_ptr(), r.data_ptr(), w.data_ptr(), y.data_ptr(), h.data_ptr(),
                    inv.data_ptr(), t, d, d, d, d, d, _lib.DTYPE_BF16, _lib.DTYPE_BF16, 1e-6,
                    stream.cuda_stream)
            for _ in range(50):
                fn(*args)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            rc = 0
            for _ in range(calls):
                rc |= fn(*args)
            e1.record(stream)
            torch.cuda.synchronize()
            _lib.check(rc, "decode calls")
            dev_us = e0.elapsed_time(e1) * 1e3 / calls
            iso = []
            for _ in range(200):
                e0.record(stream)
                fn(*args)
                e1.record(stream)
                torch.cuda.synchronize()
                iso.append(e0.elapsed_time(e1) * 1e3)
            host_c, host_py = [], []
            for _ in range(calls):
                t0 = time.perf_counter()
                fn(*args)
                host_c.append(time.perf_counter() - t0)
            torch.cuda.synchronize()
            for _ in range(calls):
                t0 = time.perf_counter()
                vk.fused_rmsnorm_residual_forward(x, r, w, 1e-6)
                host_py.append(time.perf_counter() - t0)
            torch.cuda.synchronize()
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(3):
                    vk.fused_rmsnorm_residual_forward(x, r, w, 1e-6)
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for _ in range(32):
                    vk.fused_rmsnorm_residual_forward(x, r, w, 1e-6)
            for _ in range(3):
                g.replay()
            torch.cuda.synchronize()
            e0.record(stream)
            for _ in range(30):
                g.replay()
            e1.record(stream)
            torch.cuda.synchronize()
            med = lambda v: sorted(v)[len(v) // 2]  # noqa: E731
            out.append({"T": t, "D": d, "device_us_back_to_back": round(dev_us, 2),
                        "isolated_us_median": round(med(iso), 2),
                        "host_us_c_abi_median": round(med(host_c) * 1e6, 2),
                        "host_us_python_api_median": round(med(host_py) * 1e6, 2),
                        "graph_replay_us_per_call": round(e0.elapsed_time(e1) * 1e3 / 960, 2),
                        "bytes": 8 * t * d + 2 * d + 4 * t})
            del g
    return out


def rope_timing(lib, tokens: int, stream, sets: int = 2, norm_rope: bool = True,
                hid: int = 4096) -> dict:
    """Fused RoPE (velograd_rope) on a Llama-3-8B-like attention input of the same token
    count: q [tokens, 32, 128] and k [tokens, 8, 128] bf16, theta 500000, one launch each per
    step, rotating over `sets` buffer sets.  Bytes: q and k read once and written once.  Then
    the interleaved RoPE and the norm + RoPE legs over [tokens, hid]."""
    import torch

    from velograd_amd import _lib

    dev = torch.device("cuda", 0)
    shapes = ((32, 128), (8, 128))
    bufs = []
    for _ in range(sets):
        b = []
        for heads, hd in shapes:
            x = torch.randn(tokens, heads, hd, device=dev).to(torch.bfloat16)
            b.append((x, torch.empty_like(x), heads, hd))
        bufs.append(b)
    fn = lib.velograd_rope
    sp = stream.cuda_stream

    def step(i):
        rc = 0
        for x, out, heads, hd in bufs[i % sets]:
            rc |= fn(x.data_ptr(), out.data_ptr(), 1, tokens, heads, hd, hd, 500000.0, 0,
                     _lib.ROPE_HALF, _lib.DTYPE_BF16, sp)
        return rc

    for i in range(sets * 2):
        _lib.check(step(i), "rope warm-up")
    reps = 40
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    rc = 0
    for i in range(reps):
        rc |= step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    _lib.check(rc, "rope timed")
    us = e0.elapsed_time(e1) * 1e3 / reps
    nbytes = sum(2 * tokens * h * d * 2 for h, d in shapes)
    del bufs

    # The reference model's RoPE (functional.py:287-315): interleaved pairs over the whole
    # hidden vector of the normalised attention input, [tokens, hid] bf16, base 10000.
    ibufs = [(torch.randn(tokens, hid, device=dev).to(torch.bfloat16),
              torch.empty(tokens, hid, device=dev, dtype=torch.bfloat16)) for _ in range(sets)]

    def istep(i):
        x, out = ibufs[i % sets]
        return fn(x.data_ptr(), out.data_ptr(), 1, tokens, 1, hid, hid, 10000.0, 0,
                  _lib.ROPE_INTERLEAVED, _lib.DTYPE_BF16, sp)

    out = {"rope_qk_us_mean": round(us, 2), "rope_qk_bytes": nbytes,
           "rope_qk_gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
           "rope_workload": f"q [{tokens},32,128] + k [{tokens},8,128] bf16, theta 5e5"}
    # velograd_rope rotates more than 8192 elements per token on 16-byte rows only (bf16 rows of
    # a multiple of 8 elements): other wide rows have no standalone leg and no two-pass comparison
    standalone = hid <= 8192 or hid % 8 == 0
    if standalone:
        for i in range(sets * 2):
            _lib.check(istep(i), "interleaved rope warm-up")
        torch.cuda.synchronize()
        e0.record(stream)
        rc = 0
        for i in range(reps):
            rc |= istep(i)
        e1.record(stream)
        torch.cuda.synchronize()
        _lib.check(rc, "interleaved rope timed")
        ius = e0.elapsed_time(e1) * 1e3 / reps
        ibytes = 2 * tokens * hid * 2
        out.update({
            "rope_interleaved_us_mean": round(ius, 2), "rope_interleaved_bytes": ibytes,
            "rope_interleaved_gbs": round(ibytes / (ius * 1e-6) / 1e9, 1),
            "rope_interleaved_workload": f"x [{tokens},{hid}] bf16, pairs (2i, 2i+1) over the "
                                         f"hidden vector, base 1e4 (functional.apply_rotary_emb)"})
    if not norm_rope:
        del ibufs
        return out

    # The model's attention-branch input (models/llama.py:48-49): RMSNorm then the interleaved
    # RoPE, fused in one pass (velograd_rmsnorm_rope_fwd) and as two passes (module-form norm,
    # then velograd_rope) over the same buffers.
    w = (1 + 0.1 * torch.randn(hid, device=dev)).to(torch.bfloat16)
    inv = torch.empty(tokens, device=dev)
    mid = torch.empty(tokens, hid, device=dev, dtype=torch.bfloat16)
    fused_fn, norm_fn = lib.velograd_rmsnorm_rope_fwd, lib.velograd_rmsnorm_fwd

    def fstep(i):
        x, out = ibufs[i % sets]
        return fused_fn(x.data_ptr(), None, w.data_ptr(), out.data_ptr(), None, inv.data_ptr(),
                        tokens, hid, hid, hid, hid, hid, tokens, _lib.DTYPE_BF16,
                        _lib.DTYPE_BF16, 1e-6, 1e-12, 10000.0, sp)

    def tstep(i):
        x, out = ibufs[i % sets]
        rc = norm_fn(x.data_ptr(), None, w.data_ptr(), mid.data_ptr(), None, inv.data_ptr(),
                     tokens, hid, hid, hid, hid, hid, _lib.DTYPE_BF16, _lib.DTYPE_BF16, 1e-6,
                     1e-12, sp)
        return rc | fn(mid.data_ptr(), out.data_ptr(), 1, tokens, 1, hid, hid, 10000.0, 0,
                       _lib.ROPE_INTERLEAVED, _lib.DTYPE_BF16, sp)

    def nstep(i):
        x, out = ibufs[i % sets]
        return norm_fn(x.data_ptr(), None, w.data_ptr(), out.data_ptr(), None, inv.data_ptr(),
                       tokens, hid, hid, hid, hid, hid, _lib.DTYPE_BF16, _lib.DTYPE_BF16, 1e-6,
                       1e-12, sp)

    times = {}
    legs = (("fused", fstep), ("two_pass", tstep), ("norm_only", nstep))
    for name, st in (legs if standalone else (legs[0], legs[2])):
        for i in range(sets * 2):
            _lib.check(st(i), f"norm+rope {name} warm-up")
        torch.cuda.synchronize()
        e0.record(stream)
        rc = 0
        for i in range(reps):
            rc |= st(i)
        e1.record(stream)
        torch.cuda.synchronize()
        _lib.check(rc, f"norm+rope {name} timed")
        times[name] = e0.elapsed_time(e1) * 1e3 / reps
    nbytes_fused = 2 * tokens * hid * 2 + hid * 2 + 4 * tokens

    # Its backward: grad_y rotated back and the norm's backward in one pass
    # (velograd_rmsnorm_rope_bwd), against the two passes (velograd_rope inverse into `mid`,
    # then velograd_rmsnorm_residual_bwd).  grad_y is the forward's output buffer, h is x.
    from velograd_amd import kernels as vk
    dxb = torch.empty(tokens, hid, device=dev, dtype=torch.bfloat16)
    dwb = torch.empty(hid, device=dev, dtype=torch.float32)
    ws_bytes = vk.bwd_workspace_bytes(tokens, hid, dev)
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    rope_bwd_fn, bwd_fn = lib.velograd_rmsnorm_rope_bwd, lib.velograd_rmsnorm_residual_bwd

    def bstep(i):
        x, gy = ibufs[i % sets]
        return rope_bwd_fn(gy.data_ptr(), x.data_ptr(), w.data_ptr(), inv.data_ptr(),
                           dxb.data_ptr(), dwb.data_ptr(), ws.data_ptr(), ws_bytes, tokens, hid,
                           hid, hid, hid, tokens, _lib.DTYPE_BF16, _lib.DTYPE_BF16, 10000.0, sp)

    def b2step(i):
        x, gy = ibufs[i % sets]
        rc = fn(gy.data_ptr(), mid.data_ptr(), 1, tokens, 1, hid, hid, 10000.0, 1,
                _lib.ROPE_INTERLEAVED, _lib.DTYPE_BF16, sp)
        return rc | bwd_fn(mid.data_ptr(), x.data_ptr(), 1, w.data_ptr(), inv.data_ptr(), None,
                           dxb.data_ptr(), None, dwb.data_ptr(), ws.data_ptr(), ws_bytes, tokens,
                           hid, hid, hid, hid, hid, hid, _lib.DTYPE_BF16, _lib.DTYPE_BF16, sp)

    for name, st in ((("bwd_fused", bstep), ("bwd_two_pass", b2step)) if standalone
                     else (("bwd_fused", bstep),)):
        for i in range(sets * 2):
            _lib.check(st(i), f"norm+rope {name} warm-up")
        torch.cuda.synchronize()
        e0.record(stream)
        rc = 0
        for i in range(reps):
            rc |= st(i)
        e1.record(stream)
        torch.cuda.synchronize()
        _lib.check(rc, f"norm+rope {name} timed")
        times[name] = e0.elapsed_time(e1) * 1e3 / reps
    nbytes_bwd = 3 * tokens * hid * 2 + hid * 2 + 4 * tokens + 4 * hid
    del ibufs, mid, dxb, ws
    out.update({
        "norm_rope_bwd_fused_us_mean": round(times["bwd_fused"], 2),
        "norm_rope_bwd_fused_gbs": round(nbytes_bwd / (times["bwd_fused"] * 1e-6) / 1e9, 1),
        "norm_rope_bwd_two_pass_us_mean": (round(times["bwd_two_pass"], 2) if standalone
                                           else None),
        "norm_rope_fused_us_mean": round(times["fused"], 2),
        "norm_rope_fused_gbs": round(nbytes_fused / (times["fused"] * 1e-6) / 1e9, 1),
        "norm_rope_two_pass_us_mean": round(times["two_pass"], 2) if standalone else None,
        # the module-form RMSNorm alone (nn.py:338-355: x read, y written, no residual)
        "norm_module_us_mean": round(times["norm_only"], 2),
        "norm_module_gbs": round(nbytes_fused / (times["norm_only"] * 1e-6) / 1e9, 1),
        "norm_rope_workload": f"RMSNorm (1e-12 floor) then interleaved RoPE of x [{tokens},"
                              f"{hid}] bf16 (models/llama.py:48-49), fused vs two passes"})
    return out


def measure(lib, config: str, steps: int, warmup: int, nsets: int, kernel_events: int,
            stream) -> dict:
    """Time `steps` steps of `config` (forward, plus backward where the config has one) on
    `nsets` rotating buffer sets, then per-kernel HIP events over `kernel_events` more steps."""
    import torch

    from velograd_amd import _lib
    from velograd_amd import kernels as vk

    rows, d, eps, with_bwd = CONFIGS[config]
    dt = torch.bfloat16 if config != "A" else torch.float32
    s = 2 if dt == torch.bfloat16 else 4
    code = _lib.TORCH_DTYPE_CODES[dt]
    dev = torch.device("cuda", 0)
    sp = stream.cuda_stream
    gen = torch.Generator(device=dev).manual_seed(0)
    ws_bytes = vk.bwd_workspace_bytes(rows, d, dev)

    def act():
        """x / residual: N(0, 1); config D: std 2, and exactly 0.1% of the entries (distinct,
        uniformly chosen, independently for each tensor) scaled by 50."""
        a = torch.randn(rows, d, device=dev, generator=gen)
        if config == "D":
            a *= 2.0
            idx = torch.randperm(rows * d, device=dev, generator=gen)[:rows * d // 1000]
            a.view(-1)[idx] *= 50.0
            del idx
        return a.to(dt)

    sets = []
    for _ in range(nsets):
        b = {
            "x": act(),
            "res": act(),
            "w": (1 + 0.1 * torch.randn(d, device=dev, generator=gen)).to(dt),
            "y": torch.empty(rows, d, device=dev, dtype=dt),
            "h": torch.empty(rows, d, device=dev, dtype=dt),
            "inv": torch.empty(rows, device=dev, dtype=torch.float32),
        }
        if with_bwd:
            b["g"] = torch.randn(rows, d, device=dev, generator=gen).to(dt)
            b["dx"] = torch.empty(rows, d, device=dev, dtype=dt)
            b["dw"] = torch.empty(d, device=dev, dtype=torch.float32)
            b["ws"] = torch.empty(max(ws_bytes, 16), device=dev, dtype=torch.uint8)
        sets.append(b)

    fwd_fn = lib.velograd_rmsnorm_residual_fwd
    bwd_fn = lib.velograd_rmsnorm_residual_bwd
    fwd_args = [(b["x"].data_ptr(), b["res"].data_ptr(), b["w"].data_ptr(), b["y"].data_ptr(),
                 b["h"].data_ptr(), b["inv"].data_ptr(), rows, d, d, d, d, d, code, code, eps, sp)
                for b in sets]
    bwd_args = []
    if with_bwd:
        bwd_args = [(b["g"].data_ptr(), b["h"].data_ptr(), 1, b["w"].data_ptr(),
                     b["inv"].data_ptr(), None, b["dx"].data_ptr(), None, b["dw"].data_ptr(),
                     b["ws"].data_ptr(), ws_bytes, rows, d, d, d, d, d, d, code, code, sp)
                    for b in sets]

    # every set gets a valid h / inv_rms before any backward reads it
    for a in fwd_args:
        _lib.check(fwd_fn(*a), "fwd")
    torch.cuda.synchronize()

    n = nsets
    half = n // 2

    def step(k, evs=None):
        if evs is not None:
            evs[0].record(stream)
        rc = fwd_fn(*fwd_args[k % n])
        if evs is not None:
            evs[1].record(stream)
        if with_bwd:
            rc |= bwd_fn(*bwd_args[(k + half) % n])
            if evs is not None:
                evs[2].record(stream)
        return rc

    # Kernel durations, in passes of their own before the warm-up and the timed steps: the step
    # sequence with HIP events on the launch stream around each forward and each backward (both
    # stages), `kernel_events` launches of each whatever `steps` is; the first step after the
    # synchronisation is dropped (its launch starts from an idle queue).  Running them first
    # also means the timed steps start on a GPU that has been busy, as in a training loop: with
    # a 5-step warm-up straight after setup, 20 timed steps read about 4% below the steady state.
    nev = max(50, kernel_events)
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(nev + 1)]
    torch.cuda.synchronize()
    rc = 0
    for k in range(nev + 1):
        rc |= step(k, events[k])
    torch.cuda.synchronize()
    _lib.check(rc, "kernel event pass")
    events = events[1:]

    # Launch means for the rooflines: batches of `per` back-to-back launches of one entry point
    # (rotating sets), events only around each batch, so no marker sits between two launches;
    # a batch's time / `per` is one launch plus the queue's gap to the next.
    def batch_mean_ms(fn, args, per=10):
        nb = max(5, nev // per)
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(nb + 1)]
        torch.cuda.synchronize()
        rc = 0
        for b in range(nb + 1):
            evs[b][0].record(stream)
            for i in range(per):
                rc |= fn(*args[(b * per + i) % n])
            evs[b][1].record(stream)
        torch.cuda.synchronize()
        _lib.check(rc, "batched launches")
        return statistics.fmean(e0.elapsed_time(e1) / per for e0, e1 in evs[1:]), nb * per

    fwd_batch_ms, nbatched = batch_mean_ms(fwd_fn, fwd_args)
    bwd_batch_ms = batch_mean_ms(bwd_fn, bwd_args)[0] if with_bwd else None
    gh_batch_ms = None
    if with_bwd:
        # the training path's backward: the residual-stream gradient grad_h (here the set's x)
        # read too and summed into dx in the same pass
        gh_args = [(b["g"].data_ptr(), b["h"].data_ptr(), 1, b["w"].data_ptr(),
                    b["inv"].data_ptr(), b["x"].data_ptr(), b["dx"].data_ptr(), None,
                    b["dw"].data_ptr(), b["ws"].data_ptr(), ws_bytes, rows, d, d, d, d, d, d,
                    code, code, sp) for b in sets]
        gh_batch_ms = batch_mean_ms(bwd_fn, gh_args)[0]
        # the same backward with no dweight requested (dweight = NULL): stage 1 alone, without
        # its partial rows, so the line shows what the deterministic dweight reduction costs
        nodw_args = [a[:8] + (None,) + a[9:] for a in bwd_args]
        nodw_batch_ms = batch_mean_ms(bwd_fn, nodw_args)[0]

    for k in range(warmup):
        _lib.check(step(k), "warm-up step")
    torch.cuda.synchronize()

    # Wall clock over `steps` unmarked steps: no event markers inside the timed region.
    t0 = time.perf_counter()
    rc = 0
    for k in range(steps):
        rc |= step(k)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    _lib.check(rc, "timed steps")

    fwd_ms = [e[0].elapsed_time(e[1]) for e in events]
    mean_fwd_ms = fwd_batch_ms
    fb = fwd_bytes(rows, d, s)
    bb = bwd_bytes(rows, d, s) if with_bwd else 0
    ms_per_step = (t1 - t0) * 1e3 / steps
    value = (fb + bb) / (ms_per_step * 1e-3) / 1e9
    out = {
        "value": value,
        "ms_per_step": ms_per_step,
        # launch mean from the back-to-back batches (the rooflines use it)
        "fwd_us_mean": round(mean_fwd_ms * 1e3, 2),
        # per-launch events in the step sequence (a marker on each side of every launch)
        "fwd_us_event_mean": round(statistics.fmean(fwd_ms) * 1e3, 2),
        "fwd_us_event_median": round(statistics.median(fwd_ms) * 1e3, 2),
        "fwd_us_event_min": round(min(fwd_ms) * 1e3, 2),
        "fwd_gbs": round(fb / (mean_fwd_ms * 1e-3) / 1e9, 1),
        "fwd_bytes": fb,
        "kernel_event_samples": len(events),
        "batched_launches": nbatched,
    }
    if with_bwd:
        bwd_ms = [e[1].elapsed_time(e[2]) for e in events]
        mean_bwd_ms = bwd_batch_ms
        out.update({
            "bwd_us_mean": round(mean_bwd_ms * 1e3, 2),
            "bwd_us_event_mean": round(statistics.fmean(bwd_ms) * 1e3, 2),
            "bwd_us_event_median": round(statistics.median(bwd_ms) * 1e3, 2),
            "bwd_us_event_min": round(min(bwd_ms) * 1e3, 2),
            "bwd_gbs": round(bb / (mean_bwd_ms * 1e-3) / 1e9, 1),
            "bwd_bytes": bb,
            "bwd_workspace_bytes": ws_bytes,
            "bwd_grad_h_us_mean": round(gh_batch_ms * 1e3, 2),
            "bwd_grad_h_bytes": bwd_grad_h_bytes(rows, d, s),
            "bwd_no_dweight_us_mean": round(nodw_batch_ms * 1e3, 2),
            "dweight_cost_us": round((mean_bwd_ms - nodw_batch_ms) * 1e3, 2),
        })
    out["rows_per_s"] = round(rows / (ms_per_step * 1e-3), 1)
    out["pct_hbm_peak"] = round(100.0 * value / HBM_PEAK_GBS, 2)
    out.update({"_sets": sets, "_fwd_args": fwd_args, "_bwd_args": bwd_args, "_s": s,
                "_code": code})
    return out


def torch_eager_timing(sets, rows: int, d: int, s: int, eps: float, with_bwd: bool, stream,
                       steps: int = 40) -> dict:
    """The same step in PyTorch eager operations on the same GPU and buffers, for comparison
    (the reference's own benchmark compares against PyTorch, benchmarks/bench_vs_pytorch.py):
    h = x + residual; y = F.rms_norm(h, (D,), weight, eps); autograd backward of y with grad_y
    -> dx (= dresidual) and dweight.  Same rotating buffer sets; wall clock per step.
    Informational, under extra."""
    import torch
    import torch.nn.functional as F

    n = len(sets)

    def step(k):
        b = sets[k % n]
        x = b["x"].detach().requires_grad_(True)
        w = b["w"].detach().requires_grad_(True)
        h = x + b["res"]
        y = F.rms_norm(h, (d,), w, eps)
        if with_bwd:
            torch.autograd.grad(y, (x, w), grad_outputs=b["g"])

    for k in range(5):
        step(k)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(steps):
        step(k)
    torch.cuda.synchronize()
    us = (time.perf_counter() - t0) * 1e6 / steps
    total = fwd_bytes(rows, d, s) + (bwd_bytes(rows, d, s) if with_bwd else 0)
    return {"torch_eager_step_us": round(us, 2),
            "torch_eager_gbs": round(total / (us * 1e-6) / 1e9, 1),
            "torch_eager_ops": "x + residual; F.rms_norm; autograd.grad(y, (x, weight))",
            "torch_version": torch.__version__}


def reference_benchmark_shapes(stream, calls: int = 500) -> dict:
    """Device and host time per call at the shapes the reference's own benchmark uses
    (benchmarks/bench_vs_pytorch.py:43-72): fused_rmsnorm_residual(x, None, weight, 1e-5) on
    512 x 4096 fp32 with weight ~ N(0,1), and fused_rope(x, head_dim=64) on 2-D x [512, 1024]
    fp32, both through the Python API on device tensors."""
    import torch

    from velograd_amd import kernels as vk

    dev = torch.device("cuda", 0)
    x = torch.randn(512, 4096, device=dev)
    w = torch.randn(4096, device=dev)
    q = torch.randn(512, 1024, device=dev)
    out = {}
    for name, fn in (("rmsnorm_512x4096_fp32", lambda: vk.fused_rmsnorm_residual(x, None, w, 1e-5)),
                     ("rope_512x1024_hd64_fp32", lambda: vk.fused_rope(q, head_dim=64))):
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        host = []
        e0.record(stream)
        for _ in range(calls):
            t0 = time.perf_counter()
            fn()
            host.append(time.perf_counter() - t0)
        e1.record(stream)
        torch.cuda.synchronize()
        back_to_back = e0.elapsed_time(e1) * 1e3 / calls
        iso = []
        for _ in range(100):
            e0.record(stream)
            fn()
            e1.record(stream)
            torch.cuda.synchronize()
            iso.append(e0.elapsed_time(e1) * 1e3)
        # back to back, the launches come no faster than the Python API issues them
        out[name] = {"device_us_per_call_back_to_back": round(back_to_back, 2),
                     "isolated_us_median": round(sorted(iso)[50], 2),
                     "host_us_python_api_median": round(sorted(host)[calls // 2] * 1e6, 2)}
    return out


def other_configs(lib, main_config: str, stream) -> dict:
    """The other configurations at modest step counts (A forward, the reference's own fp32 case:
    6.3 MB per step, so launch-bound and MALL-resident; B forward; D forward + backward; C when it
    is not the headline; U, rows that are not 16-byte multiples), reported under extra."""
    import torch

    out = {}
    for cfg, steps, nsets in (("A", 2000, 4), ("B", 100, 4), ("C", 100, 4), ("D", 40, 2),
                              ("U", 100, 4)):
        if cfg == main_config:
            continue
        m = measure(lib, cfg, steps, 5, nsets, 400 if cfg == "A" else 50, stream)
        for k in ("_sets", "_fwd_args", "_bwd_args", "_s", "_code"):
            m.pop(k)
        m["value"] = round(m["value"], 1)
        m["ms_per_step"] = round(m["ms_per_step"], 4)
        m["steps"], m["sets"] = steps, nsets
        out[cfg] = m
        del m
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return out


PROBE_PATTERNS = (("2R2W", 2, 2), ("2R1W", 2, 1), ("3R1W", 3, 1), ("1R1W", 1, 1),
                  ("2R0W", 2, 0), ("0R2W", 0, 2))


def probe_sweep(config: str, nsets: int = 4, reps: int = 12, rounds: int = 3) -> str:
    """The stream probe's shapes (velograd_stream_probe_shape) over the config's tensors, four
    per set (the forward's x, residual, h, y), rotating over `nsets` sets: each byte pattern with
    the bench's shape, every workgroup size x vectors per thread x bytes per lane one-pass, the
    bench's and the best one-pass shape on persistent grids, each load/store cache policy, and
    the second write stream unrotated, each in guarded and flat code (the probe's two code
    styles: a branch around each access, or none in whole tiles).  Per shape the best of
    `rounds` batches of `reps`
    back-to-back launches, HIP events around each batch.  Returns a markdown table."""
    import ctypes

    import torch

    from velograd_amd.build import PROBE_LIB_PATH

    lib = ctypes.CDLL(PROBE_LIB_PATH)
    fn = lib.velograd_stream_probe_shape
    fn.restype = ctypes.c_int32
    fn.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p,
                   ctypes.c_int64] + [ctypes.c_int32] * 5 + [ctypes.c_void_p]
    fixed = lib.velograd_stream_probe
    fixed.restype = ctypes.c_int32
    fixed.argtypes = [ctypes.c_int32] + [ctypes.c_void_p] * 4 + [ctypes.c_int64, ctypes.c_void_p]
    fixed_pattern = {"2R2W": 1, "2R1W": 2, "3R1W": 5, "1R1W": 0, "2R0W": 3, "0R2W": 4}
    rows, d, _, _ = CONFIGS[config]
    s = 2 if config != "A" else 4
    nbytes = rows * d * s
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    sets = [[torch.empty(nbytes, device=dev, dtype=torch.uint8).random_(0, 256)
             for _ in range(4)] for _ in range(nsets)]
    ptr_arrays = []
    for bufs in sets:
        rd = (ctypes.c_void_p * 3)(*[t.data_ptr() for t in bufs[:3]])
        wr = (ctypes.c_void_p * 2)(bufs[3].data_ptr(), bufs[2].data_ptr())
        ptr_arrays.append((rd, wr))
    n16 = nbytes // 16
    base = dict(block=256, vpt=2, lane=16, wpc=0, flags=7)

    def time_shape(nr, nw, block, vpt, lane, wpc, flags, pattern=None):
        def launch(i):
            rd, wr = ptr_arrays[i % nsets]
            if pattern is not None:  # the bench's own ceiling kernel
                bufs = sets[i % nsets]
                rc = fixed(pattern, bufs[0].data_ptr(), bufs[1].data_ptr(), bufs[3].data_ptr(),
                           bufs[2].data_ptr(), n16, stream.cuda_stream)
            else:
                rc = fn(nr, nw, ctypes.cast(rd, ctypes.c_void_p),
                        ctypes.cast(wr, ctypes.c_void_p), n16, block, vpt, lane, wpc, flags,
                        stream.cuda_stream)
            if rc != 0:
                raise RuntimeError(f"probe shape failed: rc {rc}")
        for i in range(nsets):
            launch(i)
        best = float("inf")
        for _ in range(rounds):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for i in range(reps):
                launch(i)
            e1.record(stream)
            torch.cuda.synchronize()
            best = min(best, e0.elapsed_time(e1) * 1e3 / reps)
        return best

    lines = [f"Stream-probe sweep over config {config}'s tensors ({nbytes} B per stream, "
             f"{nsets} rotating sets of 4 streams), best of {rounds} batches of {reps} "
             "launches. µs per launch and TB/s of the streams' bytes; 'bench shape' = the "
             "bench's own ceiling kernel (velograd_stream_probe: 256 threads, 2 vectors, 16 B "
             "per lane, one pass, nt loads and stores, second write stream rotated); the other "
             "rows are velograd_stream_probe_shape.", "",
             "| pattern | block | vectors/thread | B/lane | grid | loads | stores | rotate | "
             "code | µs | TB/s |", "|---|---:|---:|---:|---|---|---|---|---|---:|---:|"]
    summary = []
    for name, nr, nw in PROBE_PATTERNS:
        nstreams = nr + nw
        results = []

        def run(block, vpt, lane, wpc, flags):
            us = time_shape(nr, nw, block, vpt, lane, wpc, flags)
            tbs = nstreams * nbytes / (us * 1e-6) / 1e12
            results.append((us, block, vpt, lane, wpc, flags))
            lines.append(f"| {name} | {block} | {vpt} | {lane} | "
                         f"{'one pass' if wpc == 0 else f'{wpc}/CU persistent'} | "
                         f"{'nt' if flags & 1 else 'plain'} | {'nt' if flags & 2 else 'plain'} | "
                         f"{'yes' if (flags & 4 and nw == 2 and vpt >= 2) else '-'} | "
                         f"{'flat' if flags & 8 else 'guarded'} | {us:.2f} | {tbs:.3f} |")
            print(lines[-1], file=sys.stderr, flush=True)  # progress; the table goes to stdout

        bench_us = time_shape(nr, nw, **base, pattern=fixed_pattern[name])
        results.append((bench_us, 256, 2, 16, 0, 7))
        lines.append(f"| {name} | 256 | 2 | 16 | one pass | nt | nt | "
                     f"{'yes' if nw == 2 else '-'} | the bench's ceiling kernel | "
                     f"{bench_us:.2f} | {nstreams * nbytes / (bench_us * 1e-6) / 1e12:.3f} |")
        print(lines[-1], file=sys.stderr, flush=True)
        for style in (0, 8):
            for block in (256, 512, 1024):
                for vpt in (1, 2, 4):
                    for lane in (16, 32):
                        run(block, vpt, lane, 0, 7 | style)
        one_pass_best = min(results, key=lambda r: r[0])
        for shape in {(256, 2, 16, 7), (one_pass_best[1], one_pass_best[2], one_pass_best[3],
                                         one_pass_best[5])}:
            for wpc in (1, 2, 4, 8):
                if shape[0] * wpc <= 2048:
                    run(shape[0], shape[1], shape[2], wpc, shape[3])
        for flags in (6, 5, 4):
            run(256, 2, 16, 0, flags)
        if nw == 2:
            run(256, 2, 16, 0, 3)
        best = min(results, key=lambda r: r[0])
        summary.append(f"| {name} | {bench_us:.2f} | {nstreams * nbytes / (bench_us * 1e-6) / 1e12:.3f} | "
                       f"{best[0]:.2f} | {nstreams * nbytes / (best[0] * 1e-6) / 1e12:.3f} | "
                       f"{best[1]} thr, {best[2]} vec, {best[3]} B/lane, "
                       f"{'one pass' if best[4] == 0 else f'{best[4]}/CU'}, "
                       f"{'flat' if best[5] & 8 else 'guarded'}, flags {best[5] & 7} |")
    out = lines + ["", "| pattern | bench shape µs | TB/s | best µs | TB/s | best shape |",
                   "|---|---:|---:|---:|---:|---|"] + summary
    return "\n".join(out)


ROW_SCALING_ROWS = (4096, 8192, 16384, 32768, 65536)


def row_scaling(d: int = 4096, rows_list=ROW_SCALING_ROWS, rounds: int = 3) -> str:
    """The forward, the backward (with and without dweight) and the streaming probes of their
    byte patterns over a range of row counts at one width (bf16): per kernel the best of
    `rounds` batches of 10 back-to-back launches over rotating buffer sets of at least 1.5 GiB,
    then per row count what the deterministic dweight reduction adds to the backward and each
    kernel's time against its pattern's probe.  Returns a markdown table."""
    import ctypes

    import torch

    from velograd_amd import _lib
    from velograd_amd import kernels as vk
    from velograd_amd.build import PROBE_LIB_PATH

    lib = _lib.load()
    plib = ctypes.CDLL(PROBE_LIB_PATH)
    probe = plib.velograd_stream_probe
    probe.restype = ctypes.c_int32
    probe.argtypes = [ctypes.c_int32] + [ctypes.c_void_p] * 4 + [ctypes.c_int64, ctypes.c_void_p]
    shape = plib.velograd_stream_probe_shape
    shape.restype = ctypes.c_int32
    shape.argtypes = ([ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p,
                       ctypes.c_int64] + [ctypes.c_int32] * 5 + [ctypes.c_void_p])
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream
    code = _lib.DTYPE_BF16
    fwd_fn, bwd_fn = lib.velograd_rmsnorm_residual_fwd, lib.velograd_rmsnorm_residual_bwd
    names = ("forward", "2R2W probe", "backward", "backward, no dweight", "2R1W probe",
             "2R1W best shape")
    table = {}
    for rows in rows_list:
        tb = rows * d * 2
        nsets = max(4, -(-(3 << 29) // (4 * tb)))
        ws_bytes = vk.bwd_workspace_bytes(rows, d, dev)
        sets = []
        for _ in range(nsets):
            b = {k: torch.randn(rows, d, device=dev).to(torch.bfloat16) for k in ("x", "r", "g")}
            for k in ("y", "h", "dx"):
                b[k] = torch.empty(rows, d, device=dev, dtype=torch.bfloat16)
            b["w"] = (1 + 0.1 * torch.randn(d, device=dev)).to(torch.bfloat16)
            b["inv"] = torch.empty(rows, device=dev)
            b["dw"] = torch.empty(d, device=dev)
            b["ws"] = torch.empty(max(ws_bytes, 16), device=dev, dtype=torch.uint8)
            sets.append(b)
        p = {k: [b[k].data_ptr() for b in sets] for k in sets[0]}
        n16 = tb // 16
        ptrs = [((ctypes.c_void_p * 3)(p["g"][i], p["h"][i], 0),
                 (ctypes.c_void_p * 2)(p["dx"][i], 0)) for i in range(nsets)]

        def fwd(i):
            return fwd_fn(p["x"][i], p["r"][i], p["w"][i], p["y"][i], p["h"][i], p["inv"][i],
                          rows, d, d, d, d, d, code, code, 1e-5, sp)

        def bwd(i, dw=True):
            return bwd_fn(p["g"][i], p["h"][i], 1, p["w"][i], p["inv"][i], None, p["dx"][i], None,
                          p["dw"][i] if dw else None, p["ws"][i], ws_bytes, rows, d, d, d, d, d,
                          d, code, code, sp)

        def best2r1w(i):
            rd, wr = ptrs[i]
            return shape(2, 1, ctypes.cast(rd, ctypes.c_void_p), ctypes.cast(wr, ctypes.c_void_p),
                         n16, 256, 4, 16, 0, 7 | 8, sp)

        fns = (fwd,
               lambda i: probe(1, p["x"][i], p["r"][i], p["y"][i], p["h"][i], n16, sp),
               bwd, lambda i: bwd(i, False),
               lambda i: probe(2, p["g"][i], p["h"][i], p["dx"][i], None, n16, sp),
               best2r1w)
        for i in range(nsets):
            _lib.check(fwd(i), "row scaling forward")
        for name, fn in zip(names, fns):
            best = float("inf")
            for _ in range(rounds):
                evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                       for _ in range(9)]
                torch.cuda.synchronize()
                rc = 0
                for bi, (e0, e1) in enumerate(evs):
                    e0.record(stream)
                    for j in range(10):
                        rc |= fn((bi * 10 + j) % nsets)
                    e1.record(stream)
                torch.cuda.synchronize()
                if rc != 0:
                    raise RuntimeError(f"row scaling {name} at {rows} rows failed: rc {rc}")
                best = min(best, statistics.fmean(e0.elapsed_time(e1) * 100.0
                                                  for e0, e1 in evs[1:]))
            table[(name, rows)] = best
            print(f"rows {rows} {name}: {best:.2f} us", file=sys.stderr, flush=True)
        del sets
        torch.cuda.empty_cache()

    lines = [f"Row scaling at dim {d} bf16: µs per launch (best of {rounds} batches of 10 "
             "back-to-back launches, rotating buffer sets of at least 1.5 GiB).", "",
             "| kernel | " + " | ".join(f"{r} rows" for r in rows_list) + " |",
             "|---|" + "---:|" * len(rows_list)]
    for name in names:
        lines.append(f"| {name} | " + " | ".join(f"{table[(name, r)]:.2f}" for r in rows_list)
                     + " |")
    if rows_list:
        lines.append("")
        lines.append("| rows | backward − backward without dweight (µs) | backward without "
                     "dweight / 2R1W probe | forward / 2R2W probe |")
        lines.append("|---:|---:|---:|---:|")
        for r in rows_list:
            lines.append(f"| {r} | {table[('backward', r)] - table[('backward, no dweight', r)]:.2f}"
                         f" | {table[('backward, no dweight', r)] / table[('2R1W probe', r)]:.3f}"
                         f" | {table[('forward', r)] / table[('2R2W probe', r)]:.3f} |")
    return "\n".join(lines)


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus "
              f"{args.gpus}", file=sys.stderr)
        return 2
    if args.probe_sweep:
        print(probe_sweep(args.config), flush=True)
        return 0
    if args.row_scaling:
        print(row_scaling(), flush=True)
        return 0

    import torch

    from velograd_amd import _lib

    lib = _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    rows, d, eps, with_bwd = CONFIGS[args.config]
    m = measure(lib, args.config, args.steps, args.warmup, args.sets, args.kernel_events,
                stream)
    sets, fwd_args, bwd_args = m.pop("_sets"), m.pop("_fwd_args"), m.pop("_bwd_args")
    fwd_fn = lib.velograd_rmsnorm_residual_fwd
    bwd_fn = lib.velograd_rmsnorm_residual_bwd
    s, code = m.pop("_s"), m.pop("_code")
    dt = torch.bfloat16 if s == 2 else torch.float32
    value, ms_per_step = m.pop("value"), m.pop("ms_per_step")
    fb, bb = m["fwd_bytes"], m.get("bwd_bytes", 0)
    mean_fwd_ms = m["fwd_us_mean"] * 1e-3
    extra = m
    if with_bwd:
        # the backward (stage 1 + stage 2, one entry-point call) against the same roofline
        bw_gbs = bb / (m["bwd_us_mean"] * 1e-6) / 1e9
        extra["roofline_bwd"] = {
            "bound": "hbm", "kernel": "bwd_ring_kernel + dweight_reduce_kernel",
            "achieved": round(bw_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(bw_gbs / HBM_PEAK_GBS, 4), "traffic": load_traffic(args.config, "bwd"),
            "us_mean": m["bwd_us_mean"], "us_event_median": m["bwd_us_event_median"]}
        gh_gbs = m["bwd_grad_h_bytes"] / (m["bwd_grad_h_us_mean"] * 1e-6) / 1e9
        extra["roofline_bwd_grad_h"] = {
            "bound": "hbm", "kernel": "bwd_ring_kernel (grad_h) + dweight_reduce_kernel",
            "achieved": round(gh_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gh_gbs / HBM_PEAK_GBS, 4),
            "traffic": load_traffic(args.config, "bwd_grad_h"),
            "us_mean": m["bwd_grad_h_us_mean"]}
    cpu_inputs = None
    if args.cpu_seconds > 0:
        b0 = sets[0]
        cpu_inputs = tuple(b0[k].float().cpu().numpy() for k in ("x", "res", "w"))
        cpu_inputs += (b0["g"].float().cpu().numpy() if with_bwd else None,)

    if not args.no_copy_ceiling:
        ceil = stream_ceilings(sets, rows * d * s, stream)
        extra.update(ceil)
        if ceil:
            # A step whose forward and backward each ran at their pattern's probe speed.
            t_ideal = fb / (ceil["ceiling_fwd_pattern_gbs"] * 1e9)
            if with_bwd:
                t_ideal += bb / (ceil["ceiling_bwd_pattern_gbs"] * 1e9)
            extra["ceiling_step_gbs"] = round((fb + bb) / t_ideal / 1e9, 1)
            extra["frac_of_ceiling"] = round(value / extra["ceiling_step_gbs"], 4)
            if with_bwd:
                # the same step with the backward's bytes moved at the best 2R1W shape's speed
                # and no dweight reduction: what any kernel of this byte mix could reach
                t_best = (fb / (ceil["ceiling_fwd_pattern_gbs"] * 1e9)
                          + bb / (ceil["ceiling_bwd_pattern_best_shape_gbs"] * 1e9))
                extra["ceiling_step_best_shapes_gbs"] = round((fb + bb) / t_best / 1e9, 1)
                extra["ceiling_step_best_shapes_pct_peak"] = round(
                    100.0 * (fb + bb) / t_best / 1e9 / HBM_PEAK_GBS, 2)
            if with_bwd and "roofline_bwd_grad_h" in extra:
                extra["roofline_bwd_grad_h"]["frac_of_3r1w_probe"] = round(
                    extra["roofline_bwd_grad_h"]["achieved"] / ceil["ceiling_grad_h_pattern_gbs"],
                    4)

    # Warm-MALL figure (informational): the same step repeated on one buffer set, whose
    # 768 MiB exceed the 256 MiB MALL only partly.
    torch.cuda.synchronize()
    tw0 = time.perf_counter()
    for _ in range(50):
        rc = fwd_fn(*fwd_args[0])
        if with_bwd:
            rc |= bwd_fn(*bwd_args[0])
    torch.cuda.synchronize()
    extra["warm_one_set_step_us"] = round((time.perf_counter() - tw0) * 1e6 / 50, 2)
    _lib.check(rc, "warm steps")
    extra["warm_one_set_gbs"] = round((fb + bb) / (extra["warm_one_set_step_us"] * 1e-6) / 1e9, 1)

    if not args.no_fp8:
        extra.update(fp8_forward_timing(lib, sets, rows, d, s, code, eps, stream))
        if d % 32 == 0:
            extra.update(mx_forward_timing(lib, sets, rows, d, s, code, eps, stream))
    if not args.no_rope:
        extra.update(rope_timing(lib, rows, stream, norm_rope=not args.no_norm_rope,
                                 hid=args.norm_rope_dim))
        # the interleaved RoPE and the fused norm + RoPE move one read and one write stream of
        # [rows, hid] bf16: against the same run's copy probe when that moved tensors of this size
        if "ceiling_copy_gbs" in extra and rows * args.norm_rope_dim * 2 == rows * d * s:
            for key in ("rope_interleaved", "norm_rope_fused"):
                if f"{key}_gbs" in extra:
                    extra[f"{key}_frac_of_copy_probe"] = round(
                        extra[f"{key}_gbs"] / extra["ceiling_copy_gbs"], 4)
    if not args.no_torch_baseline:
        extra.update(torch_eager_timing(sets, rows, d, s, eps, with_bwd, stream))
        extra["speedup_vs_torch_eager"] = round(
            extra["torch_eager_step_us"] / (ms_per_step * 1e3), 3)
        extra["reference_benchmark_shapes"] = reference_benchmark_shapes(stream)
    if not args.no_decode:
        extra["config_E_decode"] = decode_latency(lib, stream, max(10, args.decode_calls))
    if not args.no_other_configs:
        del sets, fwd_args, bwd_args
        torch.cuda.empty_cache()
        extra["other_configs"] = other_configs(lib, args.config, stream)

    cpu = None
    if cpu_inputs is not None:
        cpu = cpu_baseline(rows, d, s, eps, args.cpu_seconds, with_bwd, cpu_inputs)
        del cpu_inputs

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if dt == torch.bfloat16 else "f32",
        "data": "synthetic",
        "config": {
            "workload": (f"config {args.config}: fused RMSNorm+residual "
                         f"{'fwd+bwd' if with_bwd else 'fwd'}, {rows}x{d} "
                         f"{'bf16' if s == 2 else 'fp32'}, eps {eps}, "
                         + ("x,residual ~ N(0,2) with 0.1% x50 outliers, grad_y ~ N(0,1)"
                            if args.config == "D" else "x,residual,grad_y ~ N(0,1)")
                         + f", weight 1+0.1N(0,1), {args.sets} rotating buffer sets"),
            "rows": rows,
            "dim": d,
            "algorithmic_bytes_per_step": fb + bb,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "fwd_vec_kernel",
            "achieved": round(fb / (mean_fwd_ms * 1e-3) / 1e9, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(fb / (mean_fwd_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "traffic": load_traffic(args.config),
            "traffic_source": traffic_source(args.config),
            "us_mean": m["fwd_us_mean"],
            "launches": m["batched_launches"],
        },
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
