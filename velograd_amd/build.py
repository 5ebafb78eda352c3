"""Build of the gfx950 HIP library `velograd_amd/lib/libvelograd_kernels.so`.

The library is compiled in-tree with hipcc (no torch extension machinery, no hipify) so the
same `.so` file travels with the source tree to the GPU host.  `python -m velograd_amd.build`
runs it from the command line.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
# Translation units of the kernels library (one .so).
SRCS = [os.path.join(PKG_DIR, "csrc", name) for name in ("rmsnorm_residual.hip", "rope.hip")]
PROBE_SRC = os.path.join(PKG_DIR, "csrc", "stream_probe.hip")
INCLUDE_DIR = os.path.join(REPO_DIR, "include")
CSRC_DIR = os.path.join(PKG_DIR, "csrc")
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libvelograd_kernels.so")
# Bench-only helper (same-run HBM ceiling); not part of the kernels' C ABI.
PROBE_LIB_PATH = os.path.join(LIB_DIR, "libvelograd_stream_probe.so")

OFFLOAD_ARCH = "gfx950"

# Plain C++ check of the C ABI without torch (tests/c_abi_check.cpp, run by a GPU test): host
# code only, linked against the kernels library and the HIP runtime.
C_ABI_CHECK_SRC = os.path.join(REPO_DIR, "tests", "c_abi_check.cpp")
C_ABI_CHECK_BIN = os.path.join(REPO_DIR, "tests", "_build", "c_abi_check")

# Host-only pybind11 binding of the forward's fast path to torch tensors (a CPython extension
# module next to the package's Python files).  Optional at run time: without it the ctypes path
# runs the same kernels.
FASTPATH_SRC = os.path.join(PKG_DIR, "csrc", "torch_fastpath.cpp")

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={OFFLOAD_ARCH}",
    "-fPIC",
    "-shared",
    "-fvisibility=hidden",
    # Mirror the reference's rounding points exactly: no implicit multiply-add fusion.
    "-ffp-contract=off",
    # No packed-fp32 VALU instructions in the device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def find_hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain (ROCm) is required to build")


def _hipcc(srcs, out: str, verbose: bool) -> None:
    tmp = out + ".tmp"
    cmd = [find_hipcc(), *HIPCC_FLAGS, "-I", INCLUDE_DIR, "-I", CSRC_DIR, *srcs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(
            "hipcc failed (exit %d):\n%s\n%s" % (proc.returncode, proc.stdout, proc.stderr)
        )
    os.replace(tmp, out)


def fastpath_path() -> str:
    import sysconfig
    return os.path.join(PKG_DIR, "_fastpath" + sysconfig.get_config_var("EXT_SUFFIX"))


def build_fastpath(verbose: bool = False) -> str:
    """Compile the torch-tensor fast path against the installed torch (host C++, g++)."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    out = fastpath_path()
    tmp = out + ".tmp"
    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-shared", "-fPIC",
           "-fvisibility=hidden", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-DTORCH_EXTENSION_NAME=_fastpath", "-DTORCH_API_INCLUDE_EXTENSION_H",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           "-I", INCLUDE_DIR, "-I", sysconfig.get_paths()["include"]]
    for inc in cpp_extension.include_paths(device_type="cuda"):
        cmd += ["-I", inc]
    cmd += [FASTPATH_SRC, "-o", tmp,
            "-L", LIB_DIR, "-lvelograd_kernels", "-Wl,-rpath,$ORIGIN/lib",
            "-L", torch_lib, "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
            "-ltorch_hip", f"-Wl,-rpath,{torch_lib}"]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(
            "fast-path build failed (exit %d):\n%s\n%s" % (proc.returncode, proc.stdout, proc.stderr))
    os.replace(tmp, out)
    return out


def build_c_abi_check(verbose: bool = False) -> str:
    """Compile tests/c_abi_check.cpp against the built library (host C++ through hipcc)."""
    out = C_ABI_CHECK_BIN
    os.makedirs(os.path.dirname(out), exist_ok=True)
    tmp = out + ".tmp"
    rel = os.path.relpath(LIB_DIR, os.path.dirname(out))
    cmd = [find_hipcc(), "-O2", "-std=c++17", "-Wall", "-I", INCLUDE_DIR, C_ABI_CHECK_SRC,
           "-o", tmp, "-L", LIB_DIR, "-lvelograd_kernels", f"-Wl,-rpath,$ORIGIN/{rel}"]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(
            "C ABI check build failed (exit %d):\n%s\n%s" % (proc.returncode, proc.stdout,
                                                              proc.stderr))
    os.replace(tmp, out)
    return out


def build_library(verbose: bool = False) -> str:
    """Compile the kernels (and the bench's stream probe) for gfx950, then the torch-tensor
    fast path and the plain C++ ABI check; return the kernels' .so."""
    os.makedirs(LIB_DIR, exist_ok=True)
    _hipcc(SRCS, LIB_PATH, verbose)
    _hipcc([PROBE_SRC], PROBE_LIB_PATH, verbose)
    build_fastpath(verbose)
    build_c_abi_check(verbose)
    return LIB_PATH


if __name__ == "__main__":
    print(build_library(verbose="-v" in sys.argv[1:]))
