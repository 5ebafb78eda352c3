"""The C ABI from plain C++ without torch: tests/c_abi_check.cpp (built with the library by
velograd_amd.build) allocates with hipMalloc, launches the forward and the backward on a stream
of its own and checks them against a double-precision restatement of fused.py:28-66."""

import os
import subprocess

import pytest

from velograd_amd.build import C_ABI_CHECK_BIN

pytestmark = pytest.mark.gpu


def test_c_abi_from_plain_cpp():
    print("c_abi_check (plain C++, hipMalloc buffers, own stream)", flush=True)
    if not os.path.exists(C_ABI_CHECK_BIN):
        pytest.fail(f"{C_ABI_CHECK_BIN} is not built (python -c 'import __graft_entry__ as g; "
                    "g.build()')")
    r = subprocess.run([C_ABI_CHECK_BIN], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "c_abi ok" in r.stdout
