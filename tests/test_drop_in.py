"""velograd_amd.drop_in: routing a reference-shaped `velograd.kernels` module to this build
without editing it.  The reference package itself is not imported (it is read, not run); a
stand-in module with the reference's names (python/velograd/kernels/__init__.py:10-48,
fused.py:28-130) records which implementation each call reaches."""

import types

import numpy as np
import pytest
import torch

from velograd_amd import drop_in
from velograd_amd import kernels as vk

NAMES = ["fused_rmsnorm_residual_forward", "fused_rmsnorm_residual_backward",
         "fused_rope_forward", "fused_rmsnorm_residual", "fused_rope"]


def _stand_in():
    """A package module and its `fused` submodule whose functions return ("reference", name,
    args, kwargs) and count their calls."""
    calls = []
    pkg = types.ModuleType("velograd.kernels")
    fused = types.ModuleType("velograd.kernels.fused")

    def make(name):
        def f(*args, **kwargs):
            calls.append(name)
            return ("reference", name, args, kwargs)
        f.__name__ = name
        return f

    for name in NAMES:
        setattr(pkg, name, make(name))
    for name in NAMES[:3]:
        setattr(fused, name, make(name))
    pkg.fused = fused
    pkg.fused_streaming_cross_entropy = make("fused_streaming_cross_entropy")
    return pkg, calls


def test_install_routes_every_replaced_name_once_and_uninstall_restores():
    pkg, _ = _stand_in()
    before = {n: getattr(pkg, n) for n in NAMES}
    done = drop_in.install(pkg)
    assert sorted(done) == sorted([f"velograd.kernels.{n}" for n in NAMES] +
                                  [f"velograd.kernels.fused.{n}" for n in NAMES[:3]])
    assert drop_in.install(pkg) == []                     # idempotent
    for n in NAMES:
        assert getattr(pkg, n) is not before[n]
        assert getattr(pkg, n).__name__ == n              # functools.wraps keeps the name
    # a name this build does not replace is untouched
    assert pkg.fused_streaming_cross_entropy.__name__ == "fused_streaming_cross_entropy"
    assert not hasattr(pkg.fused_streaming_cross_entropy, "__velograd_amd_original__")
    assert len(drop_in.uninstall(pkg)) == len(done)
    for n in NAMES:
        assert getattr(pkg, n) is before[n]


def test_host_inputs_keep_the_reference_path():
    pkg, calls = _stand_in()
    drop_in.install(pkg)
    x = np.ones((2, 8), np.float32)
    out = pkg.fused_rmsnorm_residual_forward(x, None, None, 1e-6)
    assert out[:2] == ("reference", "fused_rmsnorm_residual_forward") and out[2][0] is x
    assert pkg.fused.fused_rope_forward(x, None, head_dim=8)[1] == "fused_rope_forward"
    t = torch.ones(2, 8)                                    # a CPU tensor is host data too
    assert pkg.fused_rmsnorm_residual(t)[0] == "reference"
    assert pkg.fused_rope(x=t)[0] == "reference"            # the route argument by keyword
    assert pkg.fused_rmsnorm_residual_backward([1.0], [1.0], None, [1.0])[0] == "reference"
    assert calls == ["fused_rmsnorm_residual_forward", "fused_rope_forward",
                     "fused_rmsnorm_residual", "fused_rope", "fused_rmsnorm_residual_backward"]


def test_install_without_the_reference_package_says_so(monkeypatch):
    import builtins
    real_import = builtins.__import__

    def no_velograd(name, *args, **kwargs):
        if name == "velograd.kernels" or name.startswith("velograd."):
            raise ImportError(name)
        return real_import(name, *args, **kwargs)

    monkeypatch.setattr(builtins, "__import__", no_velograd)
    with pytest.raises(ImportError, match="pass its kernels module explicitly"):
        drop_in.install()


@pytest.mark.gpu
def test_device_tensors_reach_the_hip_kernels():
    pkg, calls = _stand_in()
    drop_in.install(pkg)
    torch.manual_seed(3)
    x = torch.randn(64, 4096, device="cuda", dtype=torch.bfloat16)
    r = torch.randn(64, 4096, device="cuda", dtype=torch.bfloat16)
    w = (1 + 0.1 * torch.randn(4096, device="cuda")).to(torch.bfloat16)
    y, h, inv = pkg.fused_rmsnorm_residual_forward(x, r, w, 1e-5)
    y2, h2, inv2 = vk.fused_rmsnorm_residual_forward(x, r, w, 1e-5)
    assert torch.equal(y, y2) and torch.equal(h, h2) and torch.equal(inv, inv2)
    assert torch.equal(pkg.fused_rmsnorm_residual(x, r, w, 1e-5), y2)
    g = torch.randn_like(x)
    dx, dw = pkg.fused_rmsnorm_residual_backward(g, h * inv.to(h.dtype), w, inv)
    dx2, dw2 = vk.fused_rmsnorm_residual_backward(g, h * inv.to(h.dtype), w, inv)
    assert torch.equal(dx, dx2) and torch.equal(dw, dw2)
    q = torch.randn(16, 4, 64, device="cuda")
    assert torch.equal(pkg.fused.fused_rope_forward(q, None, head_dim=64)[0],
                       vk.fused_rope_forward(q, None, head_dim=64)[0])
    assert torch.equal(pkg.fused_rope(q, head_dim=64), vk.fused_rope(q, head_dim=64))
    assert calls == []                                      # the reference path never ran
