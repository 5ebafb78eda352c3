"""Route an imported reference package's fused kernels to this build, without editing it.

`install()` wraps, in place, the functions this build replaces in the reference's
`velograd.kernels` (python/velograd/kernels/__init__.py:10-48) and in its `fused` submodule
(python/velograd/kernels/fused.py:28-130).  A call whose leading tensor argument is a torch
tensor on the GPU runs the HIP kernels (`velograd_amd.kernels`); every other call runs the
reference's own function, so host callers (NumPy arrays, lists, `velograd.Tensor`) see no change.
The reference's wrappers `fused_rmsnorm_residual` and `fused_rope` look
`fused_rmsnorm_residual_forward` and `fused_rope_forward` up in their module when called, so
patching the module attributes reaches them too.  A name a caller bound earlier with
`from velograd.kernels import ...` keeps the function it bound: call `install()` before such
imports.  `uninstall()` puts the reference's functions back.
"""

import functools
from typing import Any, Callable, List, Optional

import torch

from . import kernels as _k

# reference name -> (this build's function, name of the argument that decides the route)
_ROUTES = {
    "fused_rmsnorm_residual_forward": (_k.fused_rmsnorm_residual_forward, "x"),    # fused.py:28
    "fused_rmsnorm_residual_backward": (_k.fused_rmsnorm_residual_backward, "grad_out"),  # :48
    "fused_rope_forward": (_k.fused_rope_forward, "q"),                            # fused.py:72
    "fused_rmsnorm_residual": (_k.fused_rmsnorm_residual, "x"),                    # __init__.py:19
    "fused_rope": (_k.fused_rope, "x"),                                            # __init__.py:34
}
_ORIGINAL = "__velograd_amd_original__"


def _on_device(a: Any) -> bool:
    return isinstance(a, torch.Tensor) and a.device.type == "cuda"


def _routed(original: Callable, hip: Callable, lead: str) -> Callable:
    @functools.wraps(original)
    def routed(*args, **kwargs):
        first = args[0] if args else kwargs.get(lead)
        if _on_device(first):
            return hip(*args, **kwargs)
        return original(*args, **kwargs)

    setattr(routed, _ORIGINAL, original)
    return routed


def _modules(target: Any) -> List[Any]:
    mods = [target]
    fused = getattr(target, "fused", None)
    if fused is not None and fused is not target:
        mods.append(fused)
    return mods


def _target(target: Optional[Any]) -> Any:
    if target is not None:
        return target
    try:
        import velograd.kernels as reference  # the reference package, when installed
    except ImportError as e:
        raise ImportError("velograd_amd.drop_in: the reference package velograd is not "
                          "importable; pass its kernels module explicitly") from e
    return reference


def install(target: Optional[Any] = None) -> List[str]:
    """Route `target` (default: the imported `velograd.kernels`) and its `fused` submodule to
    this build for device tensors.  Returns the qualified names newly routed; names already
    routed are left as they are, so calling it twice changes nothing."""
    done = []
    for mod in _modules(_target(target)):
        for name, (hip, lead) in _ROUTES.items():
            fn = getattr(mod, name, None)
            if fn is None or hasattr(fn, _ORIGINAL):
                continue
            setattr(mod, name, _routed(fn, hip, lead))
            done.append(f"{getattr(mod, '__name__', '?')}.{name}")
    return done


def uninstall(target: Optional[Any] = None) -> List[str]:
    """Put back the functions `install` wrapped in `target` and its `fused` submodule."""
    done = []
    for mod in _modules(_target(target)):
        for name in _ROUTES:
            fn = getattr(mod, name, None)
            original = getattr(fn, _ORIGINAL, None)
            if original is not None:
                setattr(mod, name, original)
                done.append(f"{getattr(mod, '__name__', '?')}.{name}")
    return done
