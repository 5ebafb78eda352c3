"""velograd_amd — MI355X (gfx950) implementation of VeloGrad's fused RMSNorm + residual path.

The public surface is `velograd_amd.kernels`, which keeps the call signatures of the reference's
`velograd.kernels.fused_rmsnorm_residual{,_forward,_backward}`
(python/velograd/kernels/fused.py:28-66, python/velograd/kernels/__init__.py:19-32) and runs
them on hand-written HIP kernels through the C ABI declared in include/velograd_kernels.h.
Importing this package does not load the native library; the first kernel call does.
"""

__version__ = "0.1.0"
