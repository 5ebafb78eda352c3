"""Host-side logic of velograd_amd.kernels that needs no GPU: argument shaping and the rule that
there is no CPU fallback."""

import numpy as np
import pytest
import torch

from velograd_amd import kernels as vk


def test_no_cpu_fallback_without_gpu():
    if torch.cuda.is_available():
        pytest.skip("a ROCm device is visible")
    x = np.ones((2, 8), np.float32)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        vk.fused_rmsnorm_residual_forward(x)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        vk.fused_rmsnorm_residual(x, x, np.ones(8))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        vk.fused_rmsnorm_residual_backward(x, x, None, np.ones((2, 1), np.float32))


def test_rows_view_flattens_leading_axes():
    t = torch.zeros(3, 5, 16)
    v = vk._rows_view(t, "t")
    assert v.shape == (15, 16) and v.data_ptr() == t.data_ptr()
    assert vk._ld(v) == 16


def test_rows_view_keeps_row_stride_of_a_column_slice():
    base = torch.zeros(6, 40)
    t = base[:, :32]
    v = vk._rows_view(t, "t")
    assert v.data_ptr() == base.data_ptr() and vk._ld(v) == 40


def test_rows_view_copies_when_last_axis_is_strided():
    t = torch.zeros(16, 6).t()  # [6, 16] with stride (1, 6)
    v = vk._rows_view(t, "t")
    assert v.stride(-1) == 1 and v.shape == (6, 16)


def test_rows_view_one_dim_and_scalar():
    assert vk._rows_view(torch.zeros(9), "t").shape == (1, 9)
    with pytest.raises(ValueError):
        vk._rows_view(torch.tensor(1.0), "t")


def test_prep_weight_shapes_and_dtypes():
    dev = torch.device("cpu")
    w, code = vk._prep_weight(torch.ones(1, 8, dtype=torch.bfloat16), 8, torch.bfloat16, dev)
    assert w.shape == (8,) and code == 2
    w, code = vk._prep_weight(torch.ones(8, dtype=torch.float64), 8, torch.bfloat16, dev)
    assert w.dtype == torch.float32 and code == 0
    w, code = vk._prep_weight(None, 8, torch.float16, dev)
    assert w is None and code == 1
    with pytest.raises(ValueError):
        vk._prep_weight(torch.ones(7), 8, torch.float32, dev)


def test_dtype_rejection():
    with pytest.raises(TypeError):
        vk._dtype_code(torch.zeros(2, dtype=torch.float64), "x")
