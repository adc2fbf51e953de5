"""The torch.library registration (CPU): the custom ops exist and their fake
kernels give the shapes and dtypes the native entry points return, so
torch.compile can trace graphs around them without a GPU."""

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import gfx1010_kernels  # noqa: F401  (registers the ops)


def test_ops_are_registered():
    assert hasattr(torch.ops.gfx1010_kernels, "rln_forward")
    assert hasattr(torch.ops.gfx1010_kernels, "rln_backward")


@pytest.mark.parametrize("shape", [(7, 128), (2, 5, 768), (1, 1, 1, 1024)])
@pytest.mark.parametrize("branch_dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("dropout_p,training", [(0.0, True), (0.1, True), (0.1, False)])
def test_fake_shapes(shape, branch_dtype, dropout_p, training):
    hidden = shape[-1]
    rows = 1
    for size in shape[:-1]:
        rows *= size
    with FakeTensorMode():
        x = torch.empty(shape, device="cuda")
        branch = torch.empty(shape, device="cuda", dtype=branch_dtype)
        weight = torch.empty(hidden, device="cuda")
        bias = torch.empty(hidden, device="cuda")
        updated, normalized, mean, rstd, mask = torch.ops.gfx1010_kernels.rln_forward(
            x, branch, weight, bias, dropout_p, 1e-5, training)
        assert updated.shape == normalized.shape == x.shape
        assert updated.dtype == normalized.dtype == torch.float32
        half = torch.ops.gfx1010_kernels.rln_forward(
            x, branch, weight, bias, dropout_p, 1e-5, training, torch.bfloat16)[1]
        assert half.shape == x.shape and half.dtype == torch.bfloat16
        assert mean.shape == rstd.shape == (rows,)
        dropping = training and dropout_p > 0.0
        assert mask.shape == ((rows * hidden // 32,) if dropping else (0,))
        assert mask.dtype == torch.int32
        grads = torch.ops.gfx1010_kernels.rln_backward(
            x, None, updated, weight, mean, rstd, mask, dropout_p, training, branch_dtype)
        grad_x, grad_branch, grad_weight, grad_bias = grads
        assert grad_x.shape == grad_branch.shape == x.shape
        assert grad_x.dtype == torch.float32 and grad_branch.dtype == branch_dtype
        assert grad_weight.shape == grad_bias.shape == (hidden,)
