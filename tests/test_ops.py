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


def _forward_nodes(graph):
    return [node for node in graph.nodes
            if node.op == "call_function" and "rln_forward" in str(node.target)]


@pytest.mark.parametrize("dropout_p", [0.1, 0.0])
def test_two_equal_calls_survive_common_subexpression_elimination(dropout_p):
    """Two calls with equal arguments draw two masks eagerly (the op reserves
    Philox offsets each time it runs), so a compiled graph must keep both.
    The graph is traced from fake CUDA tensors and put through AOTAutograd's
    common-subexpression pass (which it runs on the joint forward/backward
    graph of a training step), the pass that merged them while the op had no
    per-call input."""
    from torch._functorch.compile_utils import fx_graph_cse
    from torch.fx.experimental.proxy_tensor import make_fx

    from gfx1010_kernels._ops import residual_layer_norm_op

    def two_calls(x, branch, weight, bias):
        first = residual_layer_norm_op(x, branch, weight, bias, dropout_p, 1e-5, True)
        second = residual_layer_norm_op(x, branch, weight, bias, dropout_p, 1e-5, True)
        return (*first, *second)

    with FakeTensorMode():
        x = torch.empty(6, 768, device="cuda")
        branch = torch.empty(6, 768, device="cuda", dtype=torch.float16)
        weight = torch.empty(768, device="cuda")
        bias = torch.empty(768, device="cuda")
        module = make_fx(two_calls, tracing_mode="fake")(x, branch, weight, bias)
    assert len(_forward_nodes(module.graph)) == 2
    assert len(_forward_nodes(fx_graph_cse(module.graph))) == 2
