"""Hidden sizes beyond the reference's six: every multiple of 64 up to 8192.

These sizes run kernels with a run-time row length: one wave per row up to
1024 columns (slots past the row's end idle), and 2, 4 or 8 waves per row
above that, adding their row sums through LDS. Each kernel shape is checked
against the fp64 oracle (forward, both backward reductions, fp16 / bf16 /
fp32 branch, with and without dropout), at row counts that leave blocks
partly empty, through the public API and autograd, with half-precision
output and on misaligned pointers. (The reference serves none of these sizes
natively; its tests stop at 1024, tests/test_residual_layer_norm.py:106.)
"""

import warnings

import numpy as np
import pytest
import torch

from gfx1010_kernels import _C, residual_layer_norm
from parity import (
    TOL_PARAMETER_GRAD,
    WIDE_HIDDEN_SIZES,
    assert_bitwise,
    assert_normwise,
    check_backward,
    check_forward,
    generator_state,
    host,
    make_grads,
    make_inputs,
)
from test_gpu_backward import deterministic_algorithms, raw_backward

pytestmark = pytest.mark.gpu
EPS = 1e-5


def forward_and_check(inputs, dropout_p, training, what, normalized_dtype=None):
    seed, offset = generator_state()
    extra = {} if normalized_dtype is None else {"normalized_dtype": normalized_dtype}
    outputs = _C.residual_layer_norm_forward(*inputs, dropout_p, EPS, training, 128, **extra)
    keep, scale = check_forward(outputs, inputs, dropout_p, training, EPS, seed, offset, what)
    return outputs, keep, scale


@pytest.mark.parametrize("hidden", WIDE_HIDDEN_SIZES)
@pytest.mark.parametrize("branch_dtype", [torch.float16, torch.bfloat16, torch.float32],
                         ids=["f16", "bf16", "f32"])
@pytest.mark.parametrize("dropout_p", [0.0, 0.15])
def test_wide_forward_and_backward_match_oracle(hidden, branch_dtype, dropout_p):
    rows = 37
    print(f"[wide] H={hidden} {branch_dtype} p={dropout_p}", flush=True)
    inputs = make_inputs((rows, hidden), branch_dtype, seed=31 + hidden)
    grad_updated, grad_normalized = make_grads((rows, hidden), seed=77 + hidden)
    torch.cuda.manual_seed(hidden)
    outputs, keep, scale = forward_and_check(inputs, dropout_p, True, f"H={hidden}")
    gradients = raw_backward(grad_updated, grad_normalized, outputs, inputs[2], dropout_p,
                             branch_dtype)
    check_backward(gradients, grad_updated, grad_normalized, outputs[0], inputs[2], EPS, keep,
                   scale, f"H={hidden}")
    assert gradients[1].dtype == branch_dtype


@pytest.mark.parametrize("hidden", [1280, 4096, 8192])
@pytest.mark.parametrize("rows", [1, 3, 5, 257])
def test_wide_deterministic_row_counts(hidden, rows):
    """Blocks of several rows (or one row per block) with ragged ends; the
    deterministic reduction replays bit for bit and matches the oracle."""
    print(f"[wide] deterministic H={hidden} rows={rows}", flush=True)
    inputs = make_inputs((rows, hidden), torch.float16, seed=rows + hidden)
    grad_updated, grad_normalized = make_grads((rows, hidden), seed=rows * 3 + hidden)
    torch.cuda.manual_seed(rows)
    outputs, keep, scale = forward_and_check(inputs, 0.1, True, f"H={hidden} rows={rows}")
    with deterministic_algorithms(True):
        first = raw_backward(grad_updated, grad_normalized, outputs, inputs[2], 0.1, True)
        second = raw_backward(grad_updated, grad_normalized, outputs, inputs[2], 0.1, True)
    for a, b, name in zip(first, second, ("grad_x", "grad_branch", "grad_weight", "grad_bias")):
        assert_bitwise(host(a), host(b), name)
    check_backward(first, grad_updated, grad_normalized, outputs[0], inputs[2], EPS, keep, scale,
                   f"H={hidden} rows={rows}")


@pytest.mark.parametrize("hidden", [1600, 5120])
@pytest.mark.parametrize("normalized_dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_wide_half_precision_output(hidden, normalized_dtype):
    rows = 19
    inputs = make_inputs((rows, hidden), torch.bfloat16, seed=hidden + 5)
    grad_updated, grad_normalized = make_grads((rows, hidden), seed=hidden + 6)
    grad_normalized = grad_normalized.to(normalized_dtype)
    torch.cuda.manual_seed(5)
    outputs, keep, scale = forward_and_check(inputs, 0.1, True, f"H={hidden}", normalized_dtype)
    assert outputs[1].dtype == normalized_dtype
    gradients = raw_backward(grad_updated, grad_normalized, outputs, inputs[2], 0.1,
                             torch.bfloat16)
    check_backward(gradients, grad_updated, grad_normalized, outputs[0], inputs[2], EPS, keep,
                   scale, f"H={hidden}")


@pytest.mark.parametrize("dropout_p", [0.0, 0.2])
def test_wide_misaligned_matches_aligned(dropout_p):
    rows, hidden = 23, 2560

    def shifted(tensor):
        storage = torch.empty(tensor.numel() + 1, device=tensor.device, dtype=tensor.dtype)
        view = storage[1:].view(tensor.shape)
        view.copy_(tensor)
        return view

    inputs = make_inputs((rows, hidden), torch.float16, seed=8)
    grads = make_grads((rows, hidden), seed=9)
    results = []
    for convert in (lambda t: t, shifted):
        torch.cuda.manual_seed(12)
        args = [convert(t) for t in inputs]
        outputs = _C.residual_layer_norm_forward(*args, dropout_p, EPS, True, 128)
        with deterministic_algorithms(True):
            gradients = raw_backward(*(convert(g) for g in grads), outputs, args[2], dropout_p,
                                     True)
        results.append([host(t) for t in (*outputs, *gradients)])
    for aligned, misaligned in zip(*results):
        assert_bitwise(misaligned, aligned, "misaligned")


def test_wide_public_api_autograd_without_fallback():
    """`auto` serves H = 1600 (GPT-2 XL) natively: no fallback warning, and
    autograd gradients match the oracle."""
    rows, hidden = 33, 1600
    x, branch, weight, bias = make_inputs((rows, hidden), torch.float16, seed=1600)
    grad_updated, grad_normalized = make_grads((rows, hidden), seed=1601)
    leaves = [t.clone().requires_grad_(True) for t in (x, branch, weight, bias)]
    torch.cuda.manual_seed(3)
    seed, offset = generator_state()
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        updated, normalized = residual_layer_norm(*leaves, dropout_p=0.1, eps=EPS, training=True)
    torch.autograd.backward((updated, normalized), (grad_updated, grad_normalized))

    torch.cuda.manual_seed(3)
    outputs = _C.residual_layer_norm_forward(x, branch, weight, bias, 0.1, EPS, True, 128)
    assert_bitwise(host(updated), host(outputs[0]), "updated")
    assert_bitwise(host(normalized), host(outputs[1]), "normalized")
    keep, scale = check_forward(outputs, (x, branch, weight, bias), 0.1, True, EPS, seed, offset)
    check_backward((leaves[0].grad, leaves[1].grad, leaves[2].grad, leaves[3].grad),
                   grad_updated, grad_normalized, outputs[0], weight, EPS, keep, scale,
                   "autograd")


def test_wide_large_row_count_parameter_sums():
    """Many blocks at H = 8192 (one row per block): the atomic sums match a
    float64 reduction on the device."""
    rows, hidden = 3000, 8192
    generator = torch.Generator(device="cuda").manual_seed(4)
    x = torch.randn(rows, hidden, device="cuda", generator=generator)
    branch = torch.randn(rows, hidden, device="cuda", generator=generator).half()
    weight = 1 + 0.02 * torch.randn(hidden, device="cuda", generator=generator)
    bias = 0.02 * torch.randn(hidden, device="cuda", generator=generator)
    grad_normalized = torch.randn(rows, hidden, device="cuda", generator=generator)
    outputs = _C.residual_layer_norm_forward(x, branch, weight, bias, 0.1, EPS, True, 128)
    gradients = raw_backward(None, grad_normalized, outputs, weight, 0.1, True)
    u = outputs[0].double()
    centered = u - u.mean(dim=-1, keepdim=True)
    xhat = centered / torch.sqrt((centered * centered).mean(dim=-1, keepdim=True) + EPS)
    d_weight = (grad_normalized.double() * xhat).sum(dim=0)
    d_bias = grad_normalized.double().sum(dim=0)
    assert_normwise(host(gradients[2]), host(d_weight), TOL_PARAMETER_GRAD, "grad_weight")
    assert_normwise(host(gradients[3]), host(d_bias), TOL_PARAMETER_GRAD, "grad_bias")
    assert np.isfinite(host(gradients[0])).all()
