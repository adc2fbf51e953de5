"""Half-precision interfaces on the GPU: a bfloat16 branch and a float16 /
bfloat16 ``normalized`` output with its matching half-precision upstream
gradient (extensions beyond the reference's fp32 output and fp16/fp32
branch). Parity is against the fp64 oracle evaluated on exactly the values
the kernels read: the half ``normalized`` lies within one ulp of its dtype,
every fp32 quantity within the usual tolerances.
"""

import pytest
import torch

from gfx1010_kernels import _C, residual_layer_norm
from oracle import rln_oracle as oracle
from parity import (
    REFERENCE_THREADS,
    SPECIALIZED_HIDDEN_SIZES,
    assert_bitwise,
    check_backward,
    check_forward,
    generator_state,
    host,
    make_grads,
    make_inputs,
)

pytestmark = pytest.mark.gpu
HALF = [torch.float16, torch.bfloat16]
BRANCHES = [torch.float16, torch.bfloat16, torch.float32]


@pytest.mark.parametrize("hidden", SPECIALIZED_HIDDEN_SIZES)
@pytest.mark.parametrize("normalized_dtype", HALF, ids=["f16", "bf16"])
@pytest.mark.parametrize("branch_dtype", BRANCHES, ids=["b16", "bbf16", "b32"])
def test_half_normalized_forward_and_backward(hidden, normalized_dtype, branch_dtype):
    rows = 29
    inputs = make_inputs((rows, hidden), branch_dtype, seed=hidden + 3)
    grad_updated, grad_normalized = make_grads((rows, hidden), seed=hidden + 4)
    grad_normalized = grad_normalized.to(normalized_dtype)
    torch.cuda.manual_seed(hidden)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, 0.1, 1e-5, True, 128,
                                             normalized_dtype=normalized_dtype)
    assert outputs[1].dtype == normalized_dtype
    keep, scale = check_forward(outputs, inputs, 0.1, True, 1e-5, seed, offset,
                                f"H={hidden}")
    gradients = _C.residual_layer_norm_backward(
        grad_updated, grad_normalized, outputs[0], inputs[2], outputs[2], outputs[3],
        outputs[4], 0.1, True, branch_dtype == torch.float16, 128, 64, 64, 1, True,
        branch_dtype=branch_dtype)
    assert gradients[1].dtype == branch_dtype
    check_backward(gradients, grad_updated, grad_normalized, outputs[0], inputs[2], 1e-5, keep,
                   scale, f"H={hidden}")


@pytest.mark.parametrize("normalized_dtype", [None, *HALF], ids=["f32", "f16", "bf16"])
def test_public_api_autograd_with_half_output(normalized_dtype):
    rows, hidden = 40, 768
    inputs = make_inputs((rows, hidden), torch.bfloat16, seed=8)
    leaves = [t.detach().clone().requires_grad_(True) for t in inputs]
    torch.cuda.manual_seed(9)
    seed, offset = generator_state()
    updated, normalized = residual_layer_norm(
        *leaves, dropout_p=0.2, implementation="gfx950", normalized_dtype=normalized_dtype)
    assert normalized.dtype == (normalized_dtype or torch.float32)
    grad_updated, grad_normalized = make_grads((rows, hidden), seed=10)
    grad_normalized = grad_normalized.to(normalized.dtype)
    torch.autograd.backward((updated, normalized), (grad_updated, grad_normalized))
    torch.cuda.synchronize()
    keep_words = oracle.reference_mask_words(
        rows, hidden, REFERENCE_THREADS[hidden], seed, offset, oracle.dropout_constants(0.2)[2])
    keep = oracle.decode_mask(keep_words, rows, hidden)
    _, scale, _ = oracle.dropout_constants(0.2)
    expected = oracle.forward(host(inputs[0]), host(inputs[1]), host(inputs[2]),
                              host(inputs[3]), 1e-5, keep=keep, scale=scale, branch_type="bf16")
    assert_bitwise(host(updated), expected["updated"], "updated")
    check_backward((leaves[0].grad, leaves[1].grad, leaves[2].grad, leaves[3].grad),
                   grad_updated, grad_normalized, updated, inputs[2], 1e-5, keep, scale,
                   "public")
    assert leaves[1].grad.dtype == torch.bfloat16


def test_torch_implementation_honours_normalized_dtype():
    inputs = make_inputs((6, 256), torch.float32, seed=1)
    updated, normalized = residual_layer_norm(*inputs, implementation="torch",
                                              normalized_dtype=torch.bfloat16)
    assert normalized.dtype == torch.bfloat16 and updated.dtype == torch.float32


@pytest.mark.parametrize("dropout_p", [0.0, 0.3])
def test_misaligned_bfloat16_branch_matches_aligned(dropout_p):
    rows, hidden = 33, 512
    x, branch, weight, bias = make_inputs((rows, hidden), torch.bfloat16, seed=12)
    storage = torch.empty(rows * hidden + 1, device="cuda", dtype=torch.bfloat16)
    misaligned = storage[1:].view(rows, hidden)
    misaligned.copy_(branch)
    assert misaligned.data_ptr() % 8 != 0
    torch.cuda.manual_seed(3)
    aligned = _C.residual_layer_norm_forward(x, branch, weight, bias, dropout_p, 1e-5, True, 128,
                                             normalized_dtype=torch.bfloat16)
    torch.cuda.manual_seed(3)
    element = _C.residual_layer_norm_forward(x, misaligned, weight, bias, dropout_p, 1e-5, True,
                                             128, normalized_dtype=torch.bfloat16)
    for a, b in zip(aligned, element):
        assert_bitwise(host(b), host(a), "misaligned bf16")


def test_rejects_unsupported_normalized_dtype():
    inputs = make_inputs((4, 128), torch.float16, seed=1)
    with pytest.raises(RuntimeError, match="normalized_dtype must be"):
        _C.residual_layer_norm_forward(*inputs, 0.0, 1e-5, True, 128,
                                       normalized_dtype=torch.float64)
    with pytest.raises(ValueError, match="normalized_dtype must be"):
        residual_layer_norm(*inputs, normalized_dtype=torch.float64)
