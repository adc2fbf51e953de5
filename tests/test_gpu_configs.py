"""The BASELINE.json configurations at their full sizes.

C0, C1, the C4 tail and the C4 single row run the complete oracle. The
262 144-row configs (C2 at every hidden size, C4 large), C3 and both sides of
the 768-column backward switch are checked on every row
(parity.check_full_tensor): the whole dropout mask bitwise against the C
oracle, `updated` bitwise against its fp32 recomputation from that mask, and
normalized, mean, rstd, grad_x and grad_branch against a float64 LayerNorm and
its gradient on the device; the weight/bias gradients against a float64
reduction over all rows; C3 also replays bitwise.
"""

import contextlib

import numpy as np
import pytest
import torch

from gfx1010_kernels import _C
from parity import (
    TOL_PARAMETER_GRAD,
    assert_bitwise,
    assert_normwise,
    check_backward,
    check_forward,
    check_full_tensor,
    generator_state,
    host,
    make_grads,
    make_inputs,
)

pytestmark = pytest.mark.gpu
EPS = 1e-5


@contextlib.contextmanager
def deterministic_algorithms(enabled):
    previous = torch.are_deterministic_algorithms_enabled()
    torch.use_deterministic_algorithms(enabled)
    try:
        yield
    finally:
        torch.use_deterministic_algorithms(previous)


def device_inputs(rows, hidden, branch_dtype, seed, branch_std=1.0, x_mean=0.0):
    """Large seeded inputs generated on the device (checked there, in float64)."""
    generator = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(rows, hidden, device="cuda", generator=generator) + x_mean
    branch = (torch.randn(rows, hidden, device="cuda", generator=generator) * branch_std).to(branch_dtype)
    weight = 1.0 + 0.02 * torch.randn(hidden, device="cuda", generator=generator)
    bias = 0.02 * torch.randn(hidden, device="cuda", generator=generator)
    grad_updated = torch.randn(rows, hidden, device="cuda", generator=generator)
    grad_normalized = torch.randn(rows, hidden, device="cuda", generator=generator)
    return (x, branch, weight, bias), (grad_updated, grad_normalized)


def raw_backward(grads, outputs, weight, dropout_p, branch_is_half):
    return _C.residual_layer_norm_backward(
        grads[0], grads[1], outputs[0], weight, outputs[2], outputs[3], outputs[4], dropout_p,
        True, branch_is_half, 128, 64, 64, 1, True)


def keep_count(mask):
    table = torch.tensor([bin(i).count("1") for i in range(256)], device=mask.device)
    return int(table[mask.view(torch.uint8).long()].sum())


def check_parameter_gradients(updated, grad_normalized, gradients, chunk=16384):
    """dW/db against a float64 reduction over all rows (torch on the device)."""
    rows, hidden = updated.shape
    d_weight = torch.zeros(hidden, dtype=torch.float64, device="cuda")
    d_bias = torch.zeros(hidden, dtype=torch.float64, device="cuda")
    for start in range(0, rows, chunk):
        u = updated[start:start + chunk].double()
        centered = u - u.mean(dim=-1, keepdim=True)
        xhat = centered / torch.sqrt((centered * centered).mean(dim=-1, keepdim=True) + EPS)
        gy = grad_normalized[start:start + chunk].double()
        d_weight += (gy * xhat).sum(dim=0)
        d_bias += gy.sum(dim=0)
    assert_normwise(host(gradients[2]), host(d_weight), TOL_PARAMETER_GRAD, "grad_weight")
    assert_normwise(host(gradients[3]), host(d_bias), TOL_PARAMETER_GRAD, "grad_bias")


def test_c0_forward_eval_fp32_branch():
    inputs = make_inputs((4, 1024, 768), torch.float32, seed=1000)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, 0.0, EPS, False, 128)
    check_forward(outputs, inputs, 0.0, False, EPS, seed, offset, "C0")


def test_c1_gpt2_small_training_step():
    shape = (8, 1024, 768)
    inputs = make_inputs(shape, torch.float16, seed=1001, branch_std=0.5)
    grads = make_grads(shape, seed=2001)
    torch.cuda.manual_seed(1001)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, 0.1, EPS, True, 128)
    keep, scale = check_forward(outputs, inputs, 0.1, True, EPS, seed, offset, "C1")
    with deterministic_algorithms(False):
        gradients = raw_backward(grads, outputs, inputs[2], 0.1, True)
    check_backward(gradients, grads[0], grads[1], outputs[0], inputs[2], EPS, keep, scale, "C1")


@pytest.mark.parametrize("hidden", [128, 256, 384, 512, 768, 1024])
def test_c2_hidden_sweep_at_262144_rows(hidden):
    rows = 262144
    inputs, grads = device_inputs(rows, hidden, torch.float16, seed=1002 + hidden)
    torch.cuda.manual_seed(1002 + hidden)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, 0.15, EPS, True, 128)
    gradients = raw_backward(grads, outputs, inputs[2], 0.15, True)
    check_full_tensor(inputs, grads, outputs, gradients, 0.15, EPS, seed, offset,
                      what=f"C2 H={hidden}")
    check_parameter_gradients(outputs[0], grads[1], gradients)
    n = rows * hidden
    assert abs(keep_count(outputs[4]) - 0.85 * n) < 6 * np.sqrt(n * 0.15 * 0.85)


@pytest.mark.parametrize("rows", [65535, 65536])
@pytest.mark.parametrize("branch_dtype,grad_normalized_dtype",
                         [(torch.float16, torch.float32), (torch.bfloat16, torch.bfloat16)])
def test_768_backward_on_both_sides_of_its_three_wave_switch(rows, branch_dtype,
                                                             grad_normalized_dtype):
    """From 65536 rows the backward of 768 columns runs three waves of one
    slot per row (12-wave blocks), below it one wave of three slots: both
    sides against the oracle on sampled rows and a float64 reduction of
    dW/db, and each replays bitwise in deterministic mode."""
    hidden = 768
    inputs, grads = device_inputs(rows, hidden, branch_dtype, seed=4242)
    grads = (grads[0], grads[1].to(grad_normalized_dtype))
    torch.cuda.manual_seed(4242)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, 0.1, EPS, True, 128)

    def backward():
        return _C.residual_layer_norm_backward(
            grads[0], grads[1], outputs[0], inputs[2], outputs[2], outputs[3], outputs[4], 0.1,
            True, branch_dtype == torch.float16, 128, 64, 64, 1, True, branch_dtype)

    with deterministic_algorithms(True):
        gradients = backward()
        again = backward()
    for first, second in zip(gradients, again):
        assert torch.equal(first, second)
    check_full_tensor(inputs, grads, outputs, gradients, 0.1, EPS, seed, offset,
                      what=f"768 x {rows}")
    check_parameter_gradients(outputs[0], grads[1], gradients)
    with deterministic_algorithms(False):
        atomic = backward()
    assert torch.equal(atomic[0], gradients[0]) and torch.equal(atomic[1], gradients[1])
    check_parameter_gradients(outputs[0], grads[1], atomic)


def test_c3_deterministic_bitwise_replay_over_three_runs():
    rows, hidden = 32 * 2048, 1024
    inputs, grads = device_inputs(rows, hidden, torch.float16, seed=1003, branch_std=0.5)
    runs = []
    with deterministic_algorithms(True):
        for _ in range(3):
            torch.cuda.manual_seed(1003)
            seed, offset = generator_state()
            outputs = _C.residual_layer_norm_forward(*inputs, 0.15, EPS, True, 128)
            gradients = raw_backward(grads, outputs, inputs[2], 0.15, True)
            runs.append([host(t) for t in (*outputs, *gradients)])
    for run in runs[1:]:
        for a, b in zip(runs[0], run):
            assert_bitwise(b, a, "C3 replay")
    check_full_tensor(inputs, grads, outputs, gradients, 0.15, EPS, seed, offset, what="C3")
    check_parameter_gradients(outputs[0], grads[1], gradients)


@pytest.mark.parametrize("dropout_p", [0.0, 0.1])
def test_c4_tail_rows_with_large_mean(dropout_p):
    shape = (3, 4097, 384)
    inputs = make_inputs(shape, torch.float32, seed=1004, x_mean=100.0)
    grads = make_grads(shape, seed=2004)
    torch.cuda.manual_seed(1004)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, dropout_p, EPS, True, 128)
    keep, scale = check_forward(outputs, inputs, dropout_p, True, EPS, seed, offset, "C4 tail")
    gradients = raw_backward(grads, outputs, inputs[2], dropout_p, False)
    check_backward(gradients, grads[0], grads[1], outputs[0], inputs[2], EPS, keep, scale, "C4 tail")


@pytest.mark.parametrize("dropout_p", [0.0, 0.1])
def test_c4_single_row(dropout_p):
    shape = (1, 1, 128)
    inputs = make_inputs(shape, torch.float16, seed=1005)
    grads = make_grads(shape, seed=2005)
    torch.cuda.manual_seed(1005)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, dropout_p, EPS, True, 128)
    keep, scale = check_forward(outputs, inputs, dropout_p, True, EPS, seed, offset, "C4 row")
    for deterministic in (False, True):
        with deterministic_algorithms(deterministic):
            gradients = raw_backward(grads, outputs, inputs[2], dropout_p, True)
        check_backward(gradients, grads[0], grads[1], outputs[0], inputs[2], EPS, keep, scale,
                       "C4 row")


def test_c4_large_steady_state_shape():
    rows, hidden = 64 * 4096, 1024
    inputs, grads = device_inputs(rows, hidden, torch.float16, seed=1006)
    torch.cuda.manual_seed(1006)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, 0.1, EPS, True, 128)
    gradients = raw_backward(grads, outputs, inputs[2], 0.1, True)
    check_full_tensor(inputs, grads, outputs, gradients, 0.1, EPS, seed, offset,
                      what="C4 large")
    check_parameter_gradients(outputs[0], grads[1], gradients)
    n = rows * hidden
    assert abs(keep_count(outputs[4]) - 0.9 * n) < 6 * np.sqrt(n * 0.1 * 0.9)
