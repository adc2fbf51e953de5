"""The reference's edge-case suite, run on both legs: the PyTorch decomposition
on the CPU and the gfx950 kernels on the GPU
(tests/test_residual_layer_norm_edge_cases.py:11-293 of the reference).

The GPU leg is marked ``gpu``; the CPU leg runs everywhere.
"""

import pytest
import torch
from torch.nn import functional as F

from gfx1010_kernels import residual_layer_norm
import gfx1010_kernels.normalization as normalization

BACKENDS = [
    pytest.param(torch.device("cpu"), "torch", id="cpu-torch"),
    pytest.param(torch.device("cuda"), "gfx950", id="gpu-gfx950", marks=pytest.mark.gpu),
]


def _reference(x, branch, weight, bias, dropout_p=0.0, eps=1e-5, training=True):
    branch = F.dropout(branch, dropout_p, training)
    updated = x + branch
    return updated, F.layer_norm(updated, (updated.shape[-1],), weight, bias, eps)


def _random_inputs(device, implementation, hidden_size, rows=7):
    branch_dtype = torch.float16 if implementation == "gfx950" else torch.float32
    return (
        torch.randn(rows, hidden_size, device=device, dtype=torch.float32),
        torch.randn(rows, hidden_size, device=device, dtype=branch_dtype),
        torch.randn(hidden_size, device=device, dtype=torch.float32),
        torch.randn(hidden_size, device=device, dtype=torch.float32),
    )


def _leaves(inputs):
    return tuple(value.detach().clone().requires_grad_(True) for value in inputs)


def _rng_state(device):
    return (torch.random.get_rng_state(),
            torch.cuda.get_rng_state(device) if device.type == "cuda" else None)


def _restore_rng_state(device, state):
    torch.random.set_rng_state(state[0])
    if state[1] is not None:
        torch.cuda.set_rng_state(state[1], device)


@pytest.mark.parametrize("device,implementation", BACKENDS)
def test_eval_bypasses_dropout_without_consuming_rng(device, implementation):
    torch.manual_seed(101)
    inputs = _random_inputs(device, implementation, hidden_size=384)
    state = _rng_state(device)
    actual = residual_layer_norm(*inputs, dropout_p=0.8, training=False, implementation=implementation)
    expected = _reference(*inputs, dropout_p=0.8, training=False)
    torch.testing.assert_close(actual[0], expected[0], rtol=0, atol=1e-6)
    torch.testing.assert_close(actual[1], expected[1], rtol=5e-4, atol=5e-4)
    current = _rng_state(device)
    assert torch.equal(current[0], state[0])
    if state[1] is not None:
        assert torch.equal(current[1], state[1])


@pytest.mark.parametrize("device,implementation", BACKENDS)
@pytest.mark.parametrize("used_output", [0, 1], ids=["updated-only", "normalized-only"])
def test_each_output_can_drive_backward_alone(device, implementation, used_output):
    torch.manual_seed(103)
    data = _random_inputs(device, implementation, hidden_size=384)
    actual_inputs, expected_inputs = _leaves(data), _leaves(data)
    actual_outputs = residual_layer_norm(*actual_inputs, implementation=implementation)
    expected_outputs = _reference(*expected_inputs)
    upstream = torch.randn_like(actual_outputs[used_output])
    actual = torch.autograd.grad(actual_outputs[used_output], actual_inputs, upstream, allow_unused=True)
    expected = torch.autograd.grad(expected_outputs[used_output], expected_inputs, upstream,
                                   allow_unused=True)
    for a, e, like in zip(actual, expected, actual_inputs):
        if e is None:
            assert a is None or torch.count_nonzero(a) == 0
            continue
        torch.testing.assert_close(a, e, rtol=3e-3, atol=3e-3)
        assert a.dtype == like.dtype


@pytest.mark.parametrize("device,implementation", BACKENDS)
@pytest.mark.parametrize("eps", [1e-5, 1e-3])
def test_nearly_constant_rows_respect_eps(device, implementation, eps):
    # Rows of spread 2e-4 around offsets up to 4 are ill-conditioned in fp32
    # (the fp32 mean carries ~1 ulp of 4.0); tolerances are the reference's.
    hidden_size = 384
    columns = torch.linspace(-1.0, 1.0, hidden_size, device=device)
    centers = torch.tensor([-3.0, 0.25, 4.0], device=device)[:, None]
    x = centers + columns[None, :] * 2e-4
    branch = (-columns[None, :] * 5e-5).expand_as(x).contiguous()
    if implementation == "gfx950":
        branch = branch.to(torch.float16)
    weight = torch.linspace(0.75, 1.25, hidden_size, device=device)
    bias = torch.linspace(-0.1, 0.1, hidden_size, device=device)
    actual_inputs, expected_inputs = _leaves((x, branch, weight, bias)), _leaves((x, branch, weight, bias))
    actual = residual_layer_norm(*actual_inputs, eps=eps, implementation=implementation)
    expected = _reference(*expected_inputs, eps=eps)
    upstream = torch.sin(columns)[None, :].expand_as(actual[1]).contiguous()
    actual_grads = torch.autograd.grad(actual[1], actual_inputs, upstream)
    expected_grads = torch.autograd.grad(expected[1], expected_inputs, upstream)
    assert all(torch.isfinite(value).all() for value in (*actual, *actual_grads))
    torch.testing.assert_close(actual[0], expected[0], rtol=0, atol=1e-6)
    torch.testing.assert_close(actual[1], expected[1], rtol=8e-3, atol=8e-3)
    for a, e in zip(actual_grads, expected_grads):
        torch.testing.assert_close(a.float(), e.float(), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("device,implementation", BACKENDS)
@pytest.mark.parametrize("hidden_size", [384, 768])
def test_non_power_of_two_hidden_sizes_forward_and_backward(device, implementation, hidden_size):
    torch.manual_seed(107)
    data = _random_inputs(device, implementation, hidden_size, rows=5)
    actual_inputs, expected_inputs = _leaves(data), _leaves(data)
    actual = residual_layer_norm(*actual_inputs, implementation=implementation)
    expected = _reference(*expected_inputs)
    grads = (torch.randn_like(actual[0]), torch.randn_like(actual[1]))
    actual_grads = torch.autograd.grad(actual, actual_inputs, grads)
    expected_grads = torch.autograd.grad(expected, expected_inputs, grads)
    torch.testing.assert_close(actual[0], expected[0], rtol=0, atol=1e-6)
    torch.testing.assert_close(actual[1], expected[1], rtol=5e-4, atol=5e-4)
    for a, e in zip(actual_grads, expected_grads):
        torch.testing.assert_close(a, e, rtol=3e-3, atol=3e-3)


@pytest.mark.parametrize("device,implementation", BACKENDS)
def test_dropout_replays_after_rng_state_restore(device, implementation):
    torch.manual_seed(109)
    data = _random_inputs(device, implementation, hidden_size=384, rows=11)
    first_inputs, second_inputs = _leaves(data), _leaves(data)
    grad_updated = torch.linspace(-0.5, 0.5, first_inputs[0].numel(), device=device).reshape_as(
        first_inputs[0])
    grad_normalized = torch.cos(grad_updated)
    state = _rng_state(device)
    deterministic = torch.are_deterministic_algorithms_enabled()
    warn_only = torch.is_deterministic_algorithms_warn_only_enabled()
    if implementation == "gfx950":
        torch.use_deterministic_algorithms(True)
    try:
        first = residual_layer_norm(*first_inputs, dropout_p=0.25, implementation=implementation)
        _restore_rng_state(device, state)
        second = residual_layer_norm(*second_inputs, dropout_p=0.25, implementation=implementation)
        first_grads = torch.autograd.grad(first, first_inputs, (grad_updated, grad_normalized))
        second_grads = torch.autograd.grad(second, second_inputs, (grad_updated, grad_normalized))
        for a, b in zip((*first, *first_grads), (*second, *second_grads)):
            torch.testing.assert_close(a, b, rtol=0, atol=0)
    finally:
        if implementation == "gfx950":
            torch.use_deterministic_algorithms(deterministic, warn_only=warn_only)


@pytest.mark.gpu
def test_forced_native_hot_path_skips_python_validation_and_device_guard(monkeypatch):
    inputs = _random_inputs(torch.device("cuda"), "gfx950", hidden_size=384)

    def fail_if_called(*args, **kwargs):
        raise AssertionError("forced native hot path used Python dispatch work")

    monkeypatch.setattr(normalization, "_input_reason", fail_if_called)
    monkeypatch.setattr(torch.cuda, "device", fail_if_called)
    residual_layer_norm(*inputs, implementation="gfx950")
    residual_layer_norm(*inputs, implementation="gfx1010")


@pytest.mark.gpu
def test_auto_uses_the_native_backend_on_mi355x():
    from gfx1010_kernels import can_use_residual_layer_norm, residual_layer_norm_status

    status = residual_layer_norm_status()
    assert status.available and status.architecture == "gfx950", status
    inputs = _random_inputs(torch.device("cuda"), "gfx950", hidden_size=768)
    assert can_use_residual_layer_norm(*inputs, dropout_p=0.1)
    import warnings

    with warnings.catch_warnings():
        warnings.simplefilter("error")
        auto = residual_layer_norm(*inputs, training=False)
    strict = residual_layer_norm(*inputs, training=False, implementation="gfx950")
    assert torch.equal(auto[0], strict[0]) and torch.equal(auto[1], strict[1])
