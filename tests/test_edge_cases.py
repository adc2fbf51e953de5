"""The reference's edge-case contract, as data, checked against the oracle.

The cases are the ones the reference's edge-case suite holds
(tests/test_residual_layer_norm_edge_cases.py of the reference): eval mode
bypasses dropout and draws no random numbers; either output alone can drive
the backward; hidden sizes that are not powers of two (384, 768) run forward
and backward; nearly-constant rows respect eps (1e-5 and 1e-3); and dropout
replays bit for bit after the RNG state is restored. Each case runs on two
legs through the public API: the reference's decomposition
(implementation="torch") on the CPU, and the gfx950 kernels on the GPU
(implementation="gfx950", marked `gpu`). Both are held to the parity bars of
tests/parity.py against the float64 oracle: `updated` bitwise, normalized
and grad_x normwise 1e-5, grad_branch within one ulp of its type, weight/bias
gradients 1e-4. On the GPU leg the dropout mask must also be the oracle's
(the reference's hipRAND stream for the call's seed and offset); on the CPU
leg, where torch draws the mask, the mask the decomposition applied is read
back from its output and handed to the oracle. Nearly-constant rows are the
committed golden fixtures, checked with the fp32 conditioned bounds.
"""

from dataclasses import dataclass
from pathlib import Path

import numpy as np
import pytest
import torch

import gfx1010_kernels.normalization as normalization
from gfx1010_kernels import residual_layer_norm
from oracle import rln_oracle as oracle
from parity import (
    API,
    KIND,
    TOL_FORWARD,
    TOL_INPUT_GRAD,
    TOL_PARAMETER_GRAD,
    assert_bitwise,
    assert_normwise,
    assert_rounded_close,
    assert_within,
    conditioned_bounds,
    generator_state,
    host,
    make_grads,
    make_inputs,
    oracle_keep,
)

LEGS = [
    pytest.param("cpu", id="cpu-torch"),
    pytest.param("cuda", id="gpu-gfx950", marks=pytest.mark.gpu),
]
IMPLEMENTATION = {"cpu": "torch", "cuda": "gfx950"}
EPS = 1e-5


@dataclass(frozen=True)
class EdgeCase:
    name: str
    rows: int
    hidden: int
    dropout_p: float = 0.0
    training: bool = True
    upstream: tuple = ("updated", "normalized")  # outputs that receive a gradient
    seed: int = 0

    def __str__(self):
        return self.name


CASES = [
    EdgeCase("eval-bypasses-dropout", 7, 384, dropout_p=0.8, training=False, seed=7101),
    EdgeCase("updated-alone", 7, 384, upstream=("updated",), seed=7103),
    EdgeCase("normalized-alone", 7, 384, upstream=("normalized",), seed=7105),
    EdgeCase("hidden-384", 5, 384, seed=7107),
    EdgeCase("hidden-768", 5, 768, seed=7109),
    EdgeCase("dropout-384", 11, 384, dropout_p=0.25, seed=7111),
    EdgeCase("dropout-768-updated-alone", 6, 768, dropout_p=0.1, upstream=("updated",),
             seed=7113),
]


def branch_type(leg):
    # The GPU leg runs the reference's typical fp16 branch; the CPU leg fp32.
    return torch.float16 if leg == "cuda" else torch.float32


def rng_states(leg):
    return (torch.random.get_rng_state(),
            torch.cuda.get_rng_state(0) if leg == "cuda" else None)


def applied_keep(x, branch, updated, dropout_p):
    """The mask the decomposition drew, read back from its output: a dropped
    element adds exactly 0 to x (inputs here have no zero branch values)."""
    keep = host(updated) != host(x)
    assert not np.any(host(branch) == 0)
    return keep


def run_public(leg, case):
    """Forward (+ backward of the case's upstream outputs) through the public
    API; returns inputs, outputs, upstream gradients, input gradients and the
    generator state the call drew from."""
    shape = (case.rows, case.hidden)
    inputs = make_inputs(shape, branch_type(leg), seed=case.seed, device=leg)
    grads = make_grads(shape, seed=case.seed + 1, device=leg)
    leaves = [t.detach().clone().requires_grad_(True) for t in inputs]
    seed, offset = generator_state() if leg == "cuda" else (None, None)
    before = rng_states(leg)
    outputs = residual_layer_norm(*leaves, dropout_p=case.dropout_p, eps=EPS,
                                  training=case.training, implementation=IMPLEMENTATION[leg])
    used = [i for i, name in enumerate(("updated", "normalized")) if name in case.upstream]
    gradients = torch.autograd.grad([outputs[i] for i in used], leaves,
                                    [grads[i] for i in used], allow_unused=True)
    return inputs, outputs, grads, gradients, (seed, offset), before


@pytest.mark.parametrize("case", CASES, ids=str)
@pytest.mark.parametrize("leg", LEGS)
def test_edge_case_matches_the_oracle(leg, case):
    inputs, outputs, grads, gradients, (seed, offset), before = run_public(leg, case)
    x, branch, weight, bias = (host(t) for t in inputs)
    rows, hidden = x.shape
    active, scale, _ = oracle.dropout_constants(case.dropout_p, case.training)
    keep = None
    if active:
        if leg == "cuda":
            keep, scale, _ = oracle_keep(rows, hidden, case.dropout_p, True, seed, offset, API)
        else:
            keep = applied_keep(inputs[0], inputs[1], outputs[0], case.dropout_p)
            assert 0.5 < keep.mean() < 1.0
    else:
        # No dropout (eval, or p = 0): no random numbers drawn on any generator.
        after = rng_states(leg)
        assert torch.equal(after[0], before[0])
        if after[1] is not None:
            assert torch.equal(after[1], before[1])
    expected = oracle.forward(x, branch, weight, bias, EPS, keep=keep, scale=scale,
                              branch_type=KIND[inputs[1].dtype])
    assert_bitwise(host(outputs[0]), expected["updated"], f"{case} updated")
    assert_normwise(host(outputs[1]), expected["normalized"], TOL_FORWARD, f"{case} normalized")

    grad_updated = host(grads[0]) if "updated" in case.upstream else None
    grad_normalized = host(grads[1]) if "normalized" in case.upstream else None
    want = oracle.backward(grad_updated, grad_normalized, expected["updated"], weight, EPS,
                           keep=keep, scale=scale)
    grad_x, grad_branch, grad_weight, grad_bias = gradients
    assert_normwise(host(grad_x), want["grad_x"], TOL_INPUT_GRAD, f"{case} grad_x")
    assert grad_branch.dtype == inputs[1].dtype
    if grad_branch.dtype == torch.float32:
        assert_normwise(host(grad_branch), want["grad_branch"], TOL_INPUT_GRAD,
                        f"{case} grad_branch")
    else:
        assert_rounded_close(host(grad_branch), want["grad_branch"], KIND[grad_branch.dtype],
                             f"{case} grad_branch")
    if grad_normalized is None:
        # `updated` alone: weight and bias receive no gradient (None, or zeros
        # from the decomposition's graph).
        for gradient in (grad_weight, grad_bias):
            assert gradient is None or torch.count_nonzero(gradient) == 0
    else:
        assert_normwise(host(grad_weight), want["grad_weight"], TOL_PARAMETER_GRAD,
                        f"{case} grad_weight")
        assert_normwise(host(grad_bias), want["grad_bias"], TOL_PARAMETER_GRAD,
                        f"{case} grad_bias")


NEARLY_CONSTANT = sorted((Path(__file__).parent / "golden").glob("nearly_constant_rows_*.npz"))


@pytest.mark.parametrize("path", NEARLY_CONSTANT, ids=lambda p: p.stem)
@pytest.mark.parametrize("leg", LEGS)
def test_nearly_constant_rows_respect_eps(leg, path):
    """Rows of spread 2e-4 around -3, 0.25 and 4 (var far below eps): the
    public API's outputs and normalized-driven gradients stay finite and
    within the fp32 conditioned bounds of the float64 fixture."""
    d = dict(np.load(path, allow_pickle=False))
    eps = float(d["eps"])
    leaves = [torch.from_numpy(d[name]).to(leg).requires_grad_(True)
              for name in ("x", "branch", "weight", "bias")]
    updated, normalized = residual_layer_norm(*leaves, eps=eps,
                                              implementation=IMPLEMENTATION[leg])
    grads = torch.autograd.grad(normalized, leaves, torch.from_numpy(d["grad_normalized"]).to(leg))
    assert all(torch.isfinite(t).all() for t in (updated, normalized, *grads))
    assert_bitwise(host(updated), d["updated"], "updated")
    bounds = conditioned_bounds(d["updated"], d["weight"], eps, None, d["grad_normalized"])
    assert_within(host(normalized), d["normalized"], bounds["normalized"], "normalized")
    assert_within(host(grads[0]), d["grad_x"], bounds["grad_x"], "grad_x")
    assert_within(host(grads[1]), d["grad_branch"], bounds["grad_x"], "grad_branch")
    assert_within(host(grads[2]), d["grad_weight"], bounds["grad_weight"], "grad_weight")
    assert_within(host(grads[3]), d["grad_bias"], bounds["grad_bias"], "grad_bias")


@pytest.mark.parametrize("hidden,dropout_p", [(384, 0.25), (768, 0.1)])
@pytest.mark.parametrize("leg", LEGS)
def test_dropout_replays_after_the_rng_state_is_restored(leg, hidden, dropout_p):
    """Restoring the generator state replays the same mask: outputs and
    gradients repeat bit for bit (deterministic weight/bias sums on the GPU);
    without restoring it the next call draws a different mask."""
    case = EdgeCase("replay", 11, hidden, dropout_p=dropout_p, seed=7201 + hidden)
    previous = torch.are_deterministic_algorithms_enabled()
    warn_only = torch.is_deterministic_algorithms_warn_only_enabled()
    torch.use_deterministic_algorithms(True)
    try:
        state = rng_states(leg)
        first = run_public(leg, case)
        torch.random.set_rng_state(state[0])
        if state[1] is not None:
            torch.cuda.set_rng_state(state[1], 0)
        second = run_public(leg, case)
        third = run_public(leg, case)
    finally:
        torch.use_deterministic_algorithms(previous, warn_only=warn_only)
    for a, b in zip((*first[1], *first[3]), (*second[1], *second[3])):
        assert_bitwise(host(b), host(a), "replay")
    assert not torch.equal(third[1][0], first[1][0])


@pytest.mark.gpu
def test_strict_native_call_skips_python_validation_and_device_guard(monkeypatch):
    """implementation="gfx950" (and its alias "gfx1010") goes straight to the
    native op: no Python input validation, no device-guard context."""
    inputs = make_inputs((3, 384), torch.float16, seed=7301)

    def forbidden(*args, **kwargs):
        raise AssertionError("the strict native call ran Python dispatch work")

    monkeypatch.setattr(normalization, "_input_reason", forbidden)
    monkeypatch.setattr(torch.cuda, "device", forbidden)
    for implementation in ("gfx950", "gfx1010"):
        residual_layer_norm(*inputs, implementation=implementation)


@pytest.mark.gpu
def test_auto_serves_mi355x_natively_without_a_warning():
    import warnings

    from gfx1010_kernels import can_use_residual_layer_norm, residual_layer_norm_status

    status = residual_layer_norm_status()
    assert status.available and status.architecture == "gfx950", status
    inputs = make_inputs((4, 768), torch.float16, seed=7303)
    assert can_use_residual_layer_norm(*inputs, dropout_p=0.1)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        auto = residual_layer_norm(*inputs, training=False)
    strict = residual_layer_norm(*inputs, training=False, implementation="gfx950")
    assert torch.equal(auto[0], strict[0]) and torch.equal(auto[1], strict[1])
