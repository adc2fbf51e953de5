"""torch.compile and the registered custom ops on the GPU.

The compiled graph calls ``gfx1010_kernels::rln_forward`` / ``rln_backward``
(the same kernels as the eager autograd function), so from the same RNG state
a compiled training step reproduces the eager step bit for bit (weight/bias
gradients in deterministic mode). ``backend="aot_eager"`` traces with Dynamo
and AOTAutograd without generating code for the surrounding ops.
"""

import contextlib

import numpy as np

import pytest
import torch

from gfx1010_kernels import residual_layer_norm
from parity import assert_bitwise, host, make_grads, make_inputs

pytestmark = pytest.mark.gpu


@contextlib.contextmanager
def deterministic_algorithms():
    previous = torch.are_deterministic_algorithms_enabled()
    torch.use_deterministic_algorithms(True)
    try:
        yield
    finally:
        torch.use_deterministic_algorithms(previous)


def test_opcheck_forward_and_backward():
    inputs = make_inputs((33, 512), torch.float16, seed=3)
    # Without dropout the op is a pure function of its inputs, as opcheck
    # requires (it compares several executions).
    torch.library.opcheck(torch.ops.gfx1010_kernels.rln_forward.default,
                          (*inputs, 0.0, 1e-5, True))
    torch.library.opcheck(torch.ops.gfx1010_kernels.rln_forward.default,
                          (*inputs, 0.0, 1e-5, True, torch.bfloat16))
    outputs = torch.ops.gfx1010_kernels.rln_forward(*inputs, 0.0, 1e-5, True)
    grads = make_grads((33, 512), seed=4)
    with deterministic_algorithms():
        torch.library.opcheck(
            torch.ops.gfx1010_kernels.rln_backward.default,
            (grads[0], grads[1], outputs[0], inputs[2], outputs[2], outputs[3], outputs[4],
             0.0, True, torch.float16))
        # Without the weight/bias sums (a pass that needs neither gradient).
        torch.library.opcheck(
            torch.ops.gfx1010_kernels.rln_backward.default,
            (grads[0], grads[1], outputs[0], inputs[2], outputs[2], outputs[3], outputs[4],
             0.0, True, torch.float16, False))


@pytest.mark.parametrize("implementation", ["gfx950", "auto"])
@pytest.mark.parametrize("shape,dropout_p", [((4, 64, 768), 0.1), ((3, 97, 384), 0.0),
                                             ((2, 40, 1024), 0.2), ((2, 33, 1600), 0.1)])
def test_compiled_step_matches_eager_bitwise(implementation, shape, dropout_p):
    inputs = make_inputs(shape, torch.float16, seed=11)
    grads = make_grads(shape, seed=12)

    def step(x, branch, weight, bias):
        updated, normalized = residual_layer_norm(
            x, branch, weight, bias, dropout_p=dropout_p, implementation=implementation)
        return updated, normalized

    compiled = torch.compile(step, backend="aot_eager", fullgraph=True)
    results = []
    with deterministic_algorithms():
        for function in (step, compiled):
            leaves = [t.detach().clone().requires_grad_(True) for t in inputs]
            torch.cuda.manual_seed(2024)
            outputs = function(*leaves)
            torch.autograd.backward(outputs, grads)
            torch.cuda.synchronize()
            results.append([host(t) for t in outputs] + [host(t.grad) for t in leaves])
    for eager, traced in zip(*results):
        assert_bitwise(traced, eager, "compiled vs eager")


@pytest.mark.parametrize("backend", ["inductor", "aot_eager"])
def test_compiled_step_with_frozen_parameters(backend):
    """A compiled training step whose LayerNorm weight and bias are frozen:
    the backward asks the op for no weight/bias sums, its input gradients
    equal eager's bit for bit, and the frozen parameters get no gradient."""
    shape = (4, 64, 768)
    inputs = make_inputs(shape, torch.float16, seed=13)
    grads = make_grads(shape, seed=14)

    def step(x, branch, weight, bias):
        return residual_layer_norm(x, branch, weight, bias, dropout_p=0.1,
                                   implementation="gfx950")

    compiled = torch.compile(step, backend=backend, fullgraph=True)
    results = []
    for function in (step, compiled):
        x, branch = (t.detach().clone().requires_grad_(True) for t in inputs[:2])
        weight, bias = (t.detach().clone() for t in inputs[2:])
        torch.cuda.manual_seed(77)
        outputs = function(x, branch, weight, bias)
        torch.autograd.backward(outputs, grads)
        torch.cuda.synchronize()
        assert weight.grad is None and bias.grad is None
        results.append([host(t) for t in outputs] + [host(x.grad), host(branch.grad)])
    for eager, traced in zip(*results):
        assert_bitwise(traced, eager, "compiled vs eager, frozen parameters")


def test_compiled_auto_falls_back_for_non_native_hidden_size():
    inputs = make_inputs((5, 160), torch.float32, seed=2)

    def step(x, branch, weight, bias):
        return residual_layer_norm(x, branch, weight, bias, dropout_p=0.0)

    compiled = torch.compile(step, backend="aot_eager", fullgraph=True)
    expected = torch.nn.functional.layer_norm(inputs[0] + inputs[1], (160,), inputs[2],
                                              inputs[3], 1e-5)
    torch.testing.assert_close(compiled(*inputs)[1], expected)


@pytest.mark.parametrize("backend", ["inductor", "aot_eager"])
def test_two_equal_dropout_calls_in_one_compiled_graph(backend):
    """Two calls on equal arguments in one compiled training graph draw two
    masks, equal bit for bit to two eager calls from the same RNG state, and
    leave the generator where the eager calls leave it (AOTAutograd's
    common-subexpression pass must not merge them into one draw)."""
    shape = (3, 40, 768)
    inputs = make_inputs(shape, torch.float16, seed=21)

    def two_calls(x, branch, weight, bias):
        first = residual_layer_norm(x, branch, weight, bias, dropout_p=0.5,
                                    implementation="gfx950")
        second = residual_layer_norm(x, branch, weight, bias, dropout_p=0.5,
                                     implementation="gfx950")
        return (*first, *second)

    compiled = torch.compile(two_calls, backend=backend, fullgraph=True)
    results, offsets = [], []
    for function in (two_calls, compiled):
        leaves = [t.detach().clone().requires_grad_(True) for t in inputs]
        torch.cuda.manual_seed(77)
        outputs = function(*leaves)
        offsets.append(torch.cuda.default_generators[0].get_offset())
        torch.cuda.synchronize()
        results.append([host(t) for t in outputs])
    eager, traced = results
    # The two eager draws differ (a merged call would return the same
    # `updated` twice).
    assert not np.array_equal(eager[0], eager[2])
    for index, (expected, actual) in enumerate(zip(eager, traced)):
        assert_bitwise(actual, expected, f"compiled output {index} vs eager")
    assert offsets[1] == offsets[0]


def test_reduce_overhead_training_step_replays():
    """torch.compile(mode="reduce-overhead"): inductor captures the compiled
    training step, custom ops included, into CUDA/HIP graphs and replays them.
    Without dropout every replay, on inputs that change between replays, equals
    the eager step on the same inputs bit for bit (weight gradient in
    deterministic mode); with dropout each replay draws a fresh mask and
    `updated` keeps about 1 - p of the branch."""
    shape = (4, 64, 768)
    inputs = make_inputs(shape, torch.float16, seed=31)
    grads = make_grads(shape, seed=32)
    params = [t.detach().clone().requires_grad_(True) for t in inputs[2:]]

    def body(x, branch):
        return residual_layer_norm(x, branch, params[0], params[1], dropout_p=0.0,
                                   implementation="gfx950")

    def run(function, replay):
        for p in params:
            p.grad = None
        x = (inputs[0] * (1.0 + 0.25 * replay)).detach().requires_grad_(True)
        torch.compiler.cudagraph_mark_step_begin()
        updated, normalized = function(x, inputs[1])
        torch.autograd.backward((updated, normalized), grads)
        torch.cuda.synchronize()
        return host(updated).copy(), host(params[0].grad).copy()

    with deterministic_algorithms():
        compiled = torch.compile(body, mode="reduce-overhead", fullgraph=True)
        for replay in range(5):
            expected = run(body, replay)
            actual = run(compiled, replay)
            assert_bitwise(actual[0], expected[0], f"replay {replay} updated")
            assert_bitwise(actual[1], expected[1], f"replay {replay} grad_weight")

    def dropped(x, branch):
        return residual_layer_norm(x, branch, params[0], params[1], dropout_p=0.3,
                                   implementation="gfx950")

    compiled_dropout = torch.compile(dropped, mode="reduce-overhead", fullgraph=True)
    updates = []
    for replay in range(5):
        torch.compiler.cudagraph_mark_step_begin()
        with torch.no_grad():
            updated, _ = compiled_dropout(inputs[0], inputs[1])
        torch.cuda.synchronize()
        kept = (host(updated) != host(inputs[0])).mean()
        assert 0.6 < kept < 0.8, f"replay {replay}: kept {kept}"
        updates.append(host(updated).copy())
    assert not np.array_equal(updates[3], updates[4])


@pytest.mark.parametrize("strict", [False, True], ids=["non-strict", "strict"])
def test_torch_export_keeps_the_fused_op(strict):
    """torch.export of a module that calls residual_layer_norm: the exported
    graph holds the registered custom op (no decomposition), and the exported
    program's outputs equal the module's bit for bit (eval mode; the reference
    does not support export, docs/residual_layer_norm.md:301-302)."""

    class Block(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.norm = torch.nn.LayerNorm(768)

        def forward(self, x, branch):
            return residual_layer_norm(x, branch, self.norm.weight, self.norm.bias,
                                       dropout_p=0.1, training=self.training,
                                       implementation="gfx950")

    model = Block().cuda().eval()
    with torch.no_grad():
        model.norm.weight.normal_(1.0, 0.02)
        model.norm.bias.normal_(0.0, 0.02)
    inputs = make_inputs((2, 37, 768), torch.float16, seed=41)[:2]
    exported = torch.export.export(model, inputs, strict=strict)
    targets = [str(node.target) for node in exported.graph.nodes if node.op == "call_function"]
    assert any("gfx1010_kernels.rln_forward" in target for target in targets), targets
    assert not any("layer_norm" in target for target in targets), targets
    with torch.no_grad():
        expected = model(*inputs)
        actual = exported.module()(*inputs)
    for index, (a, b) in enumerate(zip(actual, expected)):
        assert_bitwise(host(a), host(b), f"exported output {index}")
