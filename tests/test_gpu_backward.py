"""Backward parity: input gradients and weight/bias gradients, atomic and
deterministic reductions, partial upstream gradients, autograd contract.

Follows the reference's backward tests (tests/test_residual_layer_norm.py:132-184,
tests/test_residual_layer_norm_native_matrix.py:184-383,
tests/test_residual_layer_norm_vectorized.py:17-93, :167-232).
"""

import contextlib

import numpy as np
import pytest
import torch

from gfx1010_kernels import _C, residual_layer_norm
from parity import (
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


@contextlib.contextmanager
def deterministic_algorithms(enabled):
    previous = torch.are_deterministic_algorithms_enabled()
    warn_only = torch.is_deterministic_algorithms_warn_only_enabled()
    torch.use_deterministic_algorithms(enabled)
    try:
        yield
    finally:
        torch.use_deterministic_algorithms(previous, warn_only=warn_only)


def raw_backward(grad_updated, grad_normalized, outputs, weight, dropout_p, branch_is_half,
                 training=True, parameters=True):
    """``branch_is_half`` is the reference's flag, or a torch dtype (bf16 included)."""
    extra = {}
    if isinstance(branch_is_half, torch.dtype):
        extra["branch_dtype"] = branch_is_half
        branch_is_half = branch_is_half == torch.float16
    return _C.residual_layer_norm_backward(
        grad_updated, grad_normalized, outputs[0], weight, outputs[2], outputs[3], outputs[4],
        dropout_p, training, branch_is_half, 128, 64, 64, 1, parameters, **extra)


@pytest.mark.parametrize("hidden", SPECIALIZED_HIDDEN_SIZES)
@pytest.mark.parametrize("branch_dtype", [torch.float16, torch.bfloat16, torch.float32],
                         ids=["f16", "bf16", "f32"])
@pytest.mark.parametrize("dropout_p", [0.0, 0.15])
@pytest.mark.parametrize("deterministic", [False, True], ids=["atomic", "deterministic"])
def test_backward_matches_oracle(hidden, branch_dtype, dropout_p, deterministic):
    rows = 41
    inputs = make_inputs((rows, hidden), branch_dtype, seed=23 + hidden)
    grad_updated, grad_normalized = make_grads((rows, hidden), seed=99 + hidden)
    torch.cuda.manual_seed(hidden)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, dropout_p, 1e-5, True, 128)
    keep, scale = check_forward(outputs, inputs, dropout_p, True, 1e-5, seed, offset)
    with deterministic_algorithms(deterministic):
        gradients = raw_backward(grad_updated, grad_normalized, outputs, inputs[2], dropout_p,
                                 branch_dtype)
    check_backward(gradients, grad_updated, grad_normalized, outputs[0], inputs[2], 1e-5, keep,
                   scale, f"H={hidden}")
    assert gradients[1].dtype == branch_dtype


@pytest.mark.parametrize("hidden", [128, 768])
@pytest.mark.parametrize("rows", [1, 17, 513, 2049, 40000])
@pytest.mark.parametrize("deterministic", [False, True], ids=["atomic", "deterministic"])
def test_parameter_gradients_over_row_counts(hidden, rows, deterministic):
    inputs = make_inputs((rows, hidden), torch.float16, seed=rows + hidden)
    grad_updated, grad_normalized = make_grads((rows, hidden), seed=rows)
    outputs = _C.residual_layer_norm_forward(*inputs, 0.0, 1e-5, True, 128)
    with deterministic_algorithms(deterministic):
        gradients = raw_backward(grad_updated, grad_normalized, outputs, inputs[2], 0.0, True)
    check_backward(gradients, grad_updated, grad_normalized, outputs[0], inputs[2], 1e-5, None,
                   1.0, f"rows={rows}")


def test_deterministic_replay_is_bitwise_and_independent_of_launch_hints():
    rows, hidden = 4099, 1024
    inputs = make_inputs((rows, hidden), torch.float16, seed=419)
    grad_updated, grad_normalized = make_grads((rows, hidden), seed=420)
    torch.cuda.manual_seed(7)
    outputs = _C.residual_layer_norm_forward(*inputs, 0.15, 1e-5, True, 128)
    with deterministic_algorithms(True):
        runs = [
            _C.residual_layer_norm_backward(
                grad_updated, grad_normalized, outputs[0], inputs[2], outputs[2], outputs[3],
                outputs[4], 0.15, True, True, 128, block_rows, 64, groups, True)
            for block_rows, groups in ((16, 1), (64, 12), (128, rows))
        ]
    for run in runs[1:]:
        for a, b in zip(runs[0], run):
            assert_bitwise(host(b), host(a))


def test_parameter_groups_are_range_checked():
    inputs = make_inputs((257, 384), torch.float16, seed=233)
    outputs = _C.residual_layer_norm_forward(*inputs, 0.0, 1e-5, True, 128)
    g = torch.randn_like(outputs[0])
    for groups in (0, 258):
        with pytest.raises(RuntimeError, match=r"parameter_groups must be in \[1, row_count\]"):
            _C.residual_layer_norm_backward(g, g, outputs[0], inputs[2], outputs[2], outputs[3],
                                            outputs[4], 0.0, True, True, 128, 32, 64, groups, True)
    with pytest.raises(RuntimeError, match="block_rows must be 16, 32, 64 or 128"):
        _C.residual_layer_norm_backward(g, g, outputs[0], inputs[2], outputs[2], outputs[3],
                                        outputs[4], 0.0, True, True, 128, 8, 64, 1, True)
    with pytest.raises(RuntimeError, match="dropout_mask has the wrong size"):
        _C.residual_layer_norm_backward(g, g, outputs[0], inputs[2], outputs[2], outputs[3],
                                        outputs[4], 0.1, True, True, 128, 32, 64, 1, True)


def test_raw_backward_rejects_empty_rows():
    updated = torch.empty(0, 128, device="cuda")
    stats = torch.empty(0, device="cuda")
    with pytest.raises(RuntimeError, match="empty tensors are unsupported"):
        _C.residual_layer_norm_backward(
            updated, updated, updated, torch.ones(128, device="cuda"), stats, stats,
            torch.empty(0, device="cuda", dtype=torch.int32), 0.0, True, True, 128, 16, 64, 1, True)


@pytest.mark.parametrize("which", ["updated", "normalized"])
def test_missing_upstream_gradient_is_zero(which):
    rows, hidden = 33, 768
    inputs = make_inputs((rows, hidden), torch.float16, seed=31)
    grad_updated, grad_normalized = make_grads((rows, hidden), seed=32)
    torch.cuda.manual_seed(9)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, 0.1, 1e-5, True, 128)
    keep, scale = check_forward(outputs, inputs, 0.1, True, 1e-5, seed, offset)
    if which == "updated":
        grad_normalized = None
    else:
        grad_updated = None
    gradients = raw_backward(grad_updated, grad_normalized, outputs, inputs[2], 0.1, True,
                             parameters=grad_normalized is not None)
    check_backward(gradients, grad_updated, grad_normalized, outputs[0], inputs[2], 1e-5, keep,
                   scale, which, parameters=grad_normalized is not None)


def test_updated_only_autograd_is_bitwise_and_leaves_parameters_unused():
    # Reference: tests/test_residual_layer_norm_native_matrix.py:184-225.
    x, branch, weight, bias = (t.requires_grad_(True) for t in make_inputs((13, 384), torch.float16, seed=229))
    updated = residual_layer_norm(x, branch, weight, bias, implementation="gfx950")[0]
    upstream = torch.randn_like(updated)
    gradients = torch.autograd.grad(updated, (x, branch, weight, bias), upstream,
                                    allow_unused=True, materialize_grads=False)
    assert_bitwise(host(gradients[0]), host(upstream), "grad_x")
    assert_bitwise(host(gradients[1]), host(upstream.half()), "grad_branch")
    assert gradients[2] is None and gradients[3] is None


def test_autograd_matches_oracle_through_public_api():
    rows, hidden = 41, 512
    x, branch, weight, bias = (
        t.requires_grad_(True) for t in make_inputs((rows, hidden), torch.float16, seed=23))
    torch.cuda.manual_seed(3)
    seed, offset = generator_state()
    updated, normalized = residual_layer_norm(x, branch, weight, bias, dropout_p=0.1,
                                              implementation="gfx950")
    grad_updated, grad_normalized = make_grads((rows, hidden), seed=4)
    torch.autograd.backward((updated, normalized), (grad_updated, grad_normalized))
    from parity import API, oracle_keep
    keep, scale, _ = oracle_keep(rows, hidden, 0.1, True, seed, offset, API)
    check_backward((x.grad, branch.grad, weight.grad, bias.grad), grad_updated, grad_normalized,
                   updated, weight, 1e-5, keep, scale, "autograd")


@pytest.mark.parametrize("dropout_p", [0.0, 0.15])
def test_misaligned_gradients_use_element_access_with_identical_results(dropout_p):
    rows, hidden = 23, 384
    inputs = make_inputs((rows, hidden), torch.float16, seed=409)
    torch.cuda.manual_seed(1)
    outputs = _C.residual_layer_norm_forward(*inputs, dropout_p, 1e-5, True, 128)
    grad_updated, grad_normalized = make_grads((rows, hidden), seed=410)
    storage = torch.empty(rows * hidden + 1, device="cuda")
    misaligned = storage[1:].view(rows, hidden)
    misaligned.copy_(grad_updated)
    assert misaligned.data_ptr() % 16 != 0
    with deterministic_algorithms(True):
        aligned = raw_backward(grad_updated, grad_normalized, outputs, inputs[2], dropout_p, True)
        scalar = raw_backward(misaligned, grad_normalized, outputs, inputs[2], dropout_p, True)
    for a, b in zip(aligned, scalar):
        assert_bitwise(host(b), host(a))


def test_atomic_mode_is_close_to_deterministic_mode():
    rows, hidden = 8192, 768
    inputs = make_inputs((rows, hidden), torch.float16, seed=5)
    grad_updated, grad_normalized = make_grads((rows, hidden), seed=6)
    outputs = _C.residual_layer_norm_forward(*inputs, 0.0, 1e-5, True, 128)
    with deterministic_algorithms(False):
        atomic = raw_backward(grad_updated, grad_normalized, outputs, inputs[2], 0.0, True)
    with deterministic_algorithms(True):
        fixed = raw_backward(grad_updated, grad_normalized, outputs, inputs[2], 0.0, True)
    assert_bitwise(host(atomic[0]), host(fixed[0]), "grad_x")
    assert_bitwise(host(atomic[1]), host(fixed[1]), "grad_branch")
    for a, b in zip(atomic[2:], fixed[2:]):
        scale = float(b.abs().max())
        assert float((a - b).abs().max()) <= 1e-5 * scale
    assert np.isfinite(host(fixed[2])).all()


# Row counts around the team walks' edges, per row shape: teams without rows,
# with one, two and three rows (the two-rows-ahead walk ends on one or two
# held rows), paced launches, two and four rows per wave, multi-wave rows.
EARLY_COMBINE_SHAPES = [(1, 768), (5, 768), (2048, 768), (4096, 768), (6144, 768),
                        (16384, 768), (3, 128), (1000, 256), (300, 1024), (77, 2048),
                        (33, 5952), (5000, 512)]


@pytest.mark.parametrize("rows,hidden", EARLY_COMBINE_SHAPES,
                         ids=[f"{r}x{h}" for r, h in EARLY_COMBINE_SHAPES])
def test_atomic_weight_bias_sums_match_the_fixed_order_sums(rows, hidden):
    """The atomic backward adds each block's sums in LDS and its last wave adds
    them into grad_weight / grad_bias, starting with the last rows'
    contributions before those rows' gradients are stored: the input
    gradients equal the deterministic backward's bit for bit, the weight/bias
    sums are within 1e-5 of its fixed-order sums (relative to their largest
    value), for row counts at every edge of the team walks."""
    print(f"[backward] atomic vs fixed-order sums {rows}x{hidden}", flush=True)
    inputs = make_inputs((rows, hidden), torch.float16, seed=rows + hidden)
    grad_updated, grad_normalized = make_grads((rows, hidden), seed=7 + rows)
    torch.cuda.manual_seed(3)
    outputs = _C.residual_layer_norm_forward(*inputs, 0.1, 1e-5, True, 128)
    with deterministic_algorithms(False):
        atomic = raw_backward(grad_updated, grad_normalized, outputs, inputs[2], 0.1, True)
    with deterministic_algorithms(True):
        fixed = raw_backward(grad_updated, grad_normalized, outputs, inputs[2], 0.1, True)
    assert_bitwise(host(atomic[0]), host(fixed[0]), "grad_x")
    assert_bitwise(host(atomic[1]), host(fixed[1]), "grad_branch")
    for a, b, name in zip(atomic[2:], fixed[2:], ("grad_weight", "grad_bias")):
        scale = float(b.abs().max())
        assert float((a - b).abs().max()) <= 1e-5 * scale, name


@pytest.mark.parametrize("deterministic", [False, True], ids=["atomic", "deterministic"])
def test_repeated_backward_of_one_forward(deterministic):
    """The first backward of a call accumulates into sums its forward zeroed;
    a second backward of the same graph (retain_graph) must give the same
    gradients, not twice them."""
    rows, hidden = 129, 768
    leaves = [t.requires_grad_(True) for t in make_inputs((rows, hidden), torch.float16, seed=5)]
    grad_updated, grad_normalized = make_grads((rows, hidden), seed=6)
    with deterministic_algorithms(deterministic):
        updated, normalized = residual_layer_norm(*leaves, dropout_p=0.1, eps=1e-5,
                                                  training=True, implementation="gfx950")
        first = torch.autograd.grad((updated, normalized), leaves,
                                    (grad_updated, grad_normalized), retain_graph=True)
        second = torch.autograd.grad((updated, normalized), leaves,
                                     (grad_updated, grad_normalized))
    for name, a, b in zip(("x", "branch", "weight", "bias"), first, second):
        if deterministic:
            assert_bitwise(host(a), host(b), name)
        else:
            assert torch.allclose(a.float(), b.float(), rtol=1e-5, atol=1e-5), name
    assert first[2].data_ptr() != second[2].data_ptr()


@pytest.mark.parametrize("path", ["eager", "custom_op"])
def test_backward_skips_the_parameter_sums_it_does_not_need(path):
    """A backward pass that needs no weight/bias gradient (frozen LayerNorm
    parameters, or torch.autograd.grad over x and branch alone) skips their
    reduction. Its input gradients equal the full backward's bit for bit, it
    produces no parameter gradient, and a later pass over the same graph
    (retain_graph) that asks for them gets the full backward's (deterministic
    sums, bitwise). Both the C++ autograd function (eager calls) and the
    registered custom op (torch.compile's path) are checked."""
    from gfx1010_kernels._ops import residual_layer_norm_op

    def call(x, branch, weight, bias):
        if path == "eager":
            return residual_layer_norm(x, branch, weight, bias, dropout_p=0.1,
                                       implementation="gfx950")
        return residual_layer_norm_op(x, branch, weight, bias, 0.1, 1e-5, True)

    inputs = make_inputs((3, 171, 768), torch.float16, seed=61)
    grads = make_grads((3, 171, 768), seed=62)

    def leaves(*requires):
        return [t.detach().clone().requires_grad_(r) for t, r in zip(inputs, requires)]

    with deterministic_algorithms(True):
        torch.cuda.manual_seed(5)
        full_leaves = leaves(True, True, True, True)
        full = torch.autograd.grad(call(*full_leaves), full_leaves, grads)

        torch.cuda.manual_seed(5)
        split_leaves = leaves(True, True, True, True)
        out = call(*split_leaves)
        inputs_only = torch.autograd.grad(out, split_leaves[:2], grads, retain_graph=True)
        parameters = torch.autograd.grad(out, split_leaves[2:], grads)

        torch.cuda.manual_seed(5)
        frozen = leaves(True, True, False, False)
        torch.autograd.backward(call(*frozen), grads)

    for name, actual, expected in zip(("grad_x", "grad_branch", "grad_weight", "grad_bias"),
                                      (*inputs_only, *parameters), full):
        assert_bitwise(host(actual), host(expected), f"split pass {name}")
    assert_bitwise(host(frozen[0].grad), host(full[0]), "frozen grad_x")
    assert_bitwise(host(frozen[1].grad), host(full[1]), "frozen grad_branch")
    assert frozen[2].grad is None and frozen[3].grad is None


@pytest.mark.parametrize("deterministic", [False, True], ids=["atomic", "deterministic"])
def test_training_step_allocates_only_its_outputs_and_saved_state(deterministic):
    """Device memory of one training step through the public API: the forward
    allocates `updated`, `normalized`, one row-statistics tensor (mean, rstd
    and the dropout mask words, each 256-byte aligned) and the two
    weight/bias sums; the backward adds grad_x, grad_branch and, in
    deterministic mode, the per-block partials. Nothing else: no copy of an
    input or of an upstream gradient (the caching allocator rounds each
    allocation up to 512 bytes)."""
    from gfx1010_kernels import _cabi

    rows, hidden = 4096, 1024
    inputs = make_inputs((rows, hidden), torch.float16, seed=91)
    grads = make_grads((rows, hidden), seed=92)
    leaves = [t.detach().clone().requires_grad_(True) for t in inputs]

    def rounded(nbytes):
        return (nbytes + 511) // 512 * 512

    aligned_rows = (rows + 63) // 64 * 64
    forward_bytes = (2 * rounded(rows * hidden * 4)
                     + rounded(4 * (2 * aligned_rows + rows * hidden // 32))
                     + 2 * rounded(hidden * 4))
    workspace = _cabi.backward_workspace_bytes(rows, hidden, deterministic)
    backward_bytes = (rounded(rows * hidden * 4) + rounded(rows * hidden * 2)
                      + (rounded(workspace) if workspace else 0))

    with deterministic_algorithms(deterministic):
        torch.cuda.synchronize()
        base = torch.cuda.memory_allocated()
        outputs = residual_layer_norm(*leaves, dropout_p=0.1, implementation="gfx950")
        assert torch.cuda.memory_allocated() - base == forward_bytes
        torch.cuda.reset_peak_memory_stats()
        gradients = torch.autograd.grad(outputs, leaves, grads)
        torch.cuda.synchronize()
        peak = torch.cuda.max_memory_allocated() - base
    assert peak == forward_bytes + backward_bytes, (peak, forward_bytes, backward_bytes)
    assert gradients[1].dtype == torch.float16


def test_inference_call_keeps_only_its_outputs():
    """Under torch.no_grad() a call keeps `updated` and `normalized` alone: no
    saved state, no gradient sums (the row statistics it writes are freed
    when it returns)."""
    rows, hidden = 4096, 1024
    inputs = [t.detach().clone().requires_grad_(True)
              for t in make_inputs((rows, hidden), torch.float16, seed=93)]
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    with torch.no_grad():
        updated, normalized = residual_layer_norm(*inputs, dropout_p=0.1,
                                                  normalized_dtype=torch.bfloat16,
                                                  implementation="gfx950")
    torch.cuda.synchronize()
    rounded = lambda nbytes: (nbytes + 511) // 512 * 512  # noqa: E731
    assert torch.cuda.memory_allocated() - base == (rounded(rows * hidden * 4)
                                                    + rounded(rows * hidden * 2))
    assert normalized.dtype == torch.bfloat16 and updated.grad_fn is None
