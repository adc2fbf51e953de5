"""Dropout RNG contract on the GPU: the mask equals the oracle's Philox stream
for the (seed, offset) reserved from torch's generator; eval consumes no RNG;
consecutive calls use disjoint streams; restoring the RNG state replays the
mask; HIP graph replays draw fresh masks.

Reference behaviour: docs/residual_layer_norm.md:124-128,
tests/test_residual_layer_norm_edge_cases.py:76-95, :237-293, :339-375,
tests/test_residual_layer_norm.py:191-271.
"""

import numpy as np
import pytest
import torch

from gfx1010_kernels import _C, _cabi, residual_layer_norm
from oracle import rln_oracle as oracle
from parity import (
    API,
    REFERENCE_THREADS,
    assert_bitwise,
    check_forward,
    generator_state,
    host,
    make_inputs,
    philox_increment,
)

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("hidden,increment", [(128, 4), (512, 4), (768, 8), (1024, 8),
                                              (1600, 4)])
def test_call_reserves_the_reference_increment_only_when_dropout_is_active(hidden, increment):
    """The reference reserves 4 * ceil(ceil(H / threads) / 4) offset units per
    dropout call (csrc/residual_layer_norm_kernel.hip:1766-1770) with its
    threads table: 8 at H = 768 and 1024, 4 below; sizes the reference does
    not run natively reserve the library layout's 4."""
    inputs = make_inputs((8, hidden), torch.float16, seed=1)
    torch.cuda.manual_seed(5)
    _, start = generator_state()
    residual_layer_norm(*inputs, dropout_p=0.1, implementation="gfx950")
    assert generator_state()[1] == start + philox_increment(hidden, API) == start + increment
    residual_layer_norm(*inputs, dropout_p=0.1, training=False, implementation="gfx950")
    residual_layer_norm(*inputs, dropout_p=0.0, training=True, implementation="gfx950")
    assert generator_state()[1] == start + increment


def test_eval_bypasses_dropout_without_consuming_rng():
    inputs = make_inputs((7, 384), torch.float16, seed=101)
    cpu_state = torch.random.get_rng_state()
    gpu_state = torch.cuda.get_rng_state()
    updated, _ = residual_layer_norm(*inputs, dropout_p=0.8, training=False, implementation="gfx950")
    assert torch.equal(torch.random.get_rng_state(), cpu_state)
    assert torch.equal(torch.cuda.get_rng_state(), gpu_state)
    assert_bitwise(host(updated), host(inputs[0]) + host(inputs[1]).astype(np.float32))


def test_consecutive_calls_draw_the_next_disjoint_streams():
    inputs = make_inputs((3, 768), torch.float16, seed=127)
    torch.cuda.manual_seed(127)
    seed, offset = generator_state()
    first = _C.residual_layer_norm_forward(*inputs, 0.5, 1e-5, True, 128)
    second = _C.residual_layer_norm_forward(*inputs, 0.5, 1e-5, True, 128)
    check_forward(first, inputs, 0.5, True, 1e-5, seed, offset, "first")
    check_forward(second, inputs, 0.5, True, 1e-5, seed, offset + philox_increment(768),
                  "second")
    assert not torch.equal(first[4], second[4])
    # The reference's overlap probe (edge_cases:339-375).
    x = torch.zeros(3, 768, device="cuda")
    ones = torch.ones(3, 768, device="cuda", dtype=torch.float16)
    w, b = torch.ones(768, device="cuda"), torch.zeros(768, device="cuda")
    a = residual_layer_norm(x, ones, w, b, dropout_p=0.5, implementation="gfx950")[0]
    c = residual_layer_norm(x, ones, w, b, dropout_p=0.5, implementation="gfx950")[0]
    assert not torch.equal(a[:, 512:768], c[:, :256])


def test_restoring_rng_state_replays_mask_and_gradients():
    inputs = make_inputs((11, 384), torch.float16, seed=109)
    leaves = [tuple(t.detach().clone().requires_grad_(True) for t in inputs) for _ in range(2)]
    grad_updated = torch.linspace(-0.5, 0.5, 11 * 384, device="cuda").reshape(11, 384)
    grad_normalized = torch.cos(grad_updated)
    state = torch.cuda.get_rng_state()
    previous = torch.are_deterministic_algorithms_enabled()
    torch.use_deterministic_algorithms(True)
    try:
        first = residual_layer_norm(*leaves[0], dropout_p=0.25, implementation="gfx950")
        torch.cuda.set_rng_state(state)
        second = residual_layer_norm(*leaves[1], dropout_p=0.25, implementation="gfx950")
        first_grads = torch.autograd.grad(first, leaves[0], (grad_updated, grad_normalized))
        second_grads = torch.autograd.grad(second, leaves[1], (grad_updated, grad_normalized))
    finally:
        torch.use_deterministic_algorithms(previous)
    for a, b in zip((*first, *first_grads), (*second, *second_grads)):
        assert_bitwise(host(b), host(a))


@pytest.mark.parametrize("hidden", [128, 384, 1024])
@pytest.mark.parametrize("dropout_p", [0.15, 0.2])
def test_mask_scale_recovered_from_ones_branch(hidden, dropout_p):
    # Reference: tests/test_residual_layer_norm.py:191-223.
    rows = 43
    x = torch.randn(rows, hidden, device="cuda")
    branch = torch.ones(rows, hidden, device="cuda", dtype=torch.float16)
    w = torch.randn(hidden, device="cuda")
    b = torch.randn(hidden, device="cuda")
    updated, _ = residual_layer_norm(x, branch, w, b, dropout_p=dropout_p, implementation="gfx950")
    mask_scale = (updated - x) / branch.float()
    expected = torch.tensor([0.0, 1.0 / (1.0 - dropout_p)], device="cuda")
    distance = (mask_scale[..., None] - expected).abs().amin(dim=-1)
    assert distance.max().item() < 2e-3


@pytest.mark.parametrize("dropout_p", [0.1, 0.5, 0.9])
def test_keep_ratio_is_binomial(dropout_p):
    rows, hidden = 4096, 1024
    inputs = make_inputs((rows, hidden), torch.float16, seed=3)
    mask = _C.residual_layer_norm_forward(*inputs, dropout_p, 1e-5, True, 128)[4]
    kept = int(np.unpackbits(host(mask).view(np.uint8)).sum())
    n = rows * hidden
    assert abs(kept - n * (1 - dropout_p)) < 6 * np.sqrt(n * dropout_p * (1 - dropout_p))


def test_explicit_seed_and_offset_through_the_c_abi():
    rows, hidden = 19, 512
    x, branch, weight, bias = make_inputs((rows, hidden), torch.float32, seed=8)
    updated, normalized = torch.empty_like(x), torch.empty_like(x)
    mean = torch.empty(rows, device="cuda")
    rstd = torch.empty(rows, device="cuda")
    mask = torch.empty(_cabi.mask_words(rows, hidden), device="cuda", dtype=torch.int32)
    seed, offset = 0xDEADBEEF12345678, 4 * 1000
    stream = torch.cuda.current_stream().cuda_stream
    _cabi.forward(x.data_ptr(), branch.data_ptr(), _cabi.RLN_DTYPE_F32, weight.data_ptr(),
                  bias.data_ptr(), updated.data_ptr(), normalized.data_ptr(), mean.data_ptr(),
                  rstd.data_ptr(), mask.data_ptr(), rows, hidden, 0.3, 1e-5, True,
                  _cabi.RlnPhilox(seed, offset, None, None), stream)
    torch.cuda.synchronize()
    check_forward((updated, normalized, mean, rstd, mask), (x, branch, weight, bias), 0.3, True,
                  1e-5, seed, offset, "c-abi", threads=0)


def test_graph_replays_draw_fresh_masks_from_the_generator():
    rows, hidden = 64, 768
    inputs = make_inputs((rows, hidden), torch.float16, seed=12)
    torch.cuda.manual_seed(21)
    # Warm up on a side stream as torch.cuda.graphs recommends, then capture.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _C.residual_layer_norm_forward(*inputs, 0.1, 1e-5, True, 128)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = _C.residual_layer_norm_forward(*inputs, 0.1, 1e-5, True, 128)
    masks = []
    for replay in range(3):
        seed, offset = generator_state()
        graph.replay()
        torch.cuda.synchronize()
        check_forward(captured, inputs, 0.1, True, 1e-5, seed, offset, f"replay {replay}")
        masks.append(host(captured[4]).copy())
        # Eager work between replays.
        _C.residual_layer_norm_forward(*inputs, 0.1, 1e-5, True, 128)
        torch.cuda.synchronize()
    assert not np.array_equal(masks[0], masks[1]) and not np.array_equal(masks[1], masks[2])
    _, _, threshold = oracle.dropout_constants(0.1)
    assert threshold > 0
