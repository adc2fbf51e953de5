"""A whole training step of the op (forward + backward) under HIP graph capture.

The captured graph holds the forward, the weight/bias zeroing kernel (atomic
mode) or the fixed-order reduce kernel (deterministic mode) and the backward;
no memset node. Each replay, with eager work and synchronizations between
replays, draws a fresh dropout mask from the generator and must match the
oracle for the RNG state it consumed (the reference rejects capture,
csrc/residual_layer_norm_kernel.hip:1758-1777).
"""

import numpy as np
import pytest
import torch

from gfx1010_kernels import _C
from parity import (
    check_backward,
    check_forward,
    generator_state,
    host,
    make_grads,
    make_inputs,
    philox_increment,
)
from test_gpu_backward import deterministic_algorithms, raw_backward

pytestmark = pytest.mark.gpu
EPS = 1e-5


@pytest.mark.parametrize("hidden", [768, 2048])
@pytest.mark.parametrize("deterministic", [False, True], ids=["atomic", "deterministic"])
def test_captured_training_step_replays(hidden, deterministic):
    rows = 300
    inputs = make_inputs((rows, hidden), torch.float16, seed=hidden)
    grad_updated, grad_normalized = make_grads((rows, hidden), seed=hidden + 1)
    torch.cuda.manual_seed(7)

    def step():
        outputs = _C.residual_layer_norm_forward(*inputs, 0.1, EPS, True, 128)
        gradients = raw_backward(grad_updated, grad_normalized, outputs, inputs[2], 0.1, True)
        return outputs, gradients

    with deterministic_algorithms(deterministic):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            outputs, gradients = step()
        masks = []
        for replay in range(3):
            seed, offset = generator_state()
            graph.replay()
            torch.cuda.synchronize()
            keep, scale = check_forward(outputs, inputs, 0.1, True, EPS, seed, offset,
                                        f"replay {replay}")
            check_backward(gradients, grad_updated, grad_normalized, outputs[0], inputs[2], EPS,
                           keep, scale, f"replay {replay}")
            masks.append(host(outputs[4]).copy())
            step()  # eager work between replays
            torch.cuda.synchronize()
    assert not np.array_equal(masks[0], masks[1]) and not np.array_equal(masks[1], masks[2])


@pytest.mark.parametrize("hidden,threads", [(1024, 192), (128, 256), (384, 128)])
def test_captured_calls_draw_the_reference_stream_at_consecutive_offsets(hidden, threads):
    """Two forwards captured in one graph draw the reference's stream at the
    replay's base offset and at base + the reference's increment (8 at
    H = 1024 with 192 threads, 4 below), read from the generator's device
    pointers at replay time."""
    rows = 97
    inputs = make_inputs((rows, hidden), torch.float16, seed=hidden + threads)
    torch.cuda.manual_seed(11)

    def calls():
        return [_C.residual_layer_norm_forward(*inputs, 0.2, EPS, True, threads)
                for _ in range(2)]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        calls()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outputs = calls()
    increment = philox_increment(hidden, threads)
    for replay in range(2):
        seed, offset = generator_state()
        graph.replay()
        torch.cuda.synchronize()
        for index, output in enumerate(outputs):
            check_forward(output, inputs, 0.2, True, EPS, seed, offset + index * increment,
                          f"replay {replay} call {index}", threads=threads)
        assert generator_state()[1] == offset + 2 * increment


FIRST_CALL_UNDER_CAPTURE = r"""
import sys
import torch
sys.path.insert(0, sys.argv[1])
from gfx1010_kernels import _C

rows, hidden = 3001, 896
generator = torch.Generator(device="cuda").manual_seed(5)
x = torch.randn(rows, hidden, device="cuda", generator=generator)
branch = torch.randn(rows, hidden, device="cuda", generator=generator).half()
weight = torch.randn(hidden, device="cuda", generator=generator)
bias = torch.randn(hidden, device="cuda", generator=generator)
grad = torch.randn(rows, hidden, device="cuda", generator=generator)
torch.cuda.synchronize()

def step():
    out = _C.residual_layer_norm_forward(x, branch, weight, bias, 0.0, 1e-5, True, 128)
    grads = _C.residual_layer_norm_backward(grad, grad, out[0], weight, out[2], out[3], out[4],
                                            0.0, True, True, 128, 64, 64, 1, True)
    return out, grads

graph = torch.cuda.CUDAGraph()
side = torch.cuda.Stream()
side.wait_stream(torch.cuda.current_stream())
with torch.cuda.stream(side):
    with torch.cuda.graph(graph, stream=side):
        captured = step()
torch.cuda.current_stream().wait_stream(side)
for replay in range(3):
    graph.replay()
    torch.cuda.synchronize()
    eager = step()
    torch.cuda.synchronize()
    for a, b in zip(list(captured[0][:4]) + list(captured[1][:2]),
                    list(eager[0][:4]) + list(eager[1][:2])):
        assert torch.equal(a, b), f"replay {replay} differs from the eager call"
print("first call under capture: ok", flush=True)
"""


def test_first_call_of_a_process_under_capture():
    """The first forward and backward of a process captured into a graph: the
    library's one-time device queries (compute units, the forward kernel's
    resident blocks per CU) then run during capture, and must neither break
    it nor change results (replays against eager calls, bitwise; p = 0)."""
    import subprocess
    import sys
    from pathlib import Path

    package = Path(__file__).resolve().parents[1] / "gfx1010-kernels_amd"
    print("[graphs] first call under capture (child process)", flush=True)
    result = subprocess.run([sys.executable, "-c", FIRST_CALL_UNDER_CAPTURE, str(package)],
                            capture_output=True, text=True, timeout=240)
    assert result.returncode == 0, result.stdout + result.stderr
    assert "first call under capture: ok" in result.stdout


@pytest.mark.parametrize("training,dropout_p", [(False, 0.0), (True, 0.1)],
                         ids=["eval", "dropout"])
def test_captured_inference_calls_replay(training, dropout_p):
    """Public calls under torch.no_grad() (the forward-only path, no autograd
    node) captured in a HIP graph, as a serving loop would: each replay over
    new values copied into the static inputs equals, bit for bit, an eager
    call on those values from the same generator state, with eager work
    between replays; with dropout, each replay draws from a new offset of the
    generator (a fresh mask), without dropout none is consumed."""
    from gfx1010_kernels import residual_layer_norm

    rows, hidden = 257, 1024
    x, branch, weight, bias = make_inputs((rows, hidden), torch.float16, seed=31)
    fresh = [make_inputs((rows, hidden), torch.float16, seed=40 + i)[:2] for i in range(3)]
    generator = torch.cuda.default_generators[0]
    torch.cuda.manual_seed(11)

    def call(x_values, branch_values):
        return residual_layer_norm(x_values, branch_values, weight, bias, dropout_p=dropout_p,
                                   training=training, implementation="gfx950")

    with torch.no_grad():
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            call(x, branch)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            captured = call(x, branch)
        offsets = []
        for x_values, branch_values in fresh:
            x.copy_(x_values)
            branch.copy_(branch_values)
            offset = generator.get_offset()
            offsets.append(offset)
            graph.replay()
            torch.cuda.synchronize()
            replayed = [host(t).copy() for t in captured]
            generator.set_offset(offset)
            eager = call(x_values, branch_values)  # eager work between replays
            torch.cuda.synchronize()
            for actual, expected in zip(replayed, eager):
                assert np.array_equal(actual.view(np.uint32), host(expected).view(np.uint32))
    if dropout_p > 0.0:
        assert offsets[0] < offsets[1] < offsets[2]
    else:
        assert offsets[0] == offsets[1] == offsets[2]
