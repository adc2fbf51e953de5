"""Streams: every entry point runs on the caller's stream and never waits on the GPU.

The reference launches on the current HIP stream of the input's device and
returns without synchronizing (csrc/residual_layer_norm_kernel.hip:1743,
:1782-1783). The C ABI takes the stream as an argument (include/rln.h). Each
test first queues, on a side stream, a bounded spin (`torch.cuda._sleep`, a
clock loop that ends by itself) followed by a write of new input values. It
then calls the op on that stream: through the public API and the raw `_C`
entry points under `torch.cuda.stream(side)`, and through the C ABI with the
side stream passed while the default stream is current. Two properties
follow:

* the host call returned while the spin was still running (`side.query()` is
  False right after it), so the entry point did not wait for the GPU;
* the results are those of the new inputs, bit for bit against the same call
  made on settled data, so the launch was ordered after the write on that
  stream (a launch on another stream would have read the old values).

A last test calls the C ABI from two host threads at once, each on its own
stream, against the same calls made alone.
"""

import contextlib
import threading

import pytest
import torch

from gfx1010_kernels import _C, _cabi, residual_layer_norm
from parity import make_grads, make_inputs

pytestmark = pytest.mark.gpu
SPIN_CYCLES = 50_000_000  # tens of milliseconds: far longer than any host call here
EPS = 1e-5


def bits(tensor):
    return tensor.contiguous().view({4: torch.int32, 2: torch.int16}[tensor.element_size()])


def assert_same(actual, expected, what):
    assert torch.equal(bits(actual), bits(expected)), what


@contextlib.contextmanager
def deterministic():
    """torch.use_deterministic_algorithms(True) for a block (fixed-order
    weight/bias sums, so two calls agree bit for bit)."""
    previous = torch.are_deterministic_algorithms_enabled()
    torch.use_deterministic_algorithms(True)
    try:
        yield
    finally:
        torch.use_deterministic_algorithms(previous)


def queue_write_behind_spin(side, target, values):
    """On `side`: spin, then overwrite `target` with `values`."""
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        torch.cuda._sleep(SPIN_CYCLES)
        target.copy_(values)


def test_public_call_runs_on_the_current_stream_without_waiting():
    x, branch, weight, bias = make_inputs((1024, 768), torch.float16, seed=41)
    fresh = x + 0.5
    expected = residual_layer_norm(fresh, branch, weight, bias, implementation="gfx950")
    torch.cuda.synchronize()

    target = x.clone()
    side = torch.cuda.Stream()
    queue_write_behind_spin(side, target, fresh)
    with torch.cuda.stream(side):
        updated, normalized = residual_layer_norm(target, branch, weight, bias,
                                                  implementation="gfx950")
        waiting = not side.query()
    side.synchronize()
    assert waiting, "the public call waited for the GPU"
    assert_same(updated, expected[0], "updated")
    assert_same(normalized, expected[1], "normalized")


def test_raw_entry_points_run_on_the_current_stream_without_waiting():
    rows, hidden = 2048, 1024
    inputs = make_inputs((rows, hidden), torch.float16, seed=42)
    grad_updated, grad_normalized = make_grads((rows, hidden), seed=43)
    fresh_grad = grad_normalized * 2.0 - 0.25

    def backward(outputs, grad):
        return _C.residual_layer_norm_backward(
            grad_updated, grad, outputs[0], inputs[2], outputs[2], outputs[3], outputs[4],
            0.0, True, True, 192, 64, 64, 1, True)

    outputs = _C.residual_layer_norm_forward(*inputs, 0.0, EPS, True, 192)
    with deterministic():
        expected = backward(outputs, fresh_grad)
        torch.cuda.synchronize()

        target = grad_normalized.clone()
        side = torch.cuda.Stream()
        queue_write_behind_spin(side, target, fresh_grad)
        with torch.cuda.stream(side):
            forward = _C.residual_layer_norm_forward(*inputs, 0.0, EPS, True, 192)
            gradients = backward(outputs, target)
            waiting = not side.query()
        side.synchronize()
    assert waiting, "the raw entry points waited for the GPU"
    for name, actual, wanted in zip(("updated", "normalized", "mean", "rstd"), forward, outputs):
        assert_same(actual, wanted, name)
    for name, actual, wanted in zip(("grad_x", "grad_branch", "grad_weight", "grad_bias"),
                                    gradients, expected):
        assert_same(actual, wanted, name)


CODE = {torch.float32: _cabi.RLN_DTYPE_F32, torch.float16: _cabi.RLN_DTYPE_F16}
PHILOX = _cabi.RlnPhilox(0xABCDEF, 1 << 8, None, None, 0)


def c_abi_case(rows, hidden, seed):
    x, branch, weight, bias = make_inputs((rows, hidden), torch.float16, seed=seed)
    grad_updated, grad_normalized = make_grads((rows, hidden), seed=seed + 1)
    return dict(x=x, branch=branch, weight=weight, bias=bias, grad_updated=grad_updated,
                grad_normalized=grad_normalized)


def c_abi_buffers(case):
    rows, hidden = case["x"].shape
    workspace_bytes = _cabi.backward_workspace_bytes(rows, hidden, True)
    return dict(
        updated=torch.empty(rows, hidden, device="cuda"),
        normalized=torch.empty(rows, hidden, device="cuda"),
        mean=torch.empty(rows, device="cuda"), rstd=torch.empty(rows, device="cuda"),
        mask=torch.zeros(_cabi.mask_words(rows, hidden), device="cuda", dtype=torch.int32),
        grad_x=torch.empty(rows, hidden, device="cuda"),
        grad_branch=torch.empty(rows, hidden, device="cuda", dtype=case["branch"].dtype),
        sums=torch.empty(2, hidden, device="cuda"),
        workspace=torch.empty(workspace_bytes, device="cuda", dtype=torch.uint8))


C_ABI_OUTPUTS = ("updated", "normalized", "mean", "rstd", "mask", "grad_x", "grad_branch", "sums")


def c_abi_step(case, out, x, grad_normalized, stream):
    """rln_forward then rln_backward (p = 0.1, the library's own dropout layout,
    deterministic weight/bias sums) on `stream`."""
    rows, hidden = x.shape
    branch, weight = case["branch"], case["weight"]
    _cabi.forward(x.data_ptr(), branch.data_ptr(), CODE[branch.dtype], weight.data_ptr(),
                  case["bias"].data_ptr(), out["updated"].data_ptr(),
                  out["normalized"].data_ptr(), out["mean"].data_ptr(), out["rstd"].data_ptr(),
                  out["mask"].data_ptr(), rows, hidden, 0.1, EPS, True, PHILOX, stream)
    _cabi.backward(case["grad_updated"].data_ptr(), grad_normalized.data_ptr(),
                   out["updated"].data_ptr(), weight.data_ptr(), out["mean"].data_ptr(),
                   out["rstd"].data_ptr(), out["mask"].data_ptr(), out["grad_x"].data_ptr(),
                   out["grad_branch"].data_ptr(), CODE[branch.dtype], out["sums"][0].data_ptr(),
                   out["sums"][1].data_ptr(), rows, hidden, 0.1, True, True,
                   out["workspace"].data_ptr(), out["workspace"].numel(), stream)


@pytest.mark.parametrize("hidden,rows", [(768, 4096), (2048, 1024)])
def test_c_abi_runs_on_the_stream_it_is_given(hidden, rows):
    """rln_forward / rln_backward with an explicit side stream while the
    default stream is current."""
    case = c_abi_case(rows, hidden, seed=44)
    fresh_x = case["x"] * 0.5 + 1.0
    fresh_grad = case["grad_normalized"] - 1.0
    expected = c_abi_buffers(case)
    c_abi_step(case, expected, fresh_x, fresh_grad, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()

    actual = c_abi_buffers(case)
    x_target, grad_target = case["x"].clone(), case["grad_normalized"].clone()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    queue_write_behind_spin(side, x_target, fresh_x)
    with torch.cuda.stream(side):
        grad_target.copy_(fresh_grad)
    assert torch.cuda.current_stream() == torch.cuda.default_stream()
    c_abi_step(case, actual, x_target, grad_target, side.cuda_stream)
    waiting = not side.query()
    side.synchronize()
    assert waiting, "the C ABI waited for the GPU"
    for name in C_ABI_OUTPUTS:
        assert_same(actual[name], expected[name], name)


def test_c_abi_calls_from_two_host_threads_at_once():
    """Two host threads, each with its own stream, buffers and row shape, call
    rln_forward / rln_backward 12 times each at the same time (ctypes releases
    the GIL during the calls). Every result equals, bit for bit, the same call
    made alone: the library keeps no state that one call could leave for
    another (the error message is per thread, the device queries are made
    once)."""
    cases = [c_abi_case(2048, 768, seed=46), c_abi_case(512, 1600, seed=48)]
    expected = []
    for case in cases:
        out = c_abi_buffers(case)
        c_abi_step(case, out, case["x"], case["grad_normalized"],
                   torch.cuda.current_stream().cuda_stream)
        expected.append(out)
    torch.cuda.synchronize()

    barrier = threading.Barrier(len(cases), timeout=60)
    snapshots = [[] for _ in cases]
    errors = []

    def worker(index):
        try:
            case = cases[index]
            stream = torch.cuda.Stream()
            out = c_abi_buffers(case)
            barrier.wait()
            with torch.cuda.stream(stream):
                for _ in range(12):
                    c_abi_step(case, out, case["x"], case["grad_normalized"], stream.cuda_stream)
                    snapshots[index].append({name: out[name].clone() for name in C_ABI_OUTPUTS})
            stream.synchronize()
        except Exception as error:  # reported on the main thread
            errors.append(error)

    threads = [threading.Thread(target=worker, args=(index,)) for index in range(len(cases))]
    for thread in threads:
        thread.start()
    for thread in threads:
        thread.join(timeout=120)
    assert not errors, errors
    for index, case in enumerate(cases):
        assert len(snapshots[index]) == 12
        for step, snapshot in enumerate(snapshots[index]):
            for name in C_ABI_OUTPUTS:
                assert_same(snapshot[name], expected[index][name], f"case {index} step {step} {name}")
