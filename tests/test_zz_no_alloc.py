"""rln_backward_noalloc against rln_backward, through the C ABI.

The no-allocation backward keeps the deterministic weight/bias partials in
the library's static per-device scratch instead of a caller workspace; its
results must be rln_backward's: bit for bit in deterministic mode (same
kernels, same fixed-order sums), and in atomic mode the input gradients bit
for bit and the weight/bias sums within the 1e-4 parity bar. Two calls in a
row, the second over a smaller input, so the second reads a scratch the first
left full (nothing in it may need clearing).
"""

import pytest
import torch

from gfx1010_kernels import _cabi
from parity import TOL_PARAMETER_GRAD, assert_normwise, host

pytestmark = pytest.mark.gpu
EPS = 1e-5
CODE = {torch.float32: _cabi.RLN_DTYPE_F32, torch.float16: _cabi.RLN_DTYPE_F16,
        torch.bfloat16: _cabi.RLN_DTYPE_BF16}
# (rows, hidden, branch dtype, dropout_p): the second call is smaller.
CALLS = [(8192, 2048, torch.float16, 0.1), (300, 768, torch.bfloat16, 0.0)]


def forward_state(rows, hidden, branch_dtype, dropout_p, seed):
    generator = torch.Generator(device="cuda").manual_seed(seed)

    def randn(*shape):
        return torch.randn(*shape, device="cuda", generator=generator)

    x, branch = randn(rows, hidden), (0.5 * randn(rows, hidden)).to(branch_dtype)
    weight, bias = 1.0 + 0.02 * randn(hidden), 0.02 * randn(hidden)
    state = dict(
        branch_dtype=branch_dtype, weight=weight,
        grad_updated=randn(rows, hidden), grad_normalized=randn(rows, hidden),
        updated=torch.empty(rows, hidden, device="cuda"),
        normalized=torch.empty(rows, hidden, device="cuda"),
        mean=torch.empty(rows, device="cuda"), rstd=torch.empty(rows, device="cuda"),
        mask=torch.zeros(max(_cabi.mask_words(rows, hidden), 1), device="cuda",
                         dtype=torch.int32))
    stream = torch.cuda.current_stream().cuda_stream
    _cabi.forward(x.data_ptr(), branch.data_ptr(), CODE[branch_dtype], weight.data_ptr(),
                  bias.data_ptr(), state["updated"].data_ptr(), state["normalized"].data_ptr(),
                  state["mean"].data_ptr(), state["rstd"].data_ptr(), state["mask"].data_ptr(),
                  rows, hidden, dropout_p, EPS, True, _cabi.RlnPhilox(seed, 8, None, None),
                  stream)
    return state


def gradients(state, rows, hidden, dropout_p, deterministic, noalloc):
    out = dict(grad_x=torch.empty(rows, hidden, device="cuda"),
               grad_branch=torch.empty(rows, hidden, device="cuda", dtype=state["branch_dtype"]),
               parameters=torch.full((2, hidden), float("nan"), device="cuda"))
    args = (state["grad_updated"].data_ptr(), state["grad_normalized"].data_ptr(),
            state["updated"].data_ptr(), state["weight"].data_ptr(), state["mean"].data_ptr(),
            state["rstd"].data_ptr(), state["mask"].data_ptr(), out["grad_x"].data_ptr(),
            out["grad_branch"].data_ptr(), CODE[state["branch_dtype"]],
            out["parameters"][0].data_ptr(), out["parameters"][1].data_ptr(), rows, hidden,
            dropout_p, True, deterministic)
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        _cabi.backward_noalloc(*args, stream=stream)
    else:
        size = _cabi.backward_workspace_bytes(rows, hidden, deterministic)
        workspace = torch.empty(max(size, 16), device="cuda", dtype=torch.uint8)
        _cabi.backward(*args, workspace=workspace.data_ptr(), workspace_bytes=size,
                       stream=stream)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("deterministic", [True, False], ids=["deterministic", "atomic"])
def test_noalloc_backward_matches_the_workspace_backward(deterministic):
    for index, (rows, hidden, branch_dtype, dropout_p) in enumerate(CALLS):
        print(f"[noalloc] call {index}: rows={rows} H={hidden} {branch_dtype} p={dropout_p} "
              f"deterministic={deterministic}", flush=True)
        assert (_cabi.backward_workspace_bytes(rows, hidden, True)
                <= _cabi.NOALLOC_SCRATCH_BYTES)
        state = forward_state(rows, hidden, branch_dtype, dropout_p, seed=91 + index)
        expected = gradients(state, rows, hidden, dropout_p, deterministic, noalloc=False)
        actual = gradients(state, rows, hidden, dropout_p, deterministic, noalloc=True)
        for name in ("grad_x", "grad_branch"):
            assert torch.equal(actual[name], expected[name]), name
        if deterministic:
            assert torch.equal(actual["parameters"], expected["parameters"])
        else:
            assert_normwise(host(actual["parameters"]), host(expected["parameters"]),
                            TOL_PARAMETER_GRAD, "weight/bias sums")


NOALLOC_FIRST_CALL_UNDER_CAPTURE = r"""
import sys
import torch
sys.path.insert(0, sys.argv[1])
from gfx1010_kernels import _cabi

rows, hidden, dropout_p = 2049, 768, 0.1
generator = torch.Generator(device="cuda").manual_seed(17)
def randn(*shape):
    return torch.randn(*shape, device="cuda", generator=generator)
x, branch = randn(rows, hidden), (0.5 * randn(rows, hidden)).half()
weight, bias = 1.0 + 0.02 * randn(hidden), 0.02 * randn(hidden)
grad_updated, grad_normalized = randn(rows, hidden), randn(rows, hidden)
updated, normalized = torch.empty(rows, hidden, device="cuda"), torch.empty(rows, hidden, device="cuda")
mean, rstd = torch.empty(rows, device="cuda"), torch.empty(rows, device="cuda")
mask = torch.zeros(_cabi.mask_words(rows, hidden), device="cuda", dtype=torch.int32)
stream = torch.cuda.current_stream().cuda_stream
_cabi.forward(x.data_ptr(), branch.data_ptr(), _cabi.RLN_DTYPE_F16, weight.data_ptr(),
              bias.data_ptr(), updated.data_ptr(), normalized.data_ptr(), mean.data_ptr(),
              rstd.data_ptr(), mask.data_ptr(), rows, hidden, dropout_p, 1e-5, True,
              _cabi.RlnPhilox(5, 8, None, None), stream)
torch.cuda.synchronize()

def outputs():
    return dict(grad_x=torch.empty(rows, hidden, device="cuda"),
                grad_branch=torch.empty(rows, hidden, device="cuda", dtype=torch.float16),
                grad_weight=torch.full((hidden,), float("nan"), device="cuda"),
                grad_bias=torch.full((hidden,), float("nan"), device="cuda"))

def arguments(out):
    return (grad_updated.data_ptr(), grad_normalized.data_ptr(), updated.data_ptr(),
            weight.data_ptr(), mean.data_ptr(), rstd.data_ptr(), mask.data_ptr(),
            out["grad_x"].data_ptr(), out["grad_branch"].data_ptr(), _cabi.RLN_DTYPE_F16,
            out["grad_weight"].data_ptr(), out["grad_bias"].data_ptr(), rows, hidden,
            dropout_p, True, True)

captured = outputs()
graph = torch.cuda.CUDAGraph()
side = torch.cuda.Stream()
side.wait_stream(torch.cuda.current_stream())
with torch.cuda.stream(side):
    with torch.cuda.graph(graph, stream=side):
        # The process's first rln_backward_noalloc call: its one-time lookup
        # of the device's scratch address runs during capture.
        _cabi.backward_noalloc(*arguments(captured), stream=side.cuda_stream)
torch.cuda.current_stream().wait_stream(side)
size = _cabi.backward_workspace_bytes(rows, hidden, True)
workspace = torch.empty(size, device="cuda", dtype=torch.uint8)
for replay in range(3):
    for tensor in captured.values():
        tensor.fill_(float("nan"))
    graph.replay()
    torch.cuda.synchronize()
    eager = outputs()
    _cabi.backward(*arguments(eager), workspace=workspace.data_ptr(), workspace_bytes=size,
                   stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for name in captured:
        assert torch.equal(captured[name], eager[name]), f"replay {replay}: {name} differs"
print("first noalloc call under capture: ok", flush=True)
"""


def test_first_noalloc_call_of_a_process_under_capture():
    """rln_backward_noalloc serves callers under HIP graph capture: the first
    call of a fresh process (which looks up the device's scratch address)
    captured into a graph, in deterministic mode, replays bit for bit like an
    eager rln_backward with a caller workspace, three times, with the outputs
    poisoned before each replay and eager work between replays."""
    import subprocess
    import sys
    from pathlib import Path

    package = Path(__file__).resolve().parents[1] / "gfx1010-kernels_amd"
    print("[noalloc] first call under capture (child process)", flush=True)
    result = subprocess.run([sys.executable, "-c", NOALLOC_FIRST_CALL_UNDER_CAPTURE,
                             str(package)], capture_output=True, text=True, timeout=240)
    assert result.returncode == 0, result.stdout + result.stderr
    assert "first noalloc call under capture: ok" in result.stdout
