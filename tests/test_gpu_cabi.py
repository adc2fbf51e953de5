"""The C ABI on the GPU: both weight/bias reduction modes, gradient
accumulation, workspace reuse across shapes, and a backward without
parameter gradients.

Calls go through librln_gfx950.so with torch tensors as device memory only;
results are checked against the fp64 oracle.
"""

import numpy as np
import pytest
import torch

from gfx1010_kernels import _cabi
from parity import (
    TOL_PARAMETER_GRAD,
    assert_bitwise,
    assert_normwise,
    check_backward,
    check_forward,
    host,
    make_grads,
    make_inputs,
)

pytestmark = pytest.mark.gpu
EPS = 1e-5


def forward(inputs, dropout_p, seed, offset):
    x, branch, weight, bias = inputs
    rows, hidden = x.shape
    out = dict(
        updated=torch.empty_like(x),
        normalized=torch.empty_like(x),
        mean=torch.empty(rows, device="cuda"),
        rstd=torch.empty(rows, device="cuda"),
        mask=torch.zeros(_cabi.mask_words(rows, hidden), device="cuda", dtype=torch.int32),
    )
    dtype = _cabi.RLN_DTYPE_F16 if branch.dtype == torch.float16 else _cabi.RLN_DTYPE_F32
    _cabi.forward(x.data_ptr(), branch.data_ptr(), dtype, weight.data_ptr(), bias.data_ptr(),
                  out["updated"].data_ptr(), out["normalized"].data_ptr(), out["mean"].data_ptr(),
                  out["rstd"].data_ptr(), out["mask"].data_ptr(), rows, hidden, dropout_p, EPS,
                  True, _cabi.RlnPhilox(seed, offset, None, None),
                  torch.cuda.current_stream().cuda_stream)
    return out


def backward(out, grads, weight, branch_dtype, dropout_p, deterministic, accumulate,
             parameters, workspace):
    rows, hidden = out["updated"].shape
    grad_x = torch.empty_like(out["updated"])
    grad_branch = torch.empty(rows, hidden, device="cuda", dtype=branch_dtype)
    dtype = _cabi.RLN_DTYPE_F16 if branch_dtype == torch.float16 else _cabi.RLN_DTYPE_F32
    _cabi.backward(
        grads[0].data_ptr(), grads[1].data_ptr(), out["updated"].data_ptr(), weight.data_ptr(),
        out["mean"].data_ptr(), out["rstd"].data_ptr(), out["mask"].data_ptr(),
        grad_x.data_ptr(), grad_branch.data_ptr(), dtype, parameters[0].data_ptr(),
        parameters[1].data_ptr(), rows, hidden, dropout_p, True, deterministic,
        workspace.data_ptr() if workspace is not None else None,
        workspace.numel() if workspace is not None else 0,
        torch.cuda.current_stream().cuda_stream, accumulate_parameters=accumulate)
    return grad_x, grad_branch


def new_workspace(rows, hidden):
    """Uninitialised device memory of the size the deterministic backward needs."""
    size = _cabi.backward_workspace_bytes(rows, hidden, True)
    return torch.full((size,), 0xA5, device="cuda", dtype=torch.uint8)


@pytest.mark.parametrize(
    "rows,hidden",
    [(1, 128), (41, 768), (513, 768), (2049, 128), (2049, 384), (20000, 1024)],
)
@pytest.mark.parametrize("deterministic", [False, True], ids=["atomic", "deterministic"])
def test_parameter_gradients_and_accumulation(rows, hidden, deterministic):
    inputs = make_inputs((rows, hidden), torch.float16, seed=rows * 7 + hidden)
    grads = make_grads((rows, hidden), seed=rows + 3)
    seed, offset = 0x1234_5678_9ABC, 4 * rows
    out = forward(inputs, 0.1, seed, offset)
    torch.cuda.synchronize()
    keep, scale = check_forward((out["updated"], out["normalized"], out["mean"], out["rstd"],
                                 out["mask"]), inputs, 0.1, True, EPS, seed, offset, "c-abi",
                                threads=0)
    parameters = torch.full((2, hidden), float("nan"), device="cuda")
    workspace = new_workspace(rows, hidden) if deterministic else None
    grad_x, grad_branch = backward(out, grads, inputs[2], torch.float16, 0.1, deterministic,
                                   False, parameters, workspace)
    torch.cuda.synchronize()
    check_backward((grad_x, grad_branch, parameters[0], parameters[1]), grads[0], grads[1],
                   out["updated"], inputs[2], EPS, keep, scale, f"rows={rows} H={hidden}")
    first = host(parameters).copy()

    # Accumulate a second backward of the same batch into the same outputs.
    backward(out, grads, inputs[2], torch.float16, 0.1, deterministic, True, parameters,
             workspace)
    torch.cuda.synchronize()
    if deterministic:
        # The fixed-order sum is reproduced exactly, and first + first is exact.
        assert_bitwise(host(parameters), first * np.float32(2.0), "accumulated")
    else:
        assert_normwise(host(parameters), 2.0 * first.astype(np.float64), TOL_PARAMETER_GRAD,
                        "accumulated")


def test_one_workspace_serves_consecutive_shapes_bitwise():
    """Calls of different shapes reuse one workspace; each result equals the
    result computed with a fresh workspace, bit for bit."""
    hidden = 768
    largest = new_workspace(4096, hidden)
    for rows in (4096, 37, 1000, 4096):
        inputs = make_inputs((rows, hidden), torch.float32, seed=rows)
        grads = make_grads((rows, hidden), seed=rows + 1)
        out = forward(inputs, 0.0, 0, 0)
        shared = torch.empty(2, hidden, device="cuda")
        fresh = torch.empty(2, hidden, device="cuda")
        backward(out, grads, inputs[2], torch.float32, 0.0, True, False, shared, largest)
        backward(out, grads, inputs[2], torch.float32, 0.0, True, False, fresh,
                 new_workspace(rows, hidden))
        torch.cuda.synchronize()
        assert_bitwise(host(shared), host(fresh), f"rows={rows}")


def test_backward_without_parameter_gradients():
    rows, hidden = 300, 512
    inputs = make_inputs((rows, hidden), torch.float16, seed=5)
    grads = make_grads((rows, hidden), seed=6)
    out = forward(inputs, 0.2, 77, 8)
    grad_x = torch.empty_like(out["updated"])
    grad_branch = torch.empty(rows, hidden, device="cuda", dtype=torch.float16)
    stream = torch.cuda.current_stream().cuda_stream
    _cabi.backward(
        grads[0].data_ptr(), grads[1].data_ptr(), out["updated"].data_ptr(),
        inputs[2].data_ptr(), out["mean"].data_ptr(), out["rstd"].data_ptr(),
        out["mask"].data_ptr(), grad_x.data_ptr(), grad_branch.data_ptr(), _cabi.RLN_DTYPE_F16,
        None, None, rows, hidden, 0.2, True, True, None, 0, stream)
    torch.cuda.synchronize()
    keep, scale = check_forward((out["updated"], out["normalized"], out["mean"], out["rstd"],
                                 out["mask"]), inputs, 0.2, True, EPS, 77, 8, threads=0)
    check_backward((grad_x, grad_branch, None, None), grads[0], grads[1], out["updated"],
                   inputs[2], EPS, keep, scale, "no parameters", parameters=False)


@pytest.mark.parametrize("hidden", [768, 1600])
@pytest.mark.parametrize("deterministic", [False, True], ids=["atomic", "deterministic"])
def test_forward_zeroes_the_parameter_sums_of_the_next_backward(hidden, deterministic):
    """rln_forward with zero_grad_weight / zero_grad_bias clears them (they
    start as NaN here); a backward that accumulates into them then yields the
    parameter gradients alone."""
    rows = 300
    inputs = make_inputs((rows, hidden), torch.float16, seed=hidden + 9)
    grads = make_grads((rows, hidden), seed=hidden + 10)
    x, branch, weight, bias = inputs
    sums = torch.full((2, hidden), float("nan"), device="cuda")
    out = dict(
        updated=torch.empty_like(x), normalized=torch.empty_like(x),
        mean=torch.empty(rows, device="cuda"), rstd=torch.empty(rows, device="cuda"),
        mask=torch.zeros(_cabi.mask_words(rows, hidden), device="cuda", dtype=torch.int32),
    )
    seed, offset = 99, 4 * rows
    _cabi.forward(x.data_ptr(), branch.data_ptr(), _cabi.RLN_DTYPE_F16, weight.data_ptr(),
                  bias.data_ptr(), out["updated"].data_ptr(), out["normalized"].data_ptr(),
                  out["mean"].data_ptr(), out["rstd"].data_ptr(), out["mask"].data_ptr(), rows,
                  hidden, 0.1, EPS, True, _cabi.RlnPhilox(seed, offset, None, None),
                  torch.cuda.current_stream().cuda_stream, zero_grad_weight=sums[0].data_ptr(),
                  zero_grad_bias=sums[1].data_ptr())
    torch.cuda.synchronize()
    assert torch.count_nonzero(sums).item() == 0 and not torch.isnan(sums).any()
    keep, scale = check_forward((out["updated"], out["normalized"], out["mean"], out["rstd"],
                                 out["mask"]), inputs, 0.1, True, EPS, seed, offset, "zeroing",
                                threads=0)
    workspace = new_workspace(rows, hidden) if deterministic else None
    grad_x, grad_branch = backward(out, grads, weight, torch.float16, 0.1, deterministic, True,
                                   sums, workspace)
    torch.cuda.synchronize()
    check_backward((grad_x, grad_branch, sums[0], sums[1]), grads[0], grads[1], out["updated"],
                   weight, EPS, keep, scale, f"H={hidden}")
