"""The C ABI from a plain C program: HIP runtime only, no torch.

tests/cabi_host/rln_host.c allocates device memory with hipMalloc, runs one
rln_forward + rln_backward through include/rln.h (the forward zeroing the
parameter sums the backward accumulates into) and writes every output; this
test feeds it seeded inputs and checks the outputs against the oracle: the
mask and ``updated`` bit for bit, the rest within the parity tolerances. The
binary is built by ``__graft_entry__.build()`` (``make -C tests/cabi_host``).
"""

import subprocess
from pathlib import Path

import numpy as np
import pytest

from oracle import rln_oracle as oracle
from parity import (
    TOL_FORWARD,
    TOL_INPUT_GRAD,
    TOL_PARAMETER_GRAD,
    assert_bitwise,
    assert_fp16_close,
    assert_normwise,
)

pytestmark = pytest.mark.gpu
HOST = Path(__file__).resolve().parent / "cabi_host" / "rln_host"
EPS = 1e-5


@pytest.mark.parametrize(
    "rows,hidden,threads,deterministic",
    [(37, 768, 128, 0), (20, 1024, 192, 1), (9, 128, 256, 0), (11, 1600, 0, 1)])
def test_plain_c_host_matches_oracle(tmp_path, rows, hidden, threads, deterministic):
    assert HOST.exists(), "tests/cabi_host/rln_host is not built (make -C tests/cabi_host)"
    rng = np.random.default_rng(rows * hidden + threads)
    x = rng.standard_normal((rows, hidden), dtype=np.float32)
    branch = (0.5 * rng.standard_normal((rows, hidden))).astype(np.float16)
    weight = (1.0 + 0.02 * rng.standard_normal(hidden)).astype(np.float32)
    bias = (0.02 * rng.standard_normal(hidden)).astype(np.float32)
    grad_updated = rng.standard_normal((rows, hidden), dtype=np.float32)
    grad_normalized = rng.standard_normal((rows, hidden), dtype=np.float32)
    seed, offset, dropout_p = 0x0123_4567_89AB_CDEF, 4 * 321, 0.15

    source, target = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(source, "wb") as file:
        np.array([rows, hidden, threads, seed, offset, deterministic], np.int64).tofile(file)
        np.array([dropout_p, EPS], np.float64).tofile(file)
        for array in (x, branch, weight, bias, grad_updated, grad_normalized):
            array.tofile(file)
    print(f"[cabi-host] rows={rows} H={hidden} T={threads} det={deterministic}", flush=True)
    result = subprocess.run([str(HOST), str(source), str(target)], capture_output=True,
                            text=True, timeout=120)
    assert result.returncode == 0, result.stderr

    data = np.fromfile(target, np.uint8)
    n, words = rows * hidden, rows * hidden // 32
    layout = [("updated", np.float32, n), ("normalized", np.float32, n),
              ("mean", np.float32, rows), ("rstd", np.float32, rows),
              ("mask", np.uint32, words), ("grad_x", np.float32, n),
              ("grad_branch", np.float16, n), ("grad_weight", np.float32, hidden),
              ("grad_bias", np.float32, hidden)]
    out, position = {}, 0
    for name, dtype, count in layout:
        size = np.dtype(dtype).itemsize * count
        out[name] = data[position:position + size].view(dtype)
        position += size
    assert position == data.size

    active, scale, threshold = oracle.dropout_constants(dropout_p)
    if threads:
        expected_words = oracle.reference_mask_words(rows, hidden, threads, seed, offset,
                                                     threshold)
    else:
        expected_words = oracle.dropout_mask_words(rows, hidden, seed, offset, threshold)
    assert_bitwise(out["mask"], expected_words, "mask")
    keep = oracle.decode_mask(expected_words, rows, hidden)
    forward = oracle.forward(x, branch, weight, bias, EPS, keep=keep, scale=scale)
    assert_bitwise(out["updated"].reshape(rows, hidden), forward["updated"], "updated")
    assert_normwise(out["normalized"].reshape(rows, hidden), forward["normalized"],
                    TOL_FORWARD, "normalized")
    assert_normwise(out["mean"], forward["mean"], TOL_FORWARD, "mean")
    assert_normwise(out["rstd"], forward["rstd"], TOL_FORWARD, "rstd")
    backward = oracle.backward(grad_updated, grad_normalized, forward["updated"], weight, EPS,
                               keep=keep, scale=scale)
    assert_normwise(out["grad_x"].reshape(rows, hidden), backward["grad_x"], TOL_INPUT_GRAD,
                    "grad_x")
    assert_fp16_close(out["grad_branch"].reshape(rows, hidden), backward["grad_branch"],
                      "grad_branch")
    assert_normwise(out["grad_weight"], backward["grad_weight"], TOL_PARAMETER_GRAD,
                    "grad_weight")
    assert_normwise(out["grad_bias"], backward["grad_bias"], TOL_PARAMETER_GRAD, "grad_bias")
