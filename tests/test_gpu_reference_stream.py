"""The reference's own dropout stream on the GPU: masks equal the reference's.

On the reference's hidden sizes (128, 256, 384, 512, 768, 1024) the forward
draws hipRAND's Philox stream exactly as the reference's forward kernel does
for a launch of `threads` threads per row (csrc/residual_layer_norm_kernel.hip:449-511):
thread t of row r seeds hiprand_init(seed, r * threads + t, offset) and its
item i keeps column t + i * threads. The kernel reproduces it with ballots over
its own launch shape; these tests hold its masks to

* the fixtures written from rocRAND's own rocrand_init / rocrand4
  (tests/golden/hiprand_philox_vectors.json), directly, without the oracle;
* the oracle's restatement for every hidden size x threads x branch dtype x
  normalized dtype (which also fixes the kernel's lanes per row), in both row
  schedules, under the public API (the reference's threads table and Philox
  increments), and for rows whose subsequence r * threads + t passes 2^32.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from gfx1010_kernels import _C, _cabi, residual_layer_norm
from oracle import rln_oracle as oracle
from parity import (
    REFERENCE_THREADS,
    SPECIALIZED_HIDDEN_SIZES,
    assert_bitwise,
    check_forward,
    generator_state,
    host,
    make_inputs,
    philox_increment,
)

pytestmark = pytest.mark.gpu
EPS = 1e-5
VECTORS = json.loads(
    (Path(__file__).resolve().parent / "golden" / "hiprand_philox_vectors.json").read_text())
DTYPE = {torch.float32: _cabi.RLN_DTYPE_F32, torch.float16: _cabi.RLN_DTYPE_F16,
         torch.bfloat16: _cabi.RLN_DTYPE_BF16}


def cabi_forward(x, branch, weight, bias, dropout_p, seed, offset, threads,
                 normalized_dtype=torch.float32):
    rows, hidden = x.shape
    updated = torch.empty_like(x)
    normalized = torch.empty_like(x, dtype=normalized_dtype)
    mean = torch.empty(rows, device="cuda")
    rstd = torch.empty(rows, device="cuda")
    mask = torch.zeros(_cabi.mask_words(rows, hidden), device="cuda", dtype=torch.int32)
    _cabi.forward(x.data_ptr(), branch.data_ptr(), DTYPE[branch.dtype], weight.data_ptr(),
                  bias.data_ptr(), updated.data_ptr(), normalized.data_ptr(), mean.data_ptr(),
                  rstd.data_ptr(), mask.data_ptr(), rows, hidden, dropout_p, EPS, True,
                  _cabi.RlnPhilox(seed, offset, None, None, threads),
                  torch.cuda.current_stream().cuda_stream,
                  normalized_dtype=DTYPE[normalized_dtype])
    return updated, normalized, mean, rstd, mask


@pytest.mark.parametrize(
    "case", [case for case in VECTORS["masks"] if case["first_row"] < 64],
    ids=lambda c: f"H{c['hidden']}-T{c['threads']}-row{c['first_row']}-p{c['dropout_p']}")
def test_masks_equal_rocrand_fixtures(case):
    """Kernel masks against masks drawn through rocRAND itself (the rows
    [first_row, first_row + rows) of a launch over first_row + rows rows)."""
    first, hidden = case["first_row"], case["hidden"]
    rows = first + case["rows"]
    print(f"[reference-stream] fixture H={hidden} T={case['threads']} rows={rows}", flush=True)
    inputs = make_inputs((rows, hidden), torch.float16, seed=hidden + rows)
    outputs = cabi_forward(*inputs, case["dropout_p"], case["seed"], case["offset"],
                           case["threads"])
    torch.cuda.synchronize()
    words = host(outputs[4]).view(np.uint32)[first * (hidden // 32):]
    assert_bitwise(words, np.array(case["words"], np.uint32), "mask")


@pytest.mark.parametrize("normalized_dtype", [torch.float32, torch.float16],
                         ids=["n32", "n16"])
@pytest.mark.parametrize("branch_dtype", [torch.float16, torch.bfloat16, torch.float32],
                         ids=["b16", "bf16", "b32"])
@pytest.mark.parametrize("threads", [128, 192, 256])
@pytest.mark.parametrize("hidden", SPECIALIZED_HIDDEN_SIZES)
def test_forward_matches_oracle(hidden, threads, branch_dtype, normalized_dtype):
    rows = 37  # odd: the last wave of a multi-row shape holds past-the-end rows
    print(f"[reference-stream] H={hidden} T={threads} {branch_dtype} {normalized_dtype}",
          flush=True)
    inputs = make_inputs((rows, hidden), branch_dtype, seed=hidden * 7 + threads)
    torch.cuda.manual_seed(hidden + threads)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, 0.15, EPS, True, threads,
                                             normalized_dtype=normalized_dtype)
    torch.cuda.synchronize()
    check_forward(outputs, inputs, 0.15, True, EPS, seed, offset,
                  f"H={hidden} T={threads}", threads=threads)
    assert generator_state()[1] == offset + philox_increment(hidden, threads)


@pytest.mark.parametrize("hidden", [256, 768, 1024])
def test_paced_schedule_draws_the_same_stream(hidden):
    """A launch over 2^23 elements walks its rows paced; masks stay the
    reference's (checked on every row)."""
    rows = (1 << 23) // hidden + 5
    print(f"[reference-stream] paced rows={rows} H={hidden}", flush=True)
    inputs = make_inputs((rows, hidden), torch.float16, seed=hidden)
    seed, offset, threads = 0x5EED_0000_1234, 4 * 77, REFERENCE_THREADS[hidden]
    outputs = cabi_forward(*inputs, 0.1, seed, offset, threads)
    torch.cuda.synchronize()
    _, _, threshold = oracle.dropout_constants(0.1)
    expected = oracle.reference_mask_words(rows, hidden, threads, seed, offset, threshold)
    assert_bitwise(host(outputs[4]).view(np.uint32), expected, "mask")


def test_public_api_draws_the_reference_package_masks():
    """residual_layer_norm passes the reference's threads table: with a ones
    branch and zero x, updated = keep * scale exposes the mask, which equals
    the reference's for the generator state, call after call."""
    torch.cuda.manual_seed(2024)
    for hidden in SPECIALIZED_HIDDEN_SIZES:
        rows = 9
        x = torch.zeros(rows, hidden, device="cuda")
        ones = torch.ones(rows, hidden, device="cuda", dtype=torch.float16)
        w, b = torch.ones(hidden, device="cuda"), torch.zeros(hidden, device="cuda")
        for _ in range(2):
            seed, offset = generator_state()
            updated, _ = residual_layer_norm(x, ones, w, b, dropout_p=0.25,
                                             implementation="gfx950")
            _, _, threshold = oracle.dropout_constants(0.25)
            expected = oracle.decode_mask(oracle.reference_mask_words(
                rows, hidden, REFERENCE_THREADS[hidden], seed, offset, threshold), rows, hidden)
            assert np.array_equal(host(updated) != 0, expected), hidden
            assert generator_state()[1] == offset + oracle.reference_philox_increment(
                hidden, REFERENCE_THREADS[hidden])


def test_subsequences_past_2_32():
    """Row r draws subsequences r * threads + t: with 256 threads they pass
    2^32 at row 2^24, so the 64-bit subsequence reaches the counter's high
    words (26 GB of tensors, inside the 288 GB of HBM)."""
    hidden, threads = 128, 256
    boundary = 1 << 24
    rows = boundary + 8
    print(f"[reference-stream] rows={rows} H={hidden} T={threads}", flush=True)
    x = torch.zeros(rows, hidden, device="cuda")
    branch = torch.ones(rows, hidden, device="cuda", dtype=torch.float16)
    weight = torch.ones(hidden, device="cuda")
    bias = torch.zeros(hidden, device="cuda")
    seed, offset = 0xA5A5_0000_0001, 4 * 5
    outputs = cabi_forward(x, branch, weight, bias, 0.3, seed, offset, threads,
                           normalized_dtype=torch.float16)
    torch.cuda.synchronize()
    del x, branch
    _, _, threshold = oracle.dropout_constants(0.3)
    words_per_row = hidden // 32
    for first in (0, boundary - 3, rows - 4):
        expected = oracle.reference_mask_rows(first, 4, hidden, threads, seed, offset, threshold)
        got = host(outputs[4][first * words_per_row:(first + 4) * words_per_row])
        assert_bitwise(got.view(np.uint32), expected, f"rows {first}..{first + 3}")
