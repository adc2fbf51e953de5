"""Infinities and NaNs: where the kernels send them, and where they must not go.

Mixed-precision training depends on both halves. An fp16 branch that
overflowed, or an upstream gradient that did, has to show up in the outputs
(torch's GradScaler skips a step whose gradients are not finite). It also must
not reach any other row. The reference's arithmetic fixes where each value
goes:

* d = round_to_branch_dtype(float(b) * keep * scale), so a dropped inf or NaN
  is NaN (inf * 0), and the largest finite fp16 branch value times 1/(1-p)
  rounds to inf (csrc/residual_layer_norm_kernel.hip:488-498);
* u = x + d, then a two-pass mean and centred variance (:516-528), so one
  non-finite u makes the row's mean non-finite and its rstd and every
  `normalized` value NaN;
* g = g_u + rstd * (q - mean(q) - xhat * mean(q * xhat)), q = g_y * w
  (:598-603), so a non-finite g_y reaches every column of its row, while a
  non-finite g_u stays in its own element;
* dW = sum g_y * xhat and db = sum g_y (:727-869): an inf g_y at column c
  makes db[c] = +inf and dW[c] = sign(xhat) * inf, and no other column.

Each case runs the same call on clean and on poisoned data, with the same
Philox seed and offset, through the C ABI. The poisoned rows (or elements) are
checked against the oracle, which applies those formulas with IEEE arithmetic
on the host (NaN payloads aside). Every other row must equal the clean call
bit for bit. In deterministic mode so must every other column of the
weight/bias sums. The cases cover each forward and backward row shape: 2 and
4 rows per wave, half and whole waves, 2-16 waves per row, the reference's
dropout stream and the library's own, the paced schedule of large launches
and the 12- and 16-wave backward blocks of large launches.
"""

import numpy as np
import pytest
import torch

from gfx1010_kernels import _cabi
from oracle import rln_oracle as oracle
from parity import TOL_PARAMETER_GRAD, assert_normwise, host

pytestmark = pytest.mark.gpu
EPS = 1e-5
SEED, OFFSET = 0x1BADB002, 1 << 12
CODE = {torch.float32: _cabi.RLN_DTYPE_F32, torch.float16: _cabi.RLN_DTYPE_F16,
        torch.bfloat16: _cabi.RLN_DTYPE_BF16}
KIND = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}

# hidden, rows, branch dtype, dropout_p, normalized dtype, Philox layout
# (128 / 192: the reference's stream of that launch width; 0: the library's).
CASES = [
    (128, 1001, torch.float16, 0.1, torch.float32, 128),
    (256, 515, torch.bfloat16, 0.1, torch.float32, 0),
    (384, 999, torch.float32, 0.0, torch.float32, 0),
    (512, 700, torch.float16, 0.15, torch.float16, 128),
    (768, 1027, torch.float16, 0.1, torch.float32, 128),
    (768, 11000, torch.float16, 0.1, torch.float32, 0),      # paced rows, 2^23+ elements
    (768, 65600, torch.float16, 0.1, torch.float32, 0),      # 12-wave backward blocks
    (1024, 700, torch.float16, 0.1, torch.bfloat16, 192),
    (1600, 301, torch.float16, 0.1, torch.float32, 0),
    (2048, 257, torch.bfloat16, 0.1, torch.float32, 0),
    (4096, 130, torch.float32, 0.1, torch.float32, 0),
    (8192, 67, torch.float16, 0.1, torch.float32, 0),
    (8192, 8200, torch.bfloat16, 0.1, torch.float32, 0),     # 16-wave backward blocks
]


def case_id(case):
    hidden, rows, branch_dtype, p, normalized_dtype, threads = case
    return (f"{rows}x{hidden}-{KIND[branch_dtype]}-p{p}-out{KIND[normalized_dtype]}"
            f"-t{threads}")


def make_case(rows, hidden, branch_dtype):
    generator = torch.Generator(device="cuda").manual_seed(rows * 7 + hidden)

    def randn(*shape):
        return torch.randn(*shape, device="cuda", generator=generator)

    return dict(x=randn(rows, hidden), branch=(0.5 * randn(rows, hidden)).to(branch_dtype),
                weight=1.0 + 0.02 * randn(hidden), bias=0.02 * randn(hidden),
                grad_updated=randn(rows, hidden), grad_normalized=randn(rows, hidden))


def run_forward(data, dropout_p, normalized_dtype, threads):
    rows, hidden = data["x"].shape
    out = dict(
        updated=torch.empty(rows, hidden, device="cuda"),
        normalized=torch.empty(rows, hidden, device="cuda", dtype=normalized_dtype),
        mean=torch.empty(rows, device="cuda"),
        rstd=torch.empty(rows, device="cuda"),
        mask=torch.zeros(_cabi.mask_words(rows, hidden), device="cuda", dtype=torch.int32),
    )
    stream = torch.cuda.current_stream().cuda_stream
    _cabi.forward(data["x"].data_ptr(), data["branch"].data_ptr(), CODE[data["branch"].dtype],
                  data["weight"].data_ptr(), data["bias"].data_ptr(), out["updated"].data_ptr(),
                  out["normalized"].data_ptr(), out["mean"].data_ptr(), out["rstd"].data_ptr(),
                  out["mask"].data_ptr(), rows, hidden, dropout_p, EPS, True,
                  _cabi.RlnPhilox(SEED, OFFSET, None, None, threads), stream,
                  normalized_dtype=CODE[normalized_dtype])
    torch.cuda.synchronize()
    return out


def run_backward(data, state, dropout_p, deterministic):
    rows, hidden = data["x"].shape
    branch_dtype = data["branch"].dtype
    out = dict(grad_x=torch.empty(rows, hidden, device="cuda"),
               grad_branch=torch.empty(rows, hidden, device="cuda", dtype=branch_dtype),
               grad_weight=torch.full((hidden,), float("nan"), device="cuda"),
               grad_bias=torch.full((hidden,), float("nan"), device="cuda"))
    size = _cabi.backward_workspace_bytes(rows, hidden, deterministic)
    workspace = torch.empty(max(size, 1), device="cuda", dtype=torch.uint8)
    stream = torch.cuda.current_stream().cuda_stream
    _cabi.backward(data["grad_updated"].data_ptr(), data["grad_normalized"].data_ptr(),
                   state["updated"].data_ptr(), data["weight"].data_ptr(),
                   state["mean"].data_ptr(), state["rstd"].data_ptr(), state["mask"].data_ptr(),
                   out["grad_x"].data_ptr(), out["grad_branch"].data_ptr(), CODE[branch_dtype],
                   out["grad_weight"].data_ptr(), out["grad_bias"].data_ptr(), rows, hidden,
                   dropout_p, True, deterministic, workspace.data_ptr(), size, stream)
    torch.cuda.synchronize()
    return out


def bits(tensor):
    return tensor.contiguous().view({4: torch.int32, 2: torch.int16}[tensor.element_size()])


def assert_other_rows_equal(actual, expected, poisoned, what):
    """Rows outside `poisoned` are bitwise equal (compared on the device)."""
    others = torch.ones(actual.shape[0], dtype=torch.bool, device="cuda")
    others[list(poisoned)] = False
    assert torch.equal(bits(actual)[others], bits(expected)[others]), \
        f"{what}: a row without a non-finite input changed"


def keep_row(state, row, hidden):
    words = host(state["mask"])[row * hidden // 32:(row + 1) * hidden // 32].astype(np.uint32)
    return oracle.decode_mask(words, 1, hidden)[0]


def same_class(actual, expected):
    """Equal where both are finite or both +inf / -inf; NaN matches NaN."""
    return np.array_equal(np.asarray(actual, np.float64), np.asarray(expected, np.float64),
                          equal_nan=True)


def forward_poison(data, clean, dropout_p, poisoned_rows):
    """Poisoned copies of x / branch: one kind of non-finite input per row."""
    rows, hidden = data["x"].shape
    x = data["x"].clone()
    branch = data["branch"].clone()
    largest = torch.finfo(branch.dtype).max
    first, second, third, fourth, fifth, sixth = poisoned_rows
    x[first, hidden - 1] = float("inf")
    x[second, 0] = float("nan")
    branch[third, hidden // 3] = float("nan")
    branch[fourth, hidden // 2 + 1] = float("-inf")
    if dropout_p > 0.0:
        keep5 = keep_row(clean, fifth, hidden)
        keep6 = keep_row(clean, sixth, hidden)
        branch[fifth, int(np.flatnonzero(~keep5)[0])] = float("inf")   # dropped: inf * 0
        # Kept: the largest finite value times 1/(1 - p) overflows the branch type.
        branch[sixth, int(np.flatnonzero(keep6)[-1])] = largest
    else:
        branch[fifth, 5] = float("inf")
        x[sixth, 1] = float("-inf")
    return dict(data, x=x, branch=branch)


def poison_rows(rows):
    return (0, 1, 2, 3, rows // 2, rows - 1)


@pytest.mark.parametrize("case", CASES, ids=case_id)
def test_forward_keeps_non_finite_inputs_in_their_row(case):
    hidden, rows, branch_dtype, dropout_p, normalized_dtype, threads = case
    data = make_case(rows, hidden, branch_dtype)
    clean = run_forward(data, dropout_p, normalized_dtype, threads)
    poisoned_rows = poison_rows(rows)
    poisoned_data = forward_poison(data, clean, dropout_p, poisoned_rows)
    poisoned = run_forward(poisoned_data, dropout_p, normalized_dtype, threads)

    assert torch.equal(poisoned["mask"], clean["mask"]), "the mask depends on the data"
    for name in ("updated", "normalized", "mean", "rstd"):
        assert_other_rows_equal(poisoned[name], clean[name], poisoned_rows, name)

    scale = oracle.dropout_constants(dropout_p)[1]
    weight, bias = host(data["weight"]), host(data["bias"])
    with np.errstate(all="ignore"):
        for row in poisoned_rows:
            x = host(poisoned_data["x"][row])
            branch = host(poisoned_data["branch"][row])
            keep = keep_row(clean, row, hidden) if dropout_p > 0.0 else None
            expected = oracle.forward(x, branch, weight, bias, EPS, keep, scale,
                                      KIND[branch_dtype])
            assert not np.isfinite(expected["updated"]).all(), f"row {row}: no poison"
            assert same_class(host(poisoned["updated"][row]), expected["updated"]), \
                f"row {row}: updated differs from x + round(b * keep * scale)"
            # The reference's two-pass statistics turn the whole row into NaN.
            assert np.isnan(expected["normalized"]).all()
            assert np.isnan(host(poisoned["normalized"][row])).all(), \
                f"row {row}: normalized has a value that is not NaN"
            assert same_class(host(poisoned["mean"][row]), expected["mean"]), f"row {row}: mean"
            assert np.isnan(host(poisoned["rstd"][row])), f"row {row}: rstd"


@pytest.mark.parametrize("deterministic", [True, False], ids=["deterministic", "atomic"])
@pytest.mark.parametrize("case", CASES, ids=case_id)
def test_backward_sends_non_finite_gradients_where_the_formula_does(case, deterministic):
    hidden, rows, branch_dtype, dropout_p, normalized_dtype, threads = case
    data = make_case(rows, hidden, branch_dtype)
    state = run_forward(data, dropout_p, normalized_dtype, threads)
    clean = run_backward(data, state, dropout_p, deterministic)

    inf_row, nan_gu_row, nan_gy_row = 4, rows // 2 + 1, rows - 2
    inf_column, nan_gu_column, nan_gy_column = 7, hidden - 1, hidden // 2 + 1
    grad_updated = data["grad_updated"].clone()
    grad_normalized = data["grad_normalized"].clone()
    grad_normalized[inf_row, inf_column] = float("inf")
    grad_updated[nan_gu_row, nan_gu_column] = float("nan")
    grad_normalized[nan_gy_row, nan_gy_column] = float("nan")
    poisoned_data = dict(data, grad_updated=grad_updated, grad_normalized=grad_normalized)
    poisoned = run_backward(poisoned_data, state, dropout_p, deterministic)

    for name in ("grad_x", "grad_branch"):
        assert_other_rows_equal(poisoned[name], clean[name],
                                (inf_row, nan_gu_row, nan_gy_row), name)

    # A NaN in grad_updated stays in its element (it enters no row sum).
    for name in ("grad_x", "grad_branch"):
        row = host(poisoned[name][nan_gu_row])
        reference = host(clean[name][nan_gu_row])
        assert np.flatnonzero(np.isnan(row)).tolist() == [nan_gu_column], name
        others = np.arange(hidden) != nan_gu_column
        assert np.array_equal(row[others], reference[others]), name

    # A non-finite grad_normalized reaches every column of its row, as the
    # oracle's formula does.
    scale = oracle.dropout_constants(dropout_p)[1]
    weight = host(data["weight"])
    with np.errstate(all="ignore"):
        for row in (inf_row, nan_gy_row):
            keep = keep_row(state, row, hidden) if dropout_p > 0.0 else None
            expected = oracle.backward(host(grad_updated[row]), host(grad_normalized[row]),
                                       host(state["updated"][row]), weight, EPS, keep, scale)
            assert not np.isfinite(expected["grad_x"]).any()
            assert not np.isfinite(expected["grad_branch"]).any()
            assert not np.isfinite(host(poisoned["grad_x"][row])).any(), f"row {row}: grad_x"
            assert not np.isfinite(host(poisoned["grad_branch"][row])).any(), \
                f"row {row}: grad_branch"

    # The sums: +inf / sign(xhat) * inf at the inf column, NaN at the NaN
    # column, the clean sums everywhere else.
    u = host(state["updated"][inf_row]).astype(np.float64)
    xhat = (u[inf_column] - float(host(state["mean"][inf_row]))) \
        * float(host(state["rstd"][inf_row]))
    expected_weight = host(clean["grad_weight"]).copy()
    expected_bias = host(clean["grad_bias"]).copy()
    expected_weight[inf_column] = np.copysign(np.inf, xhat)
    expected_bias[inf_column] = np.inf
    expected_weight[nan_gy_column] = np.nan
    expected_bias[nan_gy_column] = np.nan
    actual_weight, actual_bias = host(poisoned["grad_weight"]), host(poisoned["grad_bias"])
    poisoned_columns = [inf_column, nan_gy_column]
    assert same_class(actual_weight[poisoned_columns], expected_weight[poisoned_columns])
    assert same_class(actual_bias[poisoned_columns], expected_bias[poisoned_columns])
    others = np.ones(hidden, dtype=bool)
    others[poisoned_columns] = False
    if deterministic:
        assert np.array_equal(actual_weight[others], expected_weight[others])
        assert np.array_equal(actual_bias[others], expected_bias[others])
    else:
        assert np.isfinite(actual_weight[others]).all() and np.isfinite(actual_bias[others]).all()
        assert_normwise(actual_weight[others], expected_weight[others], TOL_PARAMETER_GRAD,
                        "grad_weight")
        assert_normwise(actual_bias[others], expected_bias[others], TOL_PARAMETER_GRAD,
                        "grad_bias")


@pytest.mark.parametrize("case", CASES, ids=case_id)
def test_backward_of_a_non_finite_forward(case):
    """The backward of rows whose forward saw an inf or a NaN (their rstd is
    NaN): those rows' input gradients are NaN, grad_weight is NaN in every
    column, grad_bias (sum g_y, independent of the forward) is unchanged, and
    every other row is unchanged (deterministic mode)."""
    hidden, rows, branch_dtype, dropout_p, normalized_dtype, threads = case
    data = make_case(rows, hidden, branch_dtype)
    clean_state = run_forward(data, dropout_p, normalized_dtype, threads)
    poisoned_rows = poison_rows(rows)
    poisoned_state = run_forward(forward_poison(data, clean_state, dropout_p, poisoned_rows),
                                 dropout_p, normalized_dtype, threads)
    clean = run_backward(data, clean_state, dropout_p, True)
    poisoned = run_backward(data, poisoned_state, dropout_p, True)

    for name in ("grad_x", "grad_branch"):
        assert_other_rows_equal(poisoned[name], clean[name], poisoned_rows, name)
        for row in poisoned_rows:
            assert np.isnan(host(poisoned[name][row])).all(), f"{name} row {row}"
    assert np.isnan(host(poisoned["grad_weight"])).all()
    assert torch.equal(bits(poisoned["grad_bias"]), bits(clean["grad_bias"]))


def test_grad_scaler_skips_an_overflowed_step_and_takes_a_clean_one():
    """torch.amp.GradScaler through the public API. An fp16 branch that
    overflowed makes `normalized` NaN in its rows, so the weight/bias
    gradients of the op and the gradient it hands the branch's producer are
    not finite: the scaler skips the optimizer step and halves its scale. The
    same step on a finite branch updates every parameter."""
    from gfx1010_kernels import residual_layer_norm

    torch.manual_seed(3)
    hidden = 768
    x = torch.randn(4, 64, hidden, device="cuda")
    linear = torch.nn.Linear(hidden, hidden).cuda()
    weight = torch.nn.Parameter(1.0 + 0.02 * torch.randn(hidden, device="cuda"))
    bias = torch.nn.Parameter(0.02 * torch.randn(hidden, device="cuda"))
    parameters = [linear.weight, linear.bias, weight, bias]
    optimizer = torch.optim.SGD(parameters, lr=0.1)
    scaler = torch.amp.GradScaler("cuda", init_scale=2.0 ** 10)

    def step():
        optimizer.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.float16):
            branch = linear(x)
        assert branch.dtype == torch.float16
        updated, normalized = residual_layer_norm(x, branch, weight, bias, dropout_p=0.1,
                                                  implementation="gfx950")
        loss = normalized.square().mean() + 0.1 * updated.mean()
        scaler.scale(loss).backward()
        finite = [bool(torch.isfinite(p.grad).all()) for p in parameters]
        before = [p.detach().clone() for p in parameters]
        scaler.step(optimizer)
        scaler.update()
        return branch, finite, before

    saved = linear.weight.detach().clone()
    with torch.no_grad():
        linear.weight.mul_(1e5)  # outputs of order 6e4 and above: fp16 overflows
    branch, finite, before = step()
    assert not torch.isfinite(branch).all()
    assert finite == [False] * 4, "an overflowed branch left a gradient finite"
    for parameter, old in zip(parameters, before):
        assert torch.equal(parameter.detach(), old), "the scaler took an overflowed step"
    assert scaler.get_scale() == 2.0 ** 9

    with torch.no_grad():
        linear.weight.copy_(saved)
    branch, finite, before = step()
    assert torch.isfinite(branch).all() and finite == [True] * 4
    for parameter, old in zip(parameters, before):
        assert not torch.equal(parameter.detach(), old), "a clean step left a parameter unchanged"
    assert scaler.get_scale() == 2.0 ** 9
