"""Both row schedules of the kernels give the same bits.

The library walks a launch's rows with one row of look-ahead when it is
small and paced (each row's loads issued after the previous row is stored,
slice by slice) when it is large: from 2^23 elements at hidden >= 256 for
one-wave rows (forward and backward), from 2^26 elements for the forward of
multi-wave rows (hidden > 1024) except 8 waves of 4 slots. Every output of a row
except the weight/bias sums depends on that row alone, so the first rows of
a paced launch must equal, bit for bit, a look-ahead launch over just those
rows; every row of the paced launch is also checked against the oracle
(parity.check_full_tensor: the whole mask, `updated` bitwise, the rest
against float64), its sums against a float64 reduction, and the
element-access (misaligned) path against the aligned one. Calls go through
the C ABI with explicit Philox seeds and offsets (the library's own dropout
layout).
"""

import pytest
import torch

from gfx1010_kernels import _cabi
from parity import TOL_PARAMETER_GRAD, assert_bitwise, assert_normwise, check_full_tensor, host

pytestmark = pytest.mark.gpu
EPS = 1e-5
PACED_ELEMENTS = 1 << 23
WIDE_PACED_ELEMENTS = 1 << 26  # forward of multi-wave rows
SEED, OFFSET = 0x5EED_0BAD_F00D, 1 << 20
CODE = {torch.float32: _cabi.RLN_DTYPE_F32, torch.float16: _cabi.RLN_DTYPE_F16,
        torch.bfloat16: _cabi.RLN_DTYPE_BF16}


def empty(shape, dtype, shift=0):
    """An uninitialised contiguous tensor starting `shift` elements into its buffer."""
    count = 1
    for size in shape:
        count *= size
    return torch.empty(count + shift, device="cuda", dtype=dtype)[shift:].view(shape)


def make_case(rows, hidden, branch_dtype):
    """x, branch, weight, bias, grad_updated, grad_normalized (seeded, on the device)."""
    generator = torch.Generator(device="cuda").manual_seed(rows * 31 + hidden)

    def randn(*shape):
        return torch.randn(*shape, device="cuda", generator=generator)

    return (randn(rows, hidden), (0.5 * randn(rows, hidden)).to(branch_dtype),
            1.0 + 0.02 * randn(hidden), 0.02 * randn(hidden), randn(rows, hidden),
            randn(rows, hidden))


def run(case, rows, normalized_dtype, dropout_p, deterministic, shift=0):
    """Forward then backward over the first `rows` rows of `case`."""
    x, branch, weight, bias, grad_updated, grad_normalized = case
    hidden = x.shape[1]
    stream = torch.cuda.current_stream().cuda_stream
    out = dict(
        updated=empty((rows, hidden), torch.float32, shift),
        normalized=empty((rows, hidden), normalized_dtype, shift),
        mean=torch.empty(rows, device="cuda"),
        rstd=torch.empty(rows, device="cuda"),
        mask=torch.zeros(_cabi.mask_words(rows, hidden), device="cuda", dtype=torch.int32),
        grad_x=empty((rows, hidden), torch.float32, shift),
        grad_branch=empty((rows, hidden), branch.dtype, shift),
        parameters=torch.full((2, hidden), float("nan"), device="cuda"),
    )
    _cabi.forward(x.data_ptr(), branch.data_ptr(), CODE[branch.dtype], weight.data_ptr(),
                  bias.data_ptr(), out["updated"].data_ptr(), out["normalized"].data_ptr(),
                  out["mean"].data_ptr(), out["rstd"].data_ptr(), out["mask"].data_ptr(),
                  rows, hidden, dropout_p, EPS, True, _cabi.RlnPhilox(SEED, OFFSET, None, None),
                  stream, normalized_dtype=CODE[normalized_dtype])
    workspace = None
    if deterministic:
        size = _cabi.backward_workspace_bytes(rows, hidden, True)
        workspace = torch.empty(size, device="cuda", dtype=torch.uint8)
    _cabi.backward(grad_updated.data_ptr(), grad_normalized.data_ptr(),
                   out["updated"].data_ptr(), weight.data_ptr(), out["mean"].data_ptr(),
                   out["rstd"].data_ptr(), out["mask"].data_ptr(), out["grad_x"].data_ptr(),
                   out["grad_branch"].data_ptr(), CODE[branch.dtype],
                   out["parameters"][0].data_ptr(), out["parameters"][1].data_ptr(), rows,
                   hidden, dropout_p, True, deterministic,
                   workspace.data_ptr() if workspace is not None else None,
                   workspace.numel() if workspace is not None else 0, stream)
    torch.cuda.synchronize()
    return out


def assert_same_bits(actual, expected, what):
    """Bitwise equality on the device (large tensors stay there)."""
    integer = {4: torch.int32, 2: torch.int16}[actual.element_size()]
    assert actual.shape == expected.shape, what
    assert torch.equal(actual.contiguous().view(integer), expected.contiguous().view(integer)), what


def check_parameter_sums(out, grad_normalized, rows, chunk=16384):
    hidden = out["updated"].shape[1]
    grad_normalized = grad_normalized[:rows]
    d_weight = torch.zeros(hidden, dtype=torch.float64, device="cuda")
    d_bias = torch.zeros(hidden, dtype=torch.float64, device="cuda")
    for start in range(0, rows, chunk):
        u = out["updated"][start:start + chunk].double()
        centered = u - u.mean(dim=-1, keepdim=True)
        xhat = centered / torch.sqrt((centered * centered).mean(dim=-1, keepdim=True) + EPS)
        gy = grad_normalized[start:start + chunk].double()
        d_weight += (gy * xhat).sum(dim=0)
        d_bias += gy.sum(dim=0)
    assert_normwise(host(out["parameters"][0]), host(d_weight), TOL_PARAMETER_GRAD, "grad_weight")
    assert_normwise(host(out["parameters"][1]), host(d_bias), TOL_PARAMETER_GRAD, "grad_bias")


ROW_OUTPUTS = ("updated", "normalized", "mean", "rstd", "grad_x", "grad_branch")


@pytest.mark.parametrize("hidden", [256, 768, 1024, 640, 1280, 2048, 6144])
@pytest.mark.parametrize("branch_dtype,normalized_dtype",
                         [(torch.float16, torch.float32), (torch.bfloat16, torch.bfloat16),
                          (torch.float32, torch.float16)], ids=["f16-f32", "bf16-bf16", "f32-f16"])
def test_paced_rows_equal_look_ahead_rows(hidden, branch_dtype, normalized_dtype):
    threshold = PACED_ELEMENTS if hidden <= 1024 else WIDE_PACED_ELEMENTS
    paced_rows = threshold // hidden + 37
    prefix = (PACED_ELEMENTS // hidden) // 2 - 5
    print(f"[schedules] H={hidden} rows={paced_rows}/{prefix} {branch_dtype} {normalized_dtype}",
          flush=True)
    case = make_case(paced_rows, hidden, branch_dtype)
    paced = run(case, paced_rows, normalized_dtype, 0.1, deterministic=False)
    look_ahead = run(case, prefix, normalized_dtype, 0.1, deterministic=False)
    for name in ROW_OUTPUTS:
        assert_same_bits(paced[name][:prefix], look_ahead[name], name)
    words = look_ahead["mask"].numel()
    assert_same_bits(paced["mask"][:words], look_ahead["mask"], "mask")
    check_parameter_sums(paced, case[5], paced_rows)
    check_parameter_sums(look_ahead, case[5], prefix)
    check_full_tensor(case[:4], case[4:], [paced[name] for name in ("updated", "normalized",
                                                                    "mean", "rstd", "mask")],
                      [paced["grad_x"], paced["grad_branch"]], 0.1, EPS, SEED, OFFSET,
                      threads=0, what=f"paced H={hidden}")


@pytest.mark.parametrize("deterministic", [False, True], ids=["atomic", "deterministic"])
def test_paced_element_access_matches_aligned(deterministic):
    """Misaligned pointers take the element-access kernels; at a paced size
    they give the aligned kernels' bits (and the same fixed-order sums)."""
    rows, hidden = PACED_ELEMENTS // 512 + 3, 512
    print(f"[schedules] misaligned rows={rows} H={hidden} det={deterministic}", flush=True)
    aligned_case = make_case(rows, hidden, torch.bfloat16)
    shifted_case = tuple(empty(t.shape, t.dtype, shift=1) for t in aligned_case)
    for source, target in zip(aligned_case, shifted_case):
        target.copy_(source)
    aligned = run(aligned_case, rows, torch.float32, 0.2, deterministic)
    shifted = run(shifted_case, rows, torch.float32, 0.2, deterministic, shift=1)
    for name in ROW_OUTPUTS + ("mask",):
        assert_bitwise(host(shifted[name]), host(aligned[name]), name)
    if deterministic:
        assert_bitwise(host(shifted["parameters"]), host(aligned["parameters"]), "parameters")
    else:
        check_parameter_sums(shifted, aligned_case[5], rows)


# Row counts around whole multiples of the teams the look-ahead walks use
# (the backward's 2048 one-wave teams at 768 columns, 4096 rows per step at
# 384; the forward's device-dependent grid on 256 CUs: 3072 teams at 768):
# every team then walks 1 to 5 rows, so the register rings of the look-ahead
# walks end on each of their buffers with one or two rows left.
RING_CASES = [(768, rows) for rows in (2047, 2049, 3071, 3073, 4095, 4097, 6143, 6145,
                                        8193, 9215, 9217, 10241)] + \
             [(384, rows) for rows in (4095, 4097, 8193, 12287, 12289, 16385, 20479)]


@pytest.mark.parametrize("hidden,rows", RING_CASES, ids=[f"{h}x{r}" for h, r in RING_CASES])
def test_look_ahead_rows_equal_paced_rows_at_every_ring_position(hidden, rows):
    """Every row output of a look-ahead launch equals, bit for bit, the same row
    of a paced launch over more rows (fp16 branch, p = 0.1), for row counts
    that end the look-ahead walks on every buffer of their rings."""
    paced_rows = PACED_ELEMENTS // hidden + 37
    print(f"[schedules] ring H={hidden} rows={rows} (paced reference {paced_rows})", flush=True)
    case = make_case(paced_rows, hidden, torch.float16)
    paced = run(case, paced_rows, torch.float32, 0.1, deterministic=True)
    look_ahead = run(case, rows, torch.float32, 0.1, deterministic=True)
    for name in ROW_OUTPUTS:
        assert_same_bits(paced[name][:rows], look_ahead[name], name)
    words = look_ahead["mask"].numel()
    assert_same_bits(paced["mask"][:words], look_ahead["mask"], "mask")
    check_parameter_sums(look_ahead, case[5], rows)
