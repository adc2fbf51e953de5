"""Shared helpers for the GPU parity tests: inputs, oracle replay, tolerances.

Tolerances (written here once, used by every parity test):

* bit-exact: ``updated`` (always), the dropout mask, deterministic replays,
  the misaligned (element access) path against the aligned path;
* ``normalized``, ``mean``, ``rstd``, ``grad_x`` and fp32 ``grad_branch``:
  normwise relative error ``max|a - b| / max|b|`` <= 1e-5 against the fp64
  oracle;
* fp16 / bf16 ``grad_branch`` and a fp16 / bf16 ``normalized``: within one ulp
  of that type at the fp64 oracle value, plus 1e-5 of the largest magnitude
  (the kernel rounds its fp32 result once);
* ``grad_weight`` / ``grad_bias``: normwise relative error <= 1e-4.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import rln_oracle as oracle

# The reference's hidden sizes (specialized kernels), and sizes that cover
# every run-time-length kernel shape (slots per lane x waves per row) of each
# pass and both sides of each boundary where a pass changes its waves per row:
# forward 1x1, 2x1, 3x1, 4x1, 3x2 (up to 1536), 4x2 (to 2048), 3x4, 4x4 (to
# 4096), 3x8, 4x8; backward 1x1, 2x1, 3x1 (to 768), 1x4 (to 1024), 3x2 (to
# 1216), 2x4 (to 2048), 3x4 (to 2432), 2x8 (to 4096), 3x8, 4x8. Several
# leave slots partly idle (832, 1600, 1984, 2496).
SPECIALIZED_HIDDEN_SIZES = (128, 256, 384, 512, 768, 1024)
WIDE_HIDDEN_SIZES = (192, 320, 640, 832, 896, 1216, 1280, 1536, 1600, 1984, 2048, 2432, 2496,
                     3072, 4096, 5120, 8192)
TOL_FORWARD = 1e-5
TOL_INPUT_GRAD = 1e-5
TOL_PARAMETER_GRAD = 1e-4

DEVICE = torch.device("cuda", 0)


def normwise(actual, expected) -> float:
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    scale = max(float(np.max(np.abs(expected))), 1e-30)
    return float(np.max(np.abs(actual - expected)) / scale)


def assert_normwise(actual, expected, tolerance, what=""):
    error = normwise(actual, expected)
    assert error <= tolerance, f"{what}: normwise error {error:.3e} > {tolerance:.1e}"


def half_ulp(values, kind):
    """Spacing of fp16 ("f16") or bfloat16 ("bf16") numbers at |values|."""
    magnitude = np.abs(np.asarray(values, dtype=np.float64))
    if kind == "f16":
        return np.spacing(magnitude.astype(np.float16)).astype(np.float64)
    # bfloat16 keeps 8 significand bits: spacing 2^(e - 7), at least 2^-133.
    exponent = np.floor(np.log2(np.maximum(magnitude, 2.0 ** -126)))
    return np.exp2(exponent - 7)


def assert_rounded_close(actual, expected_f64, kind, what=""):
    """A value rounded once to fp16/bf16 lies within one ulp of the exact one."""
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected_f64, dtype=np.float64)
    bound = half_ulp(expected, kind) + 1e-5 * float(np.max(np.abs(expected)))
    excess = np.abs(actual - expected) - bound
    assert np.all(excess <= 0), f"{what}: {kind} error exceeds one ulp by {excess.max():.3e}"


def assert_fp16_close(actual_f16, expected_f64, what=""):
    assert_rounded_close(actual_f16, expected_f64, "f16", what)


def assert_bitwise(actual, expected, what=""):
    a = np.ascontiguousarray(actual)
    b = np.ascontiguousarray(expected)
    assert a.shape == b.shape and a.dtype == b.dtype, what
    if a.dtype.itemsize == 4:
        a, b = a.view(np.uint32), b.view(np.uint32)
    elif a.dtype.itemsize == 2:
        a, b = a.view(np.uint16), b.view(np.uint16)
    mismatches = int(np.count_nonzero(a != b))
    assert mismatches == 0, f"{what}: {mismatches} of {a.size} values differ bitwise"


KIND = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}


def host(tensor: torch.Tensor) -> np.ndarray:
    """Host copy; bfloat16 (which numpy lacks) comes back as its exact fp32 values."""
    tensor = tensor.detach()
    if tensor.dtype == torch.bfloat16:
        tensor = tensor.float()
    return tensor.cpu().numpy()


def kind(tensor: torch.Tensor) -> str:
    return KIND[tensor.dtype]


def make_inputs(shape, branch_dtype, seed, x_mean=0.0, x_std=1.0, branch_std=1.0,
                device=DEVICE):
    """Seeded CPU inputs copied to the device (CPU and GPU see identical values)."""
    generator = torch.Generator().manual_seed(seed)
    hidden = shape[-1]
    x = torch.randn(shape, generator=generator) * x_std + x_mean
    branch = (torch.randn(shape, generator=generator) * branch_std).to(branch_dtype)
    weight = 1.0 + 0.02 * torch.randn(hidden, generator=generator)
    bias = 0.02 * torch.randn(hidden, generator=generator)
    return tuple(t.contiguous().to(device) for t in (x, branch, weight, bias))


def make_grads(shape, seed, device=DEVICE):
    generator = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(shape, generator=generator).to(device) for _ in range(2))


def generator_state(device=DEVICE):
    """(seed, offset) the next native dropout call will use."""
    generator = torch.cuda.default_generators[device.index or 0]
    return generator.initial_seed(), generator.get_offset()


# The reference's threads per row (reference _normalization_native.py:5-12),
# which the public API passes too. On these hidden sizes a call's `threads`
# selects the reference's hipRAND dropout stream; on the others (and with
# threads = 0 through the C ABI) the library's own layout is drawn.
REFERENCE_THREADS = {128: 128, 256: 128, 384: 128, 512: 128, 768: 128, 1024: 192}
API = "api"  # the `threads` the public API passes for the hidden size


def stream_threads(hidden, threads):
    """The dropout layout of a call: the reference's launch width, or 0."""
    if threads == API:
        threads = REFERENCE_THREADS.get(hidden, 0)
    return threads if hidden in REFERENCE_THREADS else 0


def oracle_mask_rows(first_row, rows, hidden, seed, offset, threshold, threads=128):
    """Oracle mask words of rows [first_row, first_row + rows) for a call with `threads`."""
    layout = stream_threads(hidden, threads)
    if layout:
        return oracle.reference_mask_rows(first_row, rows, hidden, layout, seed, offset, threshold)
    return oracle.dropout_mask_rows(first_row, rows, hidden, seed, offset, threshold)


def philox_increment(hidden, threads=128):
    """Offset units a call with `threads` reserves."""
    layout = stream_threads(hidden, threads)
    return oracle.reference_philox_increment(hidden, layout) if layout else 4


def oracle_keep(rows, hidden, dropout_p, training, seed, offset, threads=128):
    active, scale, threshold = oracle.dropout_constants(dropout_p, training)
    if not active:
        return None, scale, None
    words = oracle_mask_rows(0, rows, hidden, seed, offset, threshold, threads)
    return oracle.decode_mask(words, rows, hidden), scale, words


def check_forward(outputs, inputs, dropout_p, training, eps, seed, offset, what="", threads=128):
    """Compare raw forward outputs (updated, normalized, mean, rstd, mask) to the
    oracle; `threads` is the call's (0 for the C ABI's own layout, API for the
    public API's)."""
    updated, normalized, mean, rstd, mask = outputs
    branch_kind = kind(inputs[1])
    x, branch, weight, bias = (host(t) for t in inputs)
    hidden = x.shape[-1]
    rows = x.size // hidden
    keep, scale, words = oracle_keep(rows, hidden, dropout_p, training, seed, offset, threads)
    if words is not None:
        assert_bitwise(host(mask).view(np.uint32), words, f"{what} mask")
    else:
        assert mask.numel() == 0
    x2 = x.reshape(rows, hidden)
    b2 = branch.reshape(rows, hidden)
    expected = oracle.forward(x2, b2, weight, bias, eps, keep=keep, scale=scale,
                              branch_type=branch_kind)
    assert_bitwise(host(updated).reshape(rows, hidden), expected["updated"], f"{what} updated")
    if normalized.dtype == torch.float32:
        assert_normwise(host(normalized).reshape(rows, hidden), expected["normalized"],
                        TOL_FORWARD, f"{what} normalized")
    else:
        assert_rounded_close(host(normalized).reshape(rows, hidden), expected["normalized"],
                             kind(normalized), f"{what} normalized")
    assert_normwise(host(mean), expected["mean"], TOL_FORWARD, f"{what} mean")
    assert_normwise(host(rstd), expected["rstd"], TOL_FORWARD, f"{what} rstd")
    return keep, scale


def check_backward(gradients, grad_updated, grad_normalized, updated, weight, eps, keep, scale,
                   what="", parameters=True):
    grad_x, grad_branch, grad_weight, grad_bias = gradients
    u = host(updated)
    hidden = u.shape[-1]
    u = u.reshape(-1, hidden)
    gu = None if grad_updated is None else host(grad_updated).reshape(-1, hidden)
    gy = None if grad_normalized is None else host(grad_normalized).reshape(-1, hidden)
    expected = oracle.backward(gu, gy, u, host(weight), eps, keep=keep, scale=scale)
    assert_normwise(host(grad_x).reshape(-1, hidden), expected["grad_x"], TOL_INPUT_GRAD,
                    f"{what} grad_x")
    gb = host(grad_branch).reshape(-1, hidden)
    if grad_branch.dtype == torch.float32:
        assert_normwise(gb, expected["grad_branch"], TOL_INPUT_GRAD, f"{what} grad_branch")
    else:
        assert_rounded_close(gb, expected["grad_branch"], kind(grad_branch),
                             f"{what} grad_branch")
    if parameters:
        assert_normwise(host(grad_weight), expected["grad_weight"], TOL_PARAMETER_GRAD,
                        f"{what} grad_weight")
        assert_normwise(host(grad_bias), expected["grad_bias"], TOL_PARAMETER_GRAD,
                        f"{what} grad_bias")
    return expected
