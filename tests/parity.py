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

Golden fixtures (``conditioned_bounds``): per element, a bound from fp32
error propagation through the two-pass LayerNorm, with u = 2^-24 (fp32 unit
roundoff), n = ceil(log2 H) + 4 (additions along one row reduction), R the
rows, and kappa_r = 1 + |mean_r| * rstd_r the row's conditioning (large for
nearly-constant rows, whose fp32 mean carries an error of order u * |mean|):

* mean_r: 2 n u max_i |u_ri|;  rstd_r: 4 n u kappa_r rstd_r;
* normalized: 4 n u kappa_r max|w| (1 + |xhat_ri|);
* grad_x: 8 n u kappa_r rstd_r max_i|q_ri| (1 + max_i|xhat_ri|) (1 + |xhat_ri|)
  + 2 u |grad_updated_ri|, with q = grad_normalized * w (grad_branch: the same
  times keep * scale, plus one ulp of its type);
* grad_weight_c: sum_r |gy_rc| 2 n u kappa_r (1 + |xhat_rc|)
  + 2 (ceil(log2 R) + 4) u sum_r |gy_rc xhat_rc|; grad_bias_c: 2 (ceil(log2 R)
  + 4) u sum_r |gy_rc|.

A float32 two-pass evaluation meets these with margin on every fixture; a
one-pass variance, or a gradient without its xhat * mean(q * xhat) term,
exceeds them (tests/test_parity_checker.py). For well-conditioned rows they
are as tight as the 1e-5 normwise bar.

Full-size tensors (``check_full_tensor``): the whole dropout mask against the
C oracle (drawn in row chunks on a thread pool), ``updated`` on every row
bitwise against its fp32 recomputation from that mask on the device, and
``normalized``, ``mean``, ``rstd``, ``grad_x``, ``grad_branch`` on every row
against a float64 LayerNorm and its gradient computed with torch on the
device, at the bars above (normwise over the whole tensor).
"""

from __future__ import annotations

import math
import os
from concurrent.futures import ThreadPoolExecutor

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


def oracle_mask_words_parallel(rows, hidden, seed, offset, threshold, threads=128, chunk=8192):
    """The oracle's mask words of a whole [rows, hidden] tensor, drawn in row
    chunks on a thread pool (the C oracle releases the GIL)."""
    workers = min(16, os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=workers) as pool:
        parts = pool.map(
            lambda first: oracle_mask_rows(first, min(chunk, rows - first), hidden, seed,
                                           offset, threshold, threads),
            range(0, rows, chunk))
        return np.concatenate(list(parts))


def device_keep(words, first_row, rows, hidden):
    """Keep flags of rows [first_row, first_row + rows) from int32 mask words on
    the device (bit c % 32 of word r * hidden / 32 + c / 32)."""
    per_row = hidden // 32
    block = words[first_row * per_row:(first_row + rows) * per_row]
    shifts = torch.arange(32, device=words.device, dtype=torch.int32)
    return ((block.view(rows, per_row, 1) >> shifts) & 1).view(rows, hidden).bool()


def _ulp_bound(expected, dtype):
    """One ulp of `dtype` (fp16 / bf16) at |expected|, as a float64 tensor."""
    bits, floor = (10, -14) if dtype == torch.float16 else (7, -126)
    exponent = torch.floor(torch.log2(expected.abs().clamp_min(2.0 ** floor)))
    return torch.exp2(exponent - bits)


class _Normwise:
    """Running max|actual - expected| and max|expected| over row chunks; for a
    half-precision tensor also the running max of |actual - expected| - ulp."""

    def __init__(self):
        self.error = 0.0
        self.scale = 0.0
        self.excess = -float("inf")

    def add(self, actual, expected):
        difference = (actual.to(torch.float64) - expected).abs()
        self.error = max(self.error, difference.max().item())
        self.scale = max(self.scale, expected.abs().max().item())
        if actual.dtype in (torch.float16, torch.bfloat16):
            self.excess = max(self.excess,
                              (difference - _ulp_bound(expected, actual.dtype)).max().item())

    def check(self, tolerance, what, dtype=torch.float32):
        if dtype in (torch.float16, torch.bfloat16):
            bound = 1e-5 * self.scale
            assert self.excess <= bound, (
                f"{what}: {KIND[dtype]} error exceeds one ulp by {self.excess:.3e} "
                f"(allowed {bound:.3e})")
        else:
            error = self.error / max(self.scale, 1e-30)
            assert error <= tolerance, f"{what}: normwise error {error:.3e} > {tolerance:.1e}"


def check_full_tensor(inputs, grads, outputs, gradients, dropout_p, eps, seed, offset,
                      threads=128, chunk=16384, what=""):
    """Every row of a full-size forward + backward against the oracle's mask and a
    float64 recomputation on the device (bars in the module docstring).
    `inputs` = (x, branch, weight, bias) [rows, hidden] on the device; `grads` =
    (grad_updated, grad_normalized); `outputs` = (updated, normalized, mean, rstd,
    mask); `gradients` = (grad_x, grad_branch, ...)."""
    x, branch, weight, bias = inputs
    rows, hidden = x.shape
    active, scale, threshold = oracle.dropout_constants(dropout_p, True)
    words = None
    if active:
        expected_words = oracle_mask_words_parallel(rows, hidden, seed, offset, threshold,
                                                    threads)
        assert_bitwise(host(outputs[4]).view(np.uint32), expected_words, f"{what} mask")
        words = torch.from_numpy(expected_words.view(np.int32)).to(x.device)
    f64 = torch.float64
    weight64, bias64 = weight.to(f64), bias.to(f64)
    checks = {name: _Normwise() for name in ("normalized", "mean", "rstd", "grad_x",
                                             "grad_branch")}
    for start in range(0, rows, chunk):
        stop = min(rows, start + chunk)
        count = stop - start
        branch_rows = branch[start:stop].float()
        keep = None
        if words is not None:
            keep = device_keep(words, start, count, hidden)
            branch_rows = ((branch_rows * keep.float()) * float(scale)).to(branch.dtype).float()
        updated = x[start:stop] + branch_rows
        same = torch.equal(updated.view(torch.int32), outputs[0][start:stop].view(torch.int32))
        assert same, f"{what} updated differs bitwise in rows {start}..{stop - 1}"
        u = updated.to(f64)
        mean = u.mean(dim=1, keepdim=True)
        centred = u - mean
        rstd = 1.0 / torch.sqrt((centred * centred).mean(dim=1, keepdim=True) + eps)
        xhat = centred * rstd
        checks["normalized"].add(outputs[1][start:stop], xhat * weight64 + bias64)
        checks["mean"].add(outputs[2][start:stop], mean[:, 0])
        checks["rstd"].add(outputs[3][start:stop], rstd[:, 0])
        if gradients is None:
            continue
        grad_updated, grad_normalized = grads
        q = grad_normalized[start:stop].to(f64) * weight64
        grad_x = rstd * (q - q.mean(dim=1, keepdim=True)
                         - xhat * (q * xhat).mean(dim=1, keepdim=True))
        if grad_updated is not None:
            grad_x = grad_x + grad_updated[start:stop].to(f64)
        grad_branch = grad_x if keep is None else grad_x * (keep.to(f64) * float(scale))
        checks["grad_x"].add(gradients[0][start:stop], grad_x)
        checks["grad_branch"].add(gradients[1][start:stop], grad_branch)
    checks["normalized"].check(TOL_FORWARD, f"{what} normalized", outputs[1].dtype)
    checks["mean"].check(TOL_FORWARD, f"{what} mean")
    checks["rstd"].check(TOL_FORWARD, f"{what} rstd")
    if gradients is not None:
        checks["grad_x"].check(TOL_INPUT_GRAD, f"{what} grad_x")
        checks["grad_branch"].check(TOL_INPUT_GRAD, f"{what} grad_branch", gradients[1].dtype)


FP32_UNIT_ROUNDOFF = 2.0 ** -24


def conditioned_bounds(updated, weight, eps, grad_updated=None, grad_normalized=None):
    """Per-element fp32 error bounds (module docstring) for a fixture whose
    fp32 `updated` is [R, H]; float64 numpy arrays keyed by output name."""
    u = np.asarray(updated, dtype=np.float64)
    rows, hidden = u.shape
    w = np.asarray(weight, dtype=np.float64)
    unit = FP32_UNIT_ROUNDOFF
    n = math.ceil(math.log2(hidden)) + 4
    n_rows = math.ceil(math.log2(max(rows, 2))) + 4
    mean = u.mean(axis=1)
    centred = u - mean[:, None]
    rstd = 1.0 / np.sqrt((centred * centred).mean(axis=1) + float(eps))
    xhat = centred * rstd[:, None]
    kappa = 1.0 + np.abs(mean) * rstd
    bounds = {
        "mean": 2 * n * unit * np.abs(u).max(axis=1),
        "rstd": 4 * n * unit * kappa * rstd,
        "normalized": 4 * n * unit * kappa[:, None] * np.abs(w).max() * (1 + np.abs(xhat)),
        "kappa": kappa,
    }
    if grad_updated is None and grad_normalized is None:
        return bounds
    gu = np.zeros_like(u) if grad_updated is None else np.asarray(grad_updated, np.float64)
    gy = np.zeros_like(u) if grad_normalized is None else np.asarray(grad_normalized, np.float64)
    q = gy * w
    bounds["grad_x"] = (8 * n * unit * (kappa * rstd * np.abs(q).max(axis=1)
                                        * (1 + np.abs(xhat).max(axis=1)))[:, None]
                        * (1 + np.abs(xhat)) + 2 * unit * np.abs(gu))
    bounds["grad_weight"] = ((np.abs(gy) * 2 * n * unit * kappa[:, None] * (1 + np.abs(xhat)))
                             .sum(axis=0) + 2 * n_rows * unit * np.abs(gy * xhat).sum(axis=0))
    bounds["grad_bias"] = 2 * n_rows * unit * np.abs(gy).sum(axis=0)
    return bounds


def assert_within(actual, expected, bound, what=""):
    """|actual - expected| <= bound elementwise (arrays broadcast)."""
    excess = np.abs(np.asarray(actual, np.float64) - np.asarray(expected, np.float64)) / bound
    worst = float(np.max(excess)) if excess.size else 0.0
    assert worst <= 1.0, f"{what}: error reaches {worst:.3f} of the fp32 conditioned bound"
    return worst
