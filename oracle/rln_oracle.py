"""CPU oracle for the fused residual + dropout + LayerNorm - TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
bench.py may import this module, and only as the checker. The product
(gfx1010-kernels_amd/) never imports it.

Restatement of the reference's algorithm, in numpy:

* ``dropout_constants``: scale = 1.0f / (1.0f - float(p)) in fp32 and
  threshold = uint32(double(float(p)) * 2^32)
  (csrc/residual_layer_norm_kernel.hip:893-899, :1883-1886).
* ``dropped_branch`` / ``updated``: d = round_to_branch_dtype(float(b) * keep *
  scale) with fp32 products, then one fp32 add u = x + d
  (csrc/residual_layer_norm_kernel.hip:488-498). Bit-exact by construction.
  The reference has fp16 and fp32 branches; bfloat16 (this build's addition)
  rounds with ``round_to_bfloat16``.
* ``layer_norm_forward``: two-pass mean / centred variance / rsqrt / affine in
  fp64 (csrc/residual_layer_norm_kernel.hip:516-544;
  docs/residual_layer_norm.md:85-109).
* ``backward``: q = g_y * w; g = g_u + rstd * (q - mean(q) - xhat * mean(q *
  xhat)); grad_branch = g * keep * scale; dW = sum g_y * xhat; db = sum g_y, in
  fp64 (csrc/residual_layer_norm_kernel.hip:548-618, :727-786;
  docs/residual_layer_norm.md:111-160).
* dropout mask: Philox4x32-10 stream and the reference's int32 word layout,
  in C (oracle/philox.c): this build's own counter layout
  (``dropout_mask_words``), and the reference's hipRAND layout of a
  ``threads``-wide launch (``reference_mask_words``,
  csrc/residual_layer_norm_kernel.hip:449-511).

How each function is pinned (tests/test_oracle.py):

* Philox4x32-10: Random123 known-answer vectors (tests/golden/philox4x32_10_kat.json).
* hipRAND stream and the reference's mask: vectors from rocRAND's own
  rocrand_init / rocrand4 (tests/golden/hiprand_philox_vectors.json, written by
  tests/golden/make_hiprand_vectors.py).
* mask layout / decode: per-element pure-Python restatement on small shapes,
  and the byte identity with a little-endian uint64 word layout.
* dropout constants: closed forms (p = 0.5, 0.25, 0.75 give exact powers of
  two) and the reference's probability conversion for p = 0.1.
* updated: torch's own fp32 add for p = 0; hand-computed fp16 products.
* round_to_bfloat16 / round_to_float16: torch's CPU conversions on ties,
  subnormals, overflow, infinities and NaN.
* forward / backward / parameter gradients: golden vectors written by
  tests/golden/make_golden.py from PyTorch's float64 ``F.layer_norm`` and
  autograd (the reference's fallback decomposition,
  gfx1010_kernels/normalization.py:15-33), closed-form ``linspace`` rows, and
  the row invariants sum(g_LN) = 0 and sum(g_LN * xhat) = 0.
"""

from __future__ import annotations

import ctypes
import subprocess
from functools import lru_cache
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIBRARY_PATH = ORACLE_DIR / "liboracle_rln.so"


def build() -> Path:
    """Compile oracle/philox.c into liboracle_rln.so (gcc via make)."""
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
    return LIBRARY_PATH


@lru_cache(maxsize=1)
def _library() -> ctypes.CDLL:
    if not LIBRARY_PATH.exists():
        build()
    library = ctypes.CDLL(str(LIBRARY_PATH))
    u32p = ctypes.POINTER(ctypes.c_uint32)
    library.oracle_philox4x32_10.argtypes = [u32p, u32p, u32p]
    library.oracle_philox4x32_10.restype = None
    library.oracle_dropout_uniform.argtypes = [
        ctypes.c_int64, ctypes.c_int64, ctypes.c_uint64, ctypes.c_uint64, u32p]
    library.oracle_dropout_uniform.restype = None
    library.oracle_dropout_mask.argtypes = [
        ctypes.c_int64, ctypes.c_int64, ctypes.c_uint64, ctypes.c_uint64,
        ctypes.c_uint32, u32p]
    library.oracle_dropout_mask.restype = None
    library.oracle_dropout_mask_rows.argtypes = [
        ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_uint64, ctypes.c_uint64,
        ctypes.c_uint32, u32p]
    library.oracle_dropout_mask_rows.restype = None
    library.oracle_hiprand_philox4.argtypes = [
        ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int, u32p]
    library.oracle_hiprand_philox4.restype = None
    library.oracle_reference_mask_rows.argtypes = [
        ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_uint64,
        ctypes.c_uint64, ctypes.c_uint32, u32p]
    library.oracle_reference_mask_rows.restype = ctypes.c_int
    return library


def _u32_pointer(array: np.ndarray):
    assert array.dtype == np.uint32 and array.flags.c_contiguous
    return array.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))


# ---------------------------------------------------------------------------
# Dropout.

def dropout_constants(dropout_p: float, training: bool = True):
    """Return ``(active, scale, threshold)`` as the reference derives them."""
    active = bool(training) and float(dropout_p) > 0.0
    if not active:
        return False, np.float32(1.0), 0
    p32 = np.float32(dropout_p)
    scale = np.float32(1.0) / (np.float32(1.0) - p32)
    threshold = int(float(p32) * 4294967296.0)
    return True, np.float32(scale), threshold


def philox4x32_10(counter, key) -> tuple[int, int, int, int]:
    """One Philox4x32-10 block for a 4-word counter and 2-word key."""
    c = np.asarray(counter, dtype=np.uint32).copy()
    k = np.asarray(key, dtype=np.uint32).copy()
    out = np.zeros(4, dtype=np.uint32)
    _library().oracle_philox4x32_10(_u32_pointer(c), _u32_pointer(k), _u32_pointer(out))
    return tuple(int(value) for value in out)


def dropout_uniform(rows: int, hidden: int, seed: int, offset: int) -> np.ndarray:
    """Raw u32 draw for every element, shape [rows, hidden]."""
    draws = np.zeros(rows * hidden, dtype=np.uint32)
    _library().oracle_dropout_uniform(rows, hidden, seed, offset, _u32_pointer(draws))
    return draws.reshape(rows, hidden)


def dropout_mask_words(rows: int, hidden: int, seed: int, offset: int, threshold: int) -> np.ndarray:
    """Packed keep mask, ``rows * hidden / 32`` uint32 words."""
    words = np.zeros(rows * hidden // 32, dtype=np.uint32)
    _library().oracle_dropout_mask(rows, hidden, seed, offset, threshold, _u32_pointer(words))
    return words


def dropout_mask_rows(first_row: int, rows: int, hidden: int, seed: int, offset: int,
                      threshold: int) -> np.ndarray:
    """Packed keep mask of rows [first_row, first_row + rows) only."""
    words = np.zeros(rows * hidden // 32, dtype=np.uint32)
    _library().oracle_dropout_mask_rows(first_row, rows, hidden, seed, offset, threshold,
                                        _u32_pointer(words))
    return words


# The reference's own stream: hipRAND (rocRAND) Philox, one state per
# (row, thread) of a `threads`-wide launch (oracle/philox.c).
REFERENCE_THREADS = (128, 192, 256)


def hiprand_philox4(seed: int, subsequence: int, offset: int, calls: int) -> list[int]:
    """``calls`` rocrand4 results after rocrand_init(seed, subsequence, offset), flattened."""
    out = np.zeros(4 * calls, dtype=np.uint32)
    _library().oracle_hiprand_philox4(seed, subsequence, offset, calls, _u32_pointer(out))
    return [int(value) for value in out]


def reference_philox_increment(hidden: int, threads: int) -> int:
    """Offset units the reference reserves per call: 4 * ceil(ceil(H / T) / 4)
    (csrc/residual_layer_norm_kernel.hip:1766-1770)."""
    items = -(-hidden // threads)
    return 4 * (-(-items // 4))


def reference_mask_rows(first_row: int, rows: int, hidden: int, threads: int, seed: int,
                        offset: int, threshold: int) -> np.ndarray:
    """The reference's keep mask for rows [first_row, first_row + rows), as
    drawn by its ``threads``-wide forward launch."""
    words = np.zeros(rows * hidden // 32, dtype=np.uint32)
    status = _library().oracle_reference_mask_rows(first_row, rows, hidden, threads, seed,
                                                   offset, threshold, _u32_pointer(words))
    if status != 0:
        raise ValueError(f"the reference draws at most 8 values per thread "
                         f"(hidden={hidden}, threads={threads})")
    return words


def reference_mask_words(rows: int, hidden: int, threads: int, seed: int, offset: int,
                         threshold: int) -> np.ndarray:
    """The reference's keep mask for a whole [rows, hidden] tensor."""
    return reference_mask_rows(0, rows, hidden, threads, seed, offset, threshold)


def decode_mask(words: np.ndarray, rows: int, hidden: int) -> np.ndarray:
    """Keep flags [rows, hidden] from packed words (bit c%32 of word c/32)."""
    raw = np.ascontiguousarray(words).view(np.uint32).astype("<u4")
    bits = np.unpackbits(raw.view(np.uint8), bitorder="little")
    return bits[: rows * hidden].reshape(rows, hidden).astype(bool)


def encode_mask(keep: np.ndarray) -> np.ndarray:
    """Inverse of ``decode_mask``."""
    packed = np.packbits(np.ascontiguousarray(keep, dtype=bool).ravel(), bitorder="little")
    return packed.view("<u4").astype(np.uint32)


def round_to_bfloat16(values) -> np.ndarray:
    """fp32 -> bfloat16 -> fp32, rounding to nearest even (NaN stays NaN).

    bfloat16 is the upper half of an fp32 word: add 0x7FFF plus the lowest
    kept bit, then clear the low 16 bits (the IEEE round-to-nearest-even rule
    on the dropped half; overflow carries into the exponent and gives inf)."""
    values = np.asarray(values, dtype=np.float32)
    bits = values.view(np.uint32).astype(np.uint64)
    rounded = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16) << 16
    out = (rounded & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(values), np.float32(np.nan), out).astype(np.float32)


def round_to_float16(values) -> np.ndarray:
    """fp32 -> float16 -> fp32 (numpy's conversion rounds to nearest even;
    values beyond the float16 range become infinities)."""
    with np.errstate(over="ignore"):
        return np.asarray(values, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_to(values, dtype: str) -> np.ndarray:
    """Round fp32 values through "f32" (identity), "f16" or "bf16"."""
    if dtype == "f16":
        return round_to_float16(values)
    if dtype == "bf16":
        return round_to_bfloat16(values)
    return np.asarray(values, dtype=np.float32)


def _branch_type(branch: np.ndarray, branch_type: str | None) -> str:
    if branch_type is not None:
        return branch_type
    return "f16" if branch.dtype == np.float16 else "f32"


def dropped_branch(branch: np.ndarray, keep: np.ndarray | None, scale,
                   branch_type: str | None = None) -> np.ndarray:
    """round_to_branch_dtype(float(b) * keep * scale), as fp32.

    ``branch_type`` ("f32", "f16", "bf16") defaults to the numpy dtype; a
    bfloat16 branch is passed as its exact fp32 values with "bf16"."""
    b32 = branch.astype(np.float32)
    if keep is None:
        return b32
    product = (b32 * keep.astype(np.float32)) * np.float32(scale)
    return round_to(product, _branch_type(branch, branch_type))


def updated(x: np.ndarray, branch: np.ndarray, keep=None, scale=1.0,
            branch_type: str | None = None) -> np.ndarray:
    """The residual update x + dropped branch, one fp32 add (bit-exact)."""
    assert x.dtype == np.float32
    return x + dropped_branch(branch, keep, scale, branch_type)


# ---------------------------------------------------------------------------
# LayerNorm forward / backward in fp64.

def layer_norm_forward(updated_values: np.ndarray, weight, bias, eps: float):
    """Return ``(mean, rstd, normalized)`` in fp64 over the last dimension."""
    u = np.asarray(updated_values, dtype=np.float64)
    mean = u.mean(axis=-1)
    centered = u - mean[..., None]
    variance = np.mean(centered * centered, axis=-1)
    rstd = 1.0 / np.sqrt(variance + float(eps))
    normalized = centered * rstd[..., None] * np.asarray(weight, np.float64) + np.asarray(
        bias, np.float64
    )
    return mean, rstd, normalized


def forward(x, branch, weight, bias, eps, keep=None, scale=1.0, branch_type=None) -> dict:
    """Forward outputs: ``updated`` (fp32, bit-exact) and fp64 statistics."""
    upd = updated(x, branch, keep, scale, branch_type)
    mean, rstd, normalized = layer_norm_forward(upd, weight, bias, eps)
    return {"updated": upd, "normalized": normalized, "mean": mean, "rstd": rstd}


def backward(grad_updated, grad_normalized, updated_values, weight, eps, keep=None, scale=1.0) -> dict:
    """fp64 first-order gradients; either upstream gradient may be None (zero)."""
    u = np.asarray(updated_values, dtype=np.float64)
    hidden = u.shape[-1]
    mean = u.mean(axis=-1, keepdims=True)
    centered = u - mean
    rstd = 1.0 / np.sqrt(np.mean(centered * centered, axis=-1, keepdims=True) + float(eps))
    xhat = centered * rstd
    gy = np.zeros_like(u) if grad_normalized is None else np.asarray(grad_normalized, np.float64)
    gu = np.zeros_like(u) if grad_updated is None else np.asarray(grad_updated, np.float64)
    q = gy * np.asarray(weight, np.float64)
    mean_q = q.mean(axis=-1, keepdims=True)
    mean_qx = (q * xhat).mean(axis=-1, keepdims=True)
    grad_ln = rstd * (q - mean_q - xhat * mean_qx)
    grad_x = gu + grad_ln
    grad_branch = grad_x if keep is None else grad_x * keep.astype(np.float64) * float(scale)
    flat_gy = gy.reshape(-1, hidden)
    flat_xhat = xhat.reshape(-1, hidden)
    return {
        "grad_x": grad_x,
        "grad_branch": grad_branch,
        "grad_weight": (flat_gy * flat_xhat).sum(axis=0),
        "grad_bias": flat_gy.sum(axis=0),
        "grad_ln": grad_ln,
        "xhat": xhat,
    }
