"""Native glue: loads the gfx950 extension and calls its autograd op.

Mirrors gfx1010_kernels/_normalization_native.py of the reference (lazy ``_C``
import :57-63, ``native_extension_status`` :66-68, ``native_residual_layer_norm``
:71-99). The reference chooses gfx1010-tuned launch hints here (:5-54); the
MI355X library chooses its own launch shape from (rows, hidden). Of the
hints, only ``threads`` still matters: it names the reference launch whose
hipRAND dropout stream the kernels reproduce, so this module passes the
reference's own table (:5-12) and the masks equal the reference package's
for the same generator state. The other hints are fixed, valid values that
the extension range-checks and otherwise ignores.
"""

from __future__ import annotations

from functools import lru_cache

# torch must be imported before _C: _C resolves libtorch and torch's bundled
# HIP runtime (libamdhip64.so.7) from the already-loaded copies.
import torch  # noqa: F401

# Hidden sizes the native path serves: the reference's six (specialized
# kernels, reference normalization.py:12) and every other multiple of 64 up to
# 8192 (kernels with a run-time row length).
SPECIALIZED_HIDDEN_SIZES = (128, 256, 384, 512, 768, 1024)
MIN_NATIVE_HIDDEN_SIZE = 128
MAX_NATIVE_HIDDEN_SIZE = 8192
NATIVE_HIDDEN_MULTIPLE = 64
NATIVE_HIDDEN_SIZES = tuple(
    range(MIN_NATIVE_HIDDEN_SIZE, MAX_NATIVE_HIDDEN_SIZE + 1, NATIVE_HIDDEN_MULTIPLE))
NATIVE_HIDDEN_SIZES_TEXT = (
    f"the multiples of {NATIVE_HIDDEN_MULTIPLE} from {MIN_NATIVE_HIDDEN_SIZE} "
    f"to {MAX_NATIVE_HIDDEN_SIZE}")
TARGET_ARCHITECTURE = "gfx950"

# The reference's threads per row (reference _normalization_native.py:5-12),
# which fix its dropout stream; 128 for the sizes it does not run natively.
_THREADS = {128: 128, 256: 128, 384: 128, 512: 128, 768: 128, 1024: 192}


def launch_threads(hidden_size: int) -> int:
    """The ``threads`` hint the reference passes for ``hidden_size``."""
    return _THREADS.get(hidden_size, 128)


# The remaining launch hints (block_rows, parameter_threads, parameter_groups);
# parameter_groups=1 is valid for every row count.
_LAUNCH_HINTS = (64, 64, 1)


@lru_cache(maxsize=1)
def _extension():
    try:
        from . import _C
    except ImportError as error:
        return None, str(error)
    return _C, ""


def native_extension_status():
    extension, reason = _extension()
    return extension is not None, reason


def native_residual_layer_norm(
    x,
    branch,
    weight,
    bias,
    dropout_p,
    eps,
    training,
    normalized_dtype=None,
):
    extension, reason = _extension()
    if extension is None:
        raise RuntimeError(
            f"{TARGET_ARCHITECTURE} native extension is unavailable: {reason}"
        )
    # normalized_dtype goes positionally: a keyword costs pybind11 ~0.3 us.
    return tuple(
        extension.residual_layer_norm(
            x,
            branch,
            weight,
            bias,
            float(dropout_p),
            float(eps),
            bool(training),
            _THREADS.get(x.shape[-1], 128),
            *_LAUNCH_HINTS,
            normalized_dtype,
        )
    )


def native_residual_layer_norm_if_supported(
    x,
    branch,
    weight,
    bias,
    dropout_p,
    eps,
    training,
    normalized_dtype=None,
):
    """``native_residual_layer_norm`` when the fused kernels serve the inputs
    (checked in C++, the conditions of ``normalization._input_reason`` plus a
    native hidden size), else None. For callers that already know the
    extension is loaded and the device ready; ``x`` has at least two
    dimensions."""
    result = _extension()[0].residual_layer_norm_if_supported(
        x,
        branch,
        weight,
        bias,
        float(dropout_p),
        float(eps),
        bool(training),
        _THREADS.get(x.shape[-1], 128),
        *_LAUNCH_HINTS,
        normalized_dtype,
    )
    return None if result is None else tuple(result)


__all__ = [
    "NATIVE_HIDDEN_SIZES",
    "launch_threads",
    "SPECIALIZED_HIDDEN_SIZES",
    "TARGET_ARCHITECTURE",
    "native_extension_status",
    "native_residual_layer_norm",
    "native_residual_layer_norm_if_supported",
]
