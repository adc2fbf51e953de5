"""ctypes binding of the C ABI in include/rln.h (librln_gfx950.so).

Lets Python call the library directly with device pointers (for example
``tensor.data_ptr()`` of torch tensors) without the torch glue module. Every
function declared in include/rln.h is bound here with its exact signature;
``RlnError`` carries the library's message when a call fails.

Import torch before loading this library inside a torch process: the library
then binds to torch's already-loaded HIP runtime (same SONAME) instead of a
second copy.
"""

from __future__ import annotations

import ctypes
from functools import lru_cache
from pathlib import Path

LIBRARY_PATH = Path(__file__).resolve().parent / "librln_gfx950.so"

RLN_DTYPE_F32 = 0
RLN_DTYPE_F16 = 1
RLN_DTYPE_BF16 = 2

RLN_OK = 0
RLN_ERR_INVALID = 1
RLN_ERR_UNSUPPORTED = 2
RLN_ERR_HIP = 3


class RlnPhilox(ctypes.Structure):
    """``rln_philox_t``; ``threads`` 0 selects the library's dropout layout,
    128 / 192 / 256 the reference's hipRAND stream of that launch width."""

    _fields_ = [
        ("seed", ctypes.c_uint64),
        ("offset", ctypes.c_uint64),
        ("seed_ptr", ctypes.c_void_p),
        ("offset_ptr", ctypes.c_void_p),
        ("threads", ctypes.c_int64),
    ]


class RlnError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


_P = ctypes.c_void_p
_I64 = ctypes.c_int64

# name -> (restype, argtypes), in declaration order of include/rln.h.
SIGNATURES = {
    "rln_forward": (
        ctypes.c_int,
        [_P, _P, ctypes.c_int, _P, _P, _P, _P, ctypes.c_int, _P, _P, _P, _P, _P, _I64, _I64,
         ctypes.c_double, ctypes.c_double, ctypes.c_int, ctypes.POINTER(RlnPhilox), _P],
    ),
    "rln_backward": (
        ctypes.c_int,
        [_P, _P, ctypes.c_int, _P, _P, _P, _P, _P, _P, _P, ctypes.c_int, _P, _P, _I64, _I64,
         ctypes.c_double, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P, ctypes.c_size_t, _P],
    ),
    "rln_backward_noalloc": (
        ctypes.c_int,
        [_P, _P, ctypes.c_int, _P, _P, _P, _P, _P, _P, _P, ctypes.c_int, _P, _P, _I64, _I64,
         ctypes.c_double, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P],
    ),
    "rln_backward_workspace_bytes": (ctypes.c_size_t, [_I64, _I64, ctypes.c_int]),
    "rln_philox_increment": (ctypes.c_uint64, [_I64, _I64]),
    "rln_mask_words": (_I64, [_I64, _I64]),
    "rln_hidden_supported": (ctypes.c_int, [_I64]),
    "rln_supported_hidden_sizes": (ctypes.c_int, [ctypes.POINTER(_I64), ctypes.c_int]),
    "rln_last_error": (ctypes.c_char_p, []),
    "rln_target_arch": (ctypes.c_char_p, []),
    "rln_version": (ctypes.c_char_p, []),
}


def load(path: Path) -> ctypes.CDLL:
    """Load a build of the C ABI at `path` and declare every signature (the
    benchmark's A/B runs load variant builds of the library this way)."""
    if not Path(path).exists():
        raise OSError(f"{path} is missing; build it with gfx1010-kernels_amd/build.py")
    handle = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        function = getattr(handle, name)
        function.restype = restype
        function.argtypes = argtypes
    return handle


@lru_cache(maxsize=1)
def library() -> ctypes.CDLL:
    """Load librln_gfx950.so and declare every C ABI signature."""
    return load(LIBRARY_PATH)


def last_error() -> str:
    return library().rln_last_error().decode()


def _check(status: int) -> None:
    if status != RLN_OK:
        raise RlnError(status, last_error())


def supported_hidden_sizes() -> tuple[int, ...]:
    lib = library()
    count = lib.rln_supported_hidden_sizes(None, 0)
    values = (_I64 * count)()
    lib.rln_supported_hidden_sizes(values, count)
    return tuple(int(value) for value in values)


def forward(
    x, branch, branch_dtype, weight, bias, updated, normalized, mean, rstd, mask,
    rows, hidden, dropout_p, eps, training, philox=None, stream=None,
    normalized_dtype=RLN_DTYPE_F32, zero_grad_weight=None, zero_grad_bias=None,
):
    """Call ``rln_forward`` with integer device addresses; raises RlnError."""
    pointer = ctypes.byref(philox) if philox is not None else None
    _check(
        library().rln_forward(
            x, branch, branch_dtype, weight, bias, updated, normalized, normalized_dtype,
            mean, rstd, mask, zero_grad_weight, zero_grad_bias, rows, hidden, dropout_p, eps,
            int(bool(training)), pointer, stream,
        )
    )


def backward(
    grad_updated, grad_normalized, updated, weight, mean, rstd, mask, grad_x,
    grad_branch, branch_dtype, grad_weight, grad_bias, rows, hidden, dropout_p,
    training, deterministic, workspace=None, workspace_bytes=0, stream=None,
    accumulate_parameters=False, grad_normalized_dtype=RLN_DTYPE_F32,
):
    """Call ``rln_backward`` with integer device addresses; raises RlnError."""
    _check(
        library().rln_backward(
            grad_updated, grad_normalized, grad_normalized_dtype, updated, weight, mean,
            rstd, mask, grad_x, grad_branch, branch_dtype, grad_weight, grad_bias, rows,
            hidden, dropout_p, int(bool(training)), int(bool(deterministic)),
            int(bool(accumulate_parameters)), workspace, workspace_bytes, stream,
        )
    )


# include/rln.h RLN_NOALLOC_SCRATCH_BYTES: rln_backward_noalloc's per-device scratch.
NOALLOC_SCRATCH_BYTES = 4 << 20


def backward_noalloc(
    grad_updated, grad_normalized, updated, weight, mean, rstd, mask, grad_x,
    grad_branch, branch_dtype, grad_weight, grad_bias, rows, hidden, dropout_p,
    training, deterministic, stream=None, accumulate_parameters=False,
    grad_normalized_dtype=RLN_DTYPE_F32,
):
    """Call ``rln_backward_noalloc`` (no workspace, nothing allocated); raises RlnError."""
    _check(
        library().rln_backward_noalloc(
            grad_updated, grad_normalized, grad_normalized_dtype, updated, weight, mean,
            rstd, mask, grad_x, grad_branch, branch_dtype, grad_weight, grad_bias, rows,
            hidden, dropout_p, int(bool(training)), int(bool(deterministic)),
            int(bool(accumulate_parameters)), stream,
        )
    )


def backward_workspace_bytes(rows: int, hidden: int, deterministic: bool) -> int:
    return int(library().rln_backward_workspace_bytes(rows, hidden, int(bool(deterministic))))


def philox_increment(hidden: int, threads: int = 0) -> int:
    return int(library().rln_philox_increment(hidden, threads))


def mask_words(rows: int, hidden: int) -> int:
    return int(library().rln_mask_words(rows, hidden))
