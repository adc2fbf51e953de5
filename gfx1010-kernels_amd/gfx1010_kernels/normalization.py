"""Public residual-add + dropout + LayerNorm API and its dispatch.

Drop-in for the reference's gfx1010_kernels/normalization.py:

* ``residual_layer_norm`` (reference :149-298) returns ``(updated, normalized)``;
  ``implementation`` is one of ``"auto"``, ``"gfx950"`` (strict native),
  ``"gfx1010"`` (accepted alias of the strict native mode, so callers written
  for the reference keep working), ``"torch"`` and ``"triton"``.
* ``can_use_residual_layer_norm`` (reference :135-146) and
  ``residual_layer_norm_status`` (reference :75-94) keep their signatures and
  return types.

Dispatch rules (same order and messages as the reference):

* strict native modes check only ``x.is_cuda``, ``x.ndim`` and the hidden
  size in Python, then the backend status, and leave every other check to the
  native extension (reference :174-207);
* ``auto`` validates inputs (``_input_reason``, reference :97-132) and falls
  back to the PyTorch decomposition with a ``RuntimeWarning`` when they are not
  eligible (reference :229-242, :266-285). One difference: on a gfx950 device
  whose native extension cannot be loaded, ``auto`` raises instead of falling
  back, so a broken install on the target hardware is never silently served by
  the slow path;
* ``"triton"`` is not part of this build and raises ``RuntimeError``;
* the native path serves every multiple of 64 from 128 to 8192 (the reference
  compiles 128, 256, 384, 512, 768 and 1024 only, reference :12), so ``auto``
  accepts hidden sizes up to 8192 where the reference stops at 1024 (:118-120).
"""

from __future__ import annotations

from functools import lru_cache
import warnings

import torch
from torch.nn import functional as F

from ._normalization_native import (
    MAX_NATIVE_HIDDEN_SIZE,
    NATIVE_HIDDEN_SIZES,
    NATIVE_HIDDEN_SIZES_TEXT,
    TARGET_ARCHITECTURE,
    native_residual_layer_norm,
    native_residual_layer_norm_if_supported,
)
from ._ops import residual_layer_norm_op
from ._status import BackendStatus

MIN_HIDDEN_SIZE = 128
MAX_HIDDEN_SIZE = MAX_NATIVE_HIDDEN_SIZE

IMPLEMENTATIONS = ("auto", TARGET_ARCHITECTURE, "gfx1010", "triton", "torch")
BRANCH_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
NORMALIZED_DTYPES = (torch.float32, torch.float16, torch.bfloat16)
_STRICT_NATIVE = frozenset({TARGET_ARCHITECTURE, "gfx1010"})
_NATIVE_SIZES = frozenset(NATIVE_HIDDEN_SIZES)
_UNAVAILABLE = f"{TARGET_ARCHITECTURE} native residual LayerNorm is unavailable"


def _torch_residual_layer_norm(x, branch, weight, bias, dropout_p, eps, training,
                               normalized_dtype=None):
    """PyTorch decomposition (reference normalization.py:15-33); a requested
    ``normalized_dtype`` casts the LayerNorm output."""
    dropped = F.dropout(branch, dropout_p, training) if training else branch
    updated = x + dropped
    normalized = F.layer_norm(updated, (updated.shape[-1],), weight, bias, eps)
    if normalized_dtype is not None:
        normalized = normalized.to(normalized_dtype)
    return updated, normalized


def _architecture_of(properties):
    name = getattr(properties, "gcnArchName", None)
    if name is None:
        name = getattr(properties, "gcn_arch_name", "") or ""
    return name.split(":", 1)[0]


@lru_cache(maxsize=None)
def _native_status(device_index):
    if not torch.cuda.is_available():
        return BackendStatus(False, None, None, "PyTorch CUDA/HIP is unavailable")
    if torch.version.hip is None:
        return BackendStatus(
            False,
            torch.cuda.get_device_name(device_index),
            None,
            "PyTorch was not built with ROCm",
        )
    properties = torch.cuda.get_device_properties(device_index)
    architecture = _architecture_of(properties)
    if architecture != TARGET_ARCHITECTURE:
        return BackendStatus(
            False,
            properties.name,
            architecture,
            f"the native extension targets {TARGET_ARCHITECTURE}",
        )
    from ._normalization_native import native_extension_status

    available, reason = native_extension_status()
    return BackendStatus(
        available,
        properties.name,
        architecture,
        f"{TARGET_ARCHITECTURE} native normalization backend is ready"
        if available
        else reason,
    )


def residual_layer_norm_status(device=None):
    """Return the cached ``BackendStatus`` of the native backend on ``device``."""
    if isinstance(device, torch.device) and device.type == "cuda" and device.index is not None:
        # A HIP tensor's device (the per-call case): _native_status checks
        # availability itself, once per device.
        return _native_status(device.index)
    if not torch.cuda.is_available():
        return BackendStatus(False, None, None, "PyTorch CUDA/HIP is unavailable")
    if device is None:
        device_index = torch.cuda.current_device()
    else:
        resolved = torch.device(device)
        if resolved.type != "cuda":
            return BackendStatus(False, str(resolved), None, "the device must be a HIP GPU")
        device_index = (
            torch.cuda.current_device() if resolved.index is None else resolved.index
        )
    return _native_status(device_index)


def _input_reason(x, branch, weight, bias, dropout_p, eps):
    """Why the fused path cannot serve these inputs, or None if it can."""
    if not x.is_cuda:
        return "x must be a HIP tensor"
    if not branch.is_cuda or not weight.is_cuda or not bias.is_cuda:
        return "x, branch, weight and bias must be HIP tensors"
    if not (x.device == branch.device == weight.device == bias.device):
        return "x, branch, weight and bias must be on the same device"
    if x.ndim < 2 or branch.shape != x.shape:
        return "x and branch must have the same shape with at least two dimensions"
    hidden_size = x.shape[-1]
    if not MIN_HIDDEN_SIZE <= hidden_size <= MAX_HIDDEN_SIZE:
        return f"hidden size must be between {MIN_HIDDEN_SIZE} and {MAX_HIDDEN_SIZE}"
    if hidden_size % 8 != 0:
        return "hidden size must be divisible by 8"
    if weight.shape != (hidden_size,) or bias.shape != (hidden_size,):
        return "weight and bias must match the final tensor dimension"
    if x.dtype != torch.float32:
        return "the optimized residual stream requires float32 x"
    if branch.dtype not in BRANCH_DTYPES:
        return "branch must use float16, bfloat16 or float32"
    if weight.dtype != torch.float32 or bias.dtype != torch.float32:
        return "weight and bias must use float32"
    if not all(tensor.is_contiguous() for tensor in (x, branch, weight, bias)):
        return "x, branch, weight and bias must be contiguous"
    if not 0.0 <= dropout_p < 1.0:
        return "dropout_p must be in [0, 1)"
    if eps <= 0.0:
        return "eps must be positive"
    if x.numel() == 0:
        return "empty tensors use the PyTorch fallback"
    return None


def can_use_residual_layer_norm(x, branch, weight, bias, dropout_p=0.0, eps=1e-5):
    """True when ``residual_layer_norm(..., implementation="auto")`` runs natively."""
    reason = _input_reason(x, branch, weight, bias, dropout_p, eps)
    if reason is not None or x.shape[-1] not in _NATIVE_SIZES:
        return False
    return residual_layer_norm_status(x.device).available


# Device indices whose backend status is known to be available: the per-call
# check of the strict path is one dict lookup (small calls are host-bound).
_READY_DEVICES: set = set()


def _strict_native(x, branch, weight, bias, dropout_p, eps, training, normalized_dtype):
    if not x.is_cuda:
        raise RuntimeError(f"{_UNAVAILABLE}: x must be a HIP tensor")
    if x.ndim == 0:
        raise RuntimeError(f"{_UNAVAILABLE}: x must have at least two dimensions")
    if x.shape[-1] not in _NATIVE_SIZES:
        raise RuntimeError(
            f"{_UNAVAILABLE}: native hidden size must be one of {NATIVE_HIDDEN_SIZES_TEXT}"
        )
    device_index = x.get_device()
    if device_index not in _READY_DEVICES:
        status = residual_layer_norm_status(x.device)
        if not status.available:
            raise RuntimeError(f"{_UNAVAILABLE}: {status.reason}")
        _READY_DEVICES.add(device_index)
    return native_residual_layer_norm(
        x, branch, weight, bias, dropout_p, eps, training, normalized_dtype)


def _fall_back(reason, x, branch, weight, bias, dropout_p, eps, training, normalized_dtype):
    warnings.warn(
        f"{TARGET_ARCHITECTURE} native residual LayerNorm was not used: {reason}",
        RuntimeWarning,
        stacklevel=3,
    )
    return _torch_residual_layer_norm(
        x, branch, weight, bias, dropout_p, eps, training, normalized_dtype)


def _traced(x, branch, weight, bias, dropout_p, eps, training, normalized_dtype,
            implementation):
    """Dispatch while ``torch.compile`` traces: the native kernels run through
    the registered custom op (``gfx1010_kernels::rln_forward``) so the graph
    keeps them; the backend status is not queried (the op raises at run time
    if the extension is missing) and ``auto`` falls back without a warning."""
    native = x.is_cuda and x.ndim >= 2 and x.shape[-1] in _NATIVE_SIZES
    args = (x, branch, weight, bias, dropout_p, eps, training, normalized_dtype)
    if implementation in _STRICT_NATIVE:
        if not x.is_cuda:
            raise RuntimeError(f"{_UNAVAILABLE}: x must be a HIP tensor")
        if not native:
            raise RuntimeError(
                f"{_UNAVAILABLE}: native hidden size must be one of {NATIVE_HIDDEN_SIZES_TEXT}"
            )
        return residual_layer_norm_op(*args)
    if implementation == "triton":
        raise RuntimeError(
            f"{TARGET_ARCHITECTURE} residual LayerNorm is unavailable: "
            "the Triton backend is not part of the MI355X build"
        )
    if native and _input_reason(x, branch, weight, bias, dropout_p, eps) is None:
        return residual_layer_norm_op(*args)
    return _torch_residual_layer_norm(*args)


def residual_layer_norm(
    x,
    branch,
    weight,
    bias,
    dropout_p=0.0,
    eps=1e-5,
    training=True,
    *,
    implementation="auto",
    normalized_dtype=None,
):
    """Fused ``dropout(branch) -> x + . -> LayerNorm``; returns ``(updated, normalized)``.

    ``updated`` is the new fp32 residual stream and ``normalized`` its
    LayerNorm with ``weight``/``bias``, in fp32 or, when ``normalized_dtype``
    is ``torch.float16`` / ``torch.bfloat16``, rounded to that type for a
    half-precision consumer (the reference always returns fp32). ``branch``
    may be fp32, fp16 or bf16. Supports first-order autograd, HIP graph
    capture and ``torch.compile``.
    """
    if implementation not in IMPLEMENTATIONS:
        raise ValueError(
            "implementation must be 'auto', 'gfx950', 'gfx1010', 'triton' or 'torch'"
        )
    if normalized_dtype is not None and normalized_dtype not in NORMALIZED_DTYPES:
        raise ValueError("normalized_dtype must be None, torch.float32, torch.float16 "
                         "or torch.bfloat16")
    args = (x, branch, weight, bias, dropout_p, eps, training, normalized_dtype)
    if implementation == "torch":
        return _torch_residual_layer_norm(*args)
    if torch.compiler.is_compiling():
        return _traced(*args, implementation)
    if implementation in _STRICT_NATIVE:
        return _strict_native(*args)
    # Inputs the fused kernels serve, on a device whose backend is known to be
    # ready: one C++ check and call. The reasons below are only worked out
    # when it declines.
    if (implementation == "auto" and x.is_cuda and x.ndim >= 2
            and x.get_device() in _READY_DEVICES):
        result = native_residual_layer_norm_if_supported(
            x, branch, weight, bias, dropout_p, eps, training, normalized_dtype)
        if result is not None:
            return result

    reason = _input_reason(x, branch, weight, bias, dropout_p, eps)
    if implementation == "triton":
        raise RuntimeError(
            f"{TARGET_ARCHITECTURE} residual LayerNorm is unavailable: "
            + (reason or "the Triton backend is not part of the MI355X build")
        )
    if reason is not None:
        return _fall_back(reason, *args)
    if x.shape[-1] not in _NATIVE_SIZES:
        return _fall_back(f"native hidden size must be one of {NATIVE_HIDDEN_SIZES_TEXT}", *args)
    status = residual_layer_norm_status(x.device)
    if not status.available:
        if status.architecture == TARGET_ARCHITECTURE:
            raise RuntimeError(f"{_UNAVAILABLE}: {status.reason}")
        return _fall_back(status.reason, *args)
    _READY_DEVICES.add(x.get_device())
    # The extension guards x's device itself (the reference wraps this call in
    # torch.cuda.device, normalization.py:289, which costs two device switches
    # per call here).
    return native_residual_layer_norm(
        x, branch, weight, bias, float(dropout_p), float(eps), bool(training),
        normalized_dtype=normalized_dtype,
    )
