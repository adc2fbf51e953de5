"""``torch.library`` registration of the native residual LayerNorm.

The eager path runs the C++ autograd function of the ``_C`` module
(``_C.residual_layer_norm``, mirroring csrc/residual_layer_norm_bindings.cpp:10-125).
That function is opaque to ``torch.compile``; the two operators registered here
expose the same kernels as functional custom ops with fake (meta) kernels for
shape inference and an autograd formula, so that a compiled graph keeps the
fused op instead of breaking around it (the reference does not support
``torch.compile``; docs/residual_layer_norm.md:301-302).

* ``gfx1010_kernels::rln_forward(x, branch, weight, bias, dropout_p, eps, training,
  normalized_dtype, nonce) -> (updated, normalized, mean, rstd, mask)`` runs
  ``_C.residual_layer_norm_forward`` with the eager path's ``threads``; with
  dropout it reserves its Philox offsets from the device's default generator
  when it executes, exactly as the eager path does, so compiled and eager runs
  draw the same masks from the same RNG state. ``nonce`` is a fresh zero-size
  tensor per call (``residual_layer_norm_op`` makes it): the op draws from the
  generator, so two calls with equal arguments are different computations,
  and the nonce keeps a compiler from merging them. AOTAutograd's common
  subexpression pass merges identical calls of a functional custom op, but
  never two ``aten.empty`` nodes, so each call's nonce differs.
* ``gfx1010_kernels::rln_backward(grad_updated, grad_normalized, updated, weight,
  mean, rstd, mask, dropout_p, training, branch_dtype, compute_parameters)
  -> (grad_x, grad_branch, grad_weight, grad_bias)`` runs
  ``_C.residual_layer_norm_backward``; a missing upstream gradient counts as
  zero, and the weight/bias gradients are zero when ``grad_normalized`` is.
  With ``compute_parameters`` false (the backward pass needs neither weight
  nor bias gradient: frozen parameters, or gradients taken for the inputs
  only) the weight/bias sums are skipped and those two outputs are empty.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from ._normalization_native import TARGET_ARCHITECTURE, _extension, launch_threads

_NAMESPACE = "gfx1010_kernels"

# Interface-compatibility launch hints the raw backward range-checks
# (threads, block_rows, parameter_threads, parameter_groups).
_BACKWARD_HINTS = (128, 64, 64, 1)


def _native():
    extension, reason = _extension()
    if extension is None:
        raise RuntimeError(f"{TARGET_ARCHITECTURE} native extension is unavailable: {reason}")
    return extension


@torch.library.custom_op(f"{_NAMESPACE}::rln_forward", mutates_args=(), device_types="cuda")
def rln_forward(
    x: Tensor,
    branch: Tensor,
    weight: Tensor,
    bias: Tensor,
    dropout_p: float,
    eps: float,
    training: bool,
    normalized_dtype: Optional[torch.dtype] = None,
    nonce: Optional[Tensor] = None,
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    return tuple(
        _native().residual_layer_norm_forward(
            x, branch, weight, bias, float(dropout_p), float(eps), bool(training),
            launch_threads(x.shape[-1]),
            normalized_dtype=normalized_dtype,
        )
    )


@rln_forward.register_fake
def _rln_forward_fake(x, branch, weight, bias, dropout_p, eps, training, normalized_dtype=None,
                      nonce=None):
    hidden = x.shape[-1]
    rows = x.numel() // hidden
    mask_words = rows * (hidden // 32) if (training and dropout_p > 0.0) else 0
    return (
        torch.empty_like(x, memory_format=torch.contiguous_format),
        torch.empty_like(x, dtype=normalized_dtype or torch.float32,
                         memory_format=torch.contiguous_format),
        x.new_empty((rows,)),
        x.new_empty((rows,)),
        x.new_empty((mask_words,), dtype=torch.int32),
    )


@torch.library.custom_op(f"{_NAMESPACE}::rln_backward", mutates_args=(), device_types="cuda")
def rln_backward(
    grad_updated: Optional[Tensor],
    grad_normalized: Optional[Tensor],
    updated: Tensor,
    weight: Tensor,
    mean: Tensor,
    rstd: Tensor,
    mask: Tensor,
    dropout_p: float,
    training: bool,
    branch_dtype: torch.dtype,
    compute_parameters: bool = True,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    grad_x, grad_branch, grad_weight, grad_bias = _native().residual_layer_norm_backward(
        grad_updated, grad_normalized, updated, weight, mean, rstd, mask, float(dropout_p),
        bool(training), branch_dtype == torch.float16, *_BACKWARD_HINTS,
        bool(compute_parameters), branch_dtype=branch_dtype,
    )
    if not compute_parameters:
        grad_weight = updated.new_empty((0,))
        grad_bias = updated.new_empty((0,))
    return grad_x, grad_branch, grad_weight, grad_bias


@rln_backward.register_fake
def _rln_backward_fake(grad_updated, grad_normalized, updated, weight, mean, rstd, mask,
                       dropout_p, training, branch_dtype, compute_parameters=True):
    hidden = updated.shape[-1] if compute_parameters else 0
    return (
        torch.empty_like(updated, memory_format=torch.contiguous_format),
        torch.empty_like(updated, dtype=branch_dtype, memory_format=torch.contiguous_format),
        updated.new_empty((hidden,)),
        updated.new_empty((hidden,)),
    )


def _setup_context(ctx, inputs, output):
    _, branch, weight, _, dropout_p, _, training, _, _ = inputs
    updated, _, mean, rstd, mask = output
    ctx.save_for_backward(updated, weight, mean, rstd, mask)
    ctx.dropout_p = dropout_p
    ctx.training = training
    ctx.branch_dtype = branch.dtype
    ctx.mark_non_differentiable(mean, rstd, mask)
    ctx.set_materialize_grads(False)


def _backward(ctx, grad_updated, grad_normalized, _grad_mean, _grad_rstd, _grad_mask):
    if grad_updated is None and grad_normalized is None:
        return None, None, None, None, None, None, None, None, None
    updated, weight, mean, rstd, mask = ctx.saved_tensors
    if grad_updated is not None:
        grad_updated = grad_updated.contiguous()
    if grad_normalized is not None:
        grad_normalized = grad_normalized.contiguous()
    # Weight/bias sums only when this backward pass asks for them.
    parameters = grad_normalized is not None and (ctx.needs_input_grad[2]
                                                  or ctx.needs_input_grad[3])
    grad_x, grad_branch, grad_weight, grad_bias = rln_backward(
        grad_updated, grad_normalized, updated, weight, mean, rstd, mask, ctx.dropout_p,
        ctx.training, ctx.branch_dtype, parameters,
    )
    if not parameters:
        grad_weight = grad_bias = None
    return grad_x, grad_branch, grad_weight, grad_bias, None, None, None, None, None


rln_forward.register_autograd(_backward, setup_context=_setup_context)


def residual_layer_norm_op(x, branch, weight, bias, dropout_p, eps, training,
                           normalized_dtype=None):
    """``(updated, normalized)`` through the registered custom op. Each call
    passes a new zero-size nonce, so two dropout calls on equal arguments stay
    two draws under ``torch.compile``."""
    nonce = torch.empty(0, device=x.device)
    updated, normalized, _, _, _ = rln_forward(
        x, branch, weight, bias, float(dropout_p), float(eps), bool(training), normalized_dtype,
        nonce,
    )
    return updated, normalized


__all__ = ["rln_backward", "rln_forward", "residual_layer_norm_op"]
