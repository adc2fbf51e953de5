"""Pre-norm transformer integration of the fused residual LayerNorm.

The reference documents the integration as a recipe
(docs/residual_layer_norm.md:51-83): replace ``x = x + branch; h = ln(x)`` by
one ``residual_layer_norm`` call that takes the parameters of the LayerNorm
that *consumes* the new residual stream, pass the sublayer's pre-dropout
output with the original dropout probability, and keep the existing
``LayerNorm`` modules so that checkpoint ``state_dict`` keys do not change.
This module is that recipe as code:

* :func:`residual_norm` fuses one ``x + dropout(branch)`` with the
  ``nn.LayerNorm`` that follows it, reading the module's weight, bias and eps;
* :func:`prenorm_forward` runs a stack of pre-norm blocks
  (``h = ln_1(x); x = x + drop(attn(h)); h = ln_2(x); x = x + drop(mlp(h))``
  per block, then the final norm) with every residual add fused into the
  LayerNorm after it: a block's ``ln_2`` after its attention, the next
  block's ``ln_1`` after its MLP, and the final norm after the last MLP. Only
  the first ``ln_1`` (no residual add before it) runs as a plain LayerNorm.

Neither function owns parameters: they read the caller's modules, so a model
that switches its ``forward`` to them keeps its ``state_dict`` unchanged.
"""

from __future__ import annotations

from typing import Callable, Sequence, Union

import torch
from torch import nn
from torch.nn import functional as F

from .normalization import residual_layer_norm

# How a block exposes a sublayer or norm: an attribute name, or a function of
# the block (and, for sublayers, the normalized input).
Accessor = Union[str, Callable]


def _check_norm(norm: nn.Module, hidden: int) -> None:
    if not isinstance(norm, nn.LayerNorm):
        raise TypeError(f"expected torch.nn.LayerNorm, got {type(norm).__name__}")
    if tuple(norm.normalized_shape) != (hidden,):
        raise ValueError(
            f"LayerNorm normalizes {tuple(norm.normalized_shape)}, the residual stream has "
            f"hidden size {hidden}")
    if norm.weight is None or norm.bias is None:
        raise ValueError("LayerNorm needs elementwise affine weight and bias")


def residual_norm(x, branch, norm: nn.LayerNorm, dropout_p: float = 0.0, training: bool = True,
                  *, implementation: str = "auto", normalized_dtype=None):
    """``x + dropout(branch)`` followed by ``norm``, as one fused operation.

    Returns ``(updated, normalized)`` like ``residual_layer_norm``; ``norm``
    supplies weight, bias and eps and keeps its parameters (and their
    ``state_dict`` keys) in the caller's model.
    """
    _check_norm(norm, x.shape[-1])
    return residual_layer_norm(
        x, branch, norm.weight, norm.bias, dropout_p=dropout_p, eps=norm.eps,
        training=training, implementation=implementation, normalized_dtype=normalized_dtype)


def _module(block: nn.Module, accessor: Accessor) -> nn.Module:
    return getattr(block, accessor) if isinstance(accessor, str) else accessor(block)


def _sublayer(block: nn.Module, accessor: Accessor, hidden_states):
    if isinstance(accessor, str):
        return getattr(block, accessor)(hidden_states)
    return accessor(block, hidden_states)


def prenorm_forward(
    x: torch.Tensor,
    blocks: Sequence[nn.Module],
    final_norm: nn.LayerNorm,
    *,
    dropout_p: float = 0.0,
    training: bool = True,
    attention: Accessor = "attn",
    mlp: Accessor = "mlp",
    ln1: Accessor = "ln_1",
    ln2: Accessor = "ln_2",
    implementation: str = "auto",
    normalized_dtype=None,
):
    """Run pre-norm blocks with fused residual LayerNorms; returns ``(x, out)``.

    ``x`` is the fp32 residual stream after the last block and ``out`` the
    final norm of it. ``attention`` and ``mlp`` name each block's sublayers
    (attribute names, called with the normalized input, or functions
    ``f(block, normalized)``); they must return the sublayer output *before*
    its residual dropout, which the fused operation applies with
    ``dropout_p``. ``ln1`` and ``ln2`` name the blocks' LayerNorms (attribute
    names or functions ``f(block)``). ``normalized_dtype`` (fp16 / bf16)
    rounds every normalized output, including ``out``, for half-precision
    sublayers; the residual stream stays fp32.
    """
    if len(blocks) == 0:
        raise ValueError("prenorm_forward needs at least one block")
    hidden = x.shape[-1]
    first = _module(blocks[0], ln1)
    _check_norm(first, hidden)
    normalized = F.layer_norm(x, (hidden,), first.weight, first.bias, first.eps)
    if normalized_dtype is not None:
        normalized = normalized.to(normalized_dtype)
    options = dict(implementation=implementation, normalized_dtype=normalized_dtype)
    for index, block in enumerate(blocks):
        x, normalized = residual_norm(x, _sublayer(block, attention, normalized),
                                      _module(block, ln2), dropout_p, training, **options)
        following = _module(blocks[index + 1], ln1) if index + 1 < len(blocks) else final_norm
        x, normalized = residual_norm(x, _sublayer(block, mlp, normalized), following,
                                      dropout_p, training, **options)
    return x, normalized


__all__ = ["prenorm_forward", "residual_norm"]
