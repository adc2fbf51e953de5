"""The reference's CPU path, restated - TEST INFRASTRUCTURE / CPU BASELINE ONLY.

``residual_layer_norm_torch`` is the PyTorch decomposition the reference falls
back to (gfx1010_kernels/normalization.py:15-33): ``F.dropout`` on the branch
in training, one add, ``F.layer_norm``. bench.py times it on the host CPU as
``cpu_baseline`` (kind "port"); tests use it as an independent checker.
"""

from __future__ import annotations

import torch
from torch.nn import functional as F


def residual_layer_norm_torch(x, branch, weight, bias, dropout_p=0.0, eps=1e-5, training=True):
    dropped = F.dropout(branch, dropout_p, True) if training else branch
    updated = x + dropped
    normalized = F.layer_norm(updated, (updated.shape[-1],), weight, bias, eps)
    return updated, normalized


def fwd_bwd_step(x, branch, weight, bias, grad_updated, grad_normalized, dropout_p, eps):
    """One training step of the decomposition: forward plus autograd.grad."""
    inputs = (x, branch, weight, bias)
    outputs = residual_layer_norm_torch(*inputs, dropout_p=dropout_p, eps=eps, training=True)
    return torch.autograd.grad(outputs, inputs, (grad_updated, grad_normalized))
