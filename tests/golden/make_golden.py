"""Write the golden vectors under tests/golden/ from PyTorch float64 (CPU).

The expected values come from PyTorch's own ``F.layer_norm`` and autograd,
i.e. the decomposition the reference falls back to
(gfx1010_kernels/normalization.py:15-33) and compares against in its tests
(tests/test_residual_layer_norm.py:12-31). The reference ships no stored
vectors, so these fixtures are generated here with fixed seeds; the inputs
follow the reference's test shapes and closed-form cases
(tests/test_residual_layer_norm_edge_cases.py:134-193).

Each case stores its inputs, a keep mask (dropout cases), and the float64
expected outputs. The float32 residual update is stored as torch computes it
(one fp32 add of x and the dropped branch); the float64 graph is built on
exactly that fp32 value, with gradients flowing to x and branch through the
chain rule of ``x + branch * keep * scale``.

Run: python tests/golden/make_golden.py
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch
from torch.nn import functional as F

OUT = Path(__file__).resolve().parent


def _dropout_scale(p: float) -> np.float32:
    p32 = np.float32(p)
    return np.float32(np.float32(1.0) / (np.float32(1.0) - p32))


def _case(name, x, branch, weight, bias, eps, keep=None, p=0.0, grad_updated=None,
          grad_normalized=None):
    """Compute torch float64 forward (+ backward when gradients are given)."""
    scale = _dropout_scale(p) if keep is not None else np.float32(1.0)
    xt = torch.from_numpy(x)
    bt = torch.from_numpy(branch)
    if keep is None:
        dropped = bt.float()
        mask_scale = torch.ones(x.shape, dtype=torch.float64)
    else:
        keep_t = torch.from_numpy(keep.astype(np.float32))
        dropped = bt.float() * keep_t * torch.tensor(float(scale), dtype=torch.float32)
        if branch.dtype == np.float16:
            dropped = dropped.half().float()
        mask_scale = torch.from_numpy(keep.astype(np.float64)) * float(scale)
    updated = (xt + dropped).numpy()

    x64 = torch.from_numpy(x.astype(np.float64)).requires_grad_(True)
    b64 = torch.from_numpy(branch.astype(np.float64)).requires_grad_(True)
    w64 = torch.from_numpy(weight.astype(np.float64)).requires_grad_(True)
    c64 = torch.from_numpy(bias.astype(np.float64)).requires_grad_(True)
    linear = x64 + b64 * mask_scale
    u64 = linear + (torch.from_numpy(updated.astype(np.float64)) - linear).detach()
    y64 = F.layer_norm(u64, (x.shape[-1],), w64, c64, eps)
    variance, mean = torch.var_mean(u64.detach(), dim=-1, unbiased=False)
    record = {
        "x": x,
        "branch": branch,
        "weight": weight,
        "bias": bias,
        "eps": np.float64(eps),
        "dropout_p": np.float64(p),
        "scale": np.float32(scale),
        "updated": updated,
        "normalized": y64.detach().numpy(),
        "mean": mean.numpy(),
        "rstd": (1.0 / torch.sqrt(variance + eps)).numpy(),
    }
    if keep is not None:
        record["keep"] = keep
    if grad_updated is not None or grad_normalized is not None:
        outputs, grads = [], []
        if grad_updated is not None:
            outputs.append(u64)
            grads.append(torch.from_numpy(grad_updated.astype(np.float64)))
            record["grad_updated"] = grad_updated
        if grad_normalized is not None:
            outputs.append(y64)
            grads.append(torch.from_numpy(grad_normalized.astype(np.float64)))
            record["grad_normalized"] = grad_normalized
        gx, gb, gw, gc = torch.autograd.grad(
            outputs, (x64, b64, w64, c64), grads, allow_unused=True
        )
        record["grad_x"] = gx.numpy()
        record["grad_branch"] = gb.numpy()
        if grad_normalized is not None:
            record["grad_weight"] = gw.numpy()
            record["grad_bias"] = gc.numpy()
    np.savez_compressed(OUT / f"{name}.npz", **record)
    return record


def _params(rng, hidden):
    weight = (1.0 + 0.02 * rng.standard_normal(hidden)).astype(np.float32)
    bias = (0.02 * rng.standard_normal(hidden)).astype(np.float32)
    return weight, bias


def main():
    rng = np.random.default_rng(20261201)

    rows, hidden = 5, 128
    x = rng.standard_normal((rows, hidden)).astype(np.float32)
    branch = rng.standard_normal((rows, hidden)).astype(np.float32)
    _case("forward_eval_f32_h128", x, branch, *_params(rng, hidden), 1e-5)

    rows, hidden = 7, 384
    x = rng.standard_normal((rows, hidden)).astype(np.float32)
    branch = (0.5 * rng.standard_normal((rows, hidden))).astype(np.float16)
    _case("forward_f16_h384", x, branch, *_params(rng, hidden), 1e-5)

    rows, hidden = 6, 256
    x = rng.standard_normal((rows, hidden)).astype(np.float32)
    branch = rng.standard_normal((rows, hidden)).astype(np.float16)
    keep = rng.random((rows, hidden)) >= 0.1
    _case("forward_dropout_f16_h256", x, branch, *_params(rng, hidden), 1e-5, keep=keep, p=0.1)

    rows, hidden = 9, 384
    x = rng.standard_normal((rows, hidden)).astype(np.float32)
    branch = (0.5 * rng.standard_normal((rows, hidden))).astype(np.float16)
    keep = rng.random((rows, hidden)) >= 0.15
    gu = rng.standard_normal((rows, hidden)).astype(np.float32)
    gy = rng.standard_normal((rows, hidden)).astype(np.float32)
    weight = rng.standard_normal(hidden).astype(np.float32)
    bias = rng.standard_normal(hidden).astype(np.float32)
    _case("backward_dropout_f16_h384", x, branch, weight, bias, 1e-5, keep=keep, p=0.15,
          grad_updated=gu, grad_normalized=gy)

    rows, hidden = 4, 128
    x = rng.standard_normal((rows, hidden)).astype(np.float32)
    branch = rng.standard_normal((rows, hidden)).astype(np.float32)
    gu = rng.standard_normal((rows, hidden)).astype(np.float32)
    gy = rng.standard_normal((rows, hidden)).astype(np.float32)
    _case("backward_f32_h128", x, branch, *_params(rng, hidden), 1e-5,
          grad_updated=gu, grad_normalized=gy)

    # Updated-only and normalized-only upstream gradients.
    rows, hidden = 3, 256
    x = rng.standard_normal((rows, hidden)).astype(np.float32)
    branch = rng.standard_normal((rows, hidden)).astype(np.float16)
    gu = rng.standard_normal((rows, hidden)).astype(np.float32)
    _case("backward_updated_only_h256", x, branch, *_params(rng, hidden), 1e-5, grad_updated=gu)
    gy = rng.standard_normal((rows, hidden)).astype(np.float32)
    _case("backward_normalized_only_h256", x, branch, *_params(rng, hidden), 1e-5,
          grad_normalized=gy)

    # Nearly-constant rows (reference tests/test_residual_layer_norm_edge_cases.py:134-193).
    hidden = 384
    columns = np.linspace(-1.0, 1.0, hidden, dtype=np.float32)
    centers = np.array([-3.0, 0.25, 4.0], dtype=np.float32)[:, None]
    x = (centers + columns[None, :] * np.float32(2e-4)).astype(np.float32)
    branch = np.ascontiguousarray(
        np.broadcast_to(-columns[None, :] * np.float32(5e-5), x.shape)).astype(np.float32)
    weight = np.linspace(0.75, 1.25, hidden, dtype=np.float32)
    bias = np.linspace(-0.1, 0.1, hidden, dtype=np.float32)
    upstream = np.ascontiguousarray(
        np.broadcast_to(np.sin(columns)[None, :], x.shape)).astype(np.float32)
    for eps, tag in ((1e-5, "1e-5"), (1e-3, "1e-3")):
        _case(f"nearly_constant_rows_eps{tag}", x, branch, weight, bias, eps,
              grad_normalized=upstream)

    # Large mean offset (x ~ N(100, 1)) stresses the variance.
    rows, hidden = 5, 384
    x = (100.0 + rng.standard_normal((rows, hidden))).astype(np.float32)
    branch = rng.standard_normal((rows, hidden)).astype(np.float32)
    gu = rng.standard_normal((rows, hidden)).astype(np.float32)
    gy = rng.standard_normal((rows, hidden)).astype(np.float32)
    _case("large_mean_h384", x, branch, *_params(rng, hidden), 1e-5,
          grad_updated=gu, grad_normalized=gy)


if __name__ == "__main__":
    torch.manual_seed(0)
    main()
    for path in sorted(OUT.glob("*.npz")):
        print(path.name, path.stat().st_size)
