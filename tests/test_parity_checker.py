"""The full-tensor parity checker (parity.check_full_tensor) on the CPU.

Fed the oracle's own outputs (rounded to the kernels' storage types) it must
pass; fed outputs with a planted mistake - one mask bit, one ulp of `updated`,
a normalized value off by more than the bar, one row's gradient with a
dropped term, a half-precision gradient two ulps off - it must fail. This
pins the checker the GPU tests use at the BASELINE sizes.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import rln_oracle as oracle
from parity import check_full_tensor

ROWS, HIDDEN, P, EPS = 40, 128, 0.1, 1e-5
SEED, OFFSET, THREADS = 77, 8, 128


def oracle_outputs():
    generator = torch.Generator().manual_seed(5)
    x = torch.randn(ROWS, HIDDEN, generator=generator)
    branch = torch.randn(ROWS, HIDDEN, generator=generator).half()
    weight = 1.0 + 0.02 * torch.randn(HIDDEN, generator=generator)
    bias = 0.02 * torch.randn(HIDDEN, generator=generator)
    grad_updated = torch.randn(ROWS, HIDDEN, generator=generator)
    grad_normalized = torch.randn(ROWS, HIDDEN, generator=generator)
    _, scale, threshold = oracle.dropout_constants(P, True)
    words = oracle.reference_mask_words(ROWS, HIDDEN, THREADS, SEED, OFFSET, threshold)
    keep = oracle.decode_mask(words, ROWS, HIDDEN)
    forward = oracle.forward(x.numpy(), branch.numpy(), weight.numpy(), bias.numpy(), EPS,
                             keep=keep, scale=scale, branch_type="f16")
    backward = oracle.backward(grad_updated.numpy(), grad_normalized.numpy(), forward["updated"],
                               weight.numpy(), EPS, keep=keep, scale=scale)
    inputs = (x, branch, weight, bias)
    grads = (grad_updated, grad_normalized)
    outputs = [torch.from_numpy(forward["updated"].copy()),
               torch.from_numpy(forward["normalized"]).float(),
               torch.from_numpy(forward["mean"]).float(),
               torch.from_numpy(forward["rstd"]).float(),
               torch.from_numpy(words.view(np.int32).copy())]
    gradients = [torch.from_numpy(backward["grad_x"]).float(),
                 torch.from_numpy(backward["grad_branch"]).half()]
    return inputs, grads, outputs, gradients


def run(inputs, grads, outputs, gradients):
    check_full_tensor(inputs, grads, outputs, gradients, P, EPS, SEED, OFFSET, THREADS,
                      chunk=16, what="planted")


def test_oracle_outputs_pass():
    run(*oracle_outputs())


def flip_mask_bit(outputs, gradients):
    outputs[4][7] ^= 1 << 5


def nudge_updated(outputs, gradients):
    bits = outputs[0].view(torch.int32)
    bits[33, 17] += 1


def shift_normalized(outputs, gradients):
    scale = outputs[1].abs().max()
    outputs[1][20, 3] += 3e-5 * scale


def drop_grad_term(outputs, gradients):
    # One row's grad_x without its upstream grad_updated term.
    inputs, grads, _, _ = oracle_outputs()
    gradients[0][25] -= grads[0][25]


def half_grad_two_ulps(outputs, gradients):
    value = gradients[1][11, 40].float()
    spacing = 2.0 ** (torch.floor(torch.log2(value.abs().clamp_min(2.0 ** -14))) - 10)
    gradients[1][11, 40] = (value + 2 * spacing).half()


@pytest.mark.parametrize("plant", [flip_mask_bit, nudge_updated, shift_normalized,
                                   drop_grad_term, half_grad_two_ulps])
def test_planted_mistake_is_caught(plant):
    inputs, grads, outputs, gradients = oracle_outputs()
    plant(outputs, gradients)
    with pytest.raises(AssertionError):
        run(inputs, grads, outputs, gradients)


# --- The fp32 conditioned bounds of the golden-fixture GPU test ---------------

GOLDEN = sorted((Path(__file__).parent / "golden").glob("*.npz"))


def _fixture(path):
    return dict(np.load(path, allow_pickle=False))


def _layer_norm_f32(u, w, b, eps, one_pass=False):
    """LayerNorm in float32 arithmetic: two-pass (the kernels' algorithm) or
    one-pass variance E[u^2] - E[u]^2 (the planted mistake)."""
    u = u.astype(np.float32)
    inverse = np.float32(1.0 / u.shape[1])
    mean = (u.sum(axis=1, dtype=np.float32) * inverse).astype(np.float32)
    if one_pass:
        square = (u * u).sum(axis=1, dtype=np.float32) * inverse
        variance = np.maximum(square - mean * mean, np.float32(0.0)).astype(np.float32)
    else:
        centred = u - mean[:, None]
        variance = ((centred * centred).sum(axis=1, dtype=np.float32) * inverse).astype(np.float32)
    rstd = (np.float32(1.0) / np.sqrt(variance + np.float32(eps))).astype(np.float32)
    return mean, rstd, ((u - mean[:, None]) * rstd[:, None] * w + b).astype(np.float32)


def _grad_x_f32(d, mean, rstd, drop_term=False):
    u = d["updated"]
    gy = d.get("grad_normalized", np.zeros_like(u))
    gu = d.get("grad_updated", np.zeros_like(u))
    xhat = ((u - mean[:, None]) * rstd[:, None]).astype(np.float32)
    q = (gy * d["weight"]).astype(np.float32)
    inverse = np.float32(1.0 / u.shape[1])
    mean_q = q.sum(axis=1, dtype=np.float32) * inverse
    mean_qx = (q * xhat).sum(axis=1, dtype=np.float32) * inverse
    if drop_term:
        mean_qx = mean_qx * 0
    return (gu + rstd[:, None] * ((q - mean_q[:, None]) - xhat * mean_qx[:, None])).astype(
        np.float32)


@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: p.stem)
def test_fp32_two_pass_meets_the_conditioned_bounds(path):
    from parity import assert_within, conditioned_bounds

    d = _fixture(path)
    bounds = conditioned_bounds(d["updated"], d["weight"], d["eps"], d.get("grad_updated"),
                                d.get("grad_normalized"))
    mean, rstd, normalized = _layer_norm_f32(d["updated"], d["weight"], d["bias"], d["eps"])
    assert assert_within(mean, d["mean"], bounds["mean"], "mean") < 0.5
    assert assert_within(rstd, d["rstd"], bounds["rstd"], "rstd") < 0.5
    assert assert_within(normalized, d["normalized"], bounds["normalized"], "normalized") < 0.5
    if "grad_x" in d:
        grad_x = _grad_x_f32(d, mean, rstd)
        assert assert_within(grad_x, d["grad_x"], bounds["grad_x"], "grad_x") < 0.5


@pytest.mark.parametrize("name", ["large_mean_h384", "nearly_constant_rows_eps1e-5"])
def test_one_pass_variance_breaks_the_bounds_on_ill_conditioned_rows(name):
    from parity import assert_within, conditioned_bounds

    d = _fixture(next(p for p in GOLDEN if p.stem == name))
    bounds = conditioned_bounds(d["updated"], d["weight"], d["eps"])
    _, rstd, _ = _layer_norm_f32(d["updated"], d["weight"], d["bias"], d["eps"], one_pass=True)
    with pytest.raises(AssertionError):
        assert_within(rstd, d["rstd"], bounds["rstd"], "one-pass rstd")


@pytest.mark.parametrize("name", ["backward_dropout_f16_h384", "backward_f32_h128",
                                  "backward_normalized_only_h256", "large_mean_h384",
                                  "nearly_constant_rows_eps1e-5"])
def test_a_dropped_gradient_term_breaks_the_bound(name):
    from parity import assert_within, conditioned_bounds

    d = _fixture(next(p for p in GOLDEN if p.stem == name))
    bounds = conditioned_bounds(d["updated"], d["weight"], d["eps"], d.get("grad_updated"),
                                d.get("grad_normalized"))
    mean, rstd, _ = _layer_norm_f32(d["updated"], d["weight"], d["bias"], d["eps"])
    with pytest.raises(AssertionError):
        assert_within(_grad_x_f32(d, mean, rstd, drop_term=True), d["grad_x"], bounds["grad_x"],
                      "grad_x without xhat * mean(q * xhat)")
