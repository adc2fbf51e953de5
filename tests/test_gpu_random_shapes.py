"""Seeded random configurations across the whole supported range.

Each case draws a hidden size (any multiple of 64 from 128 to 8192), a row
count, branch and normalized dtypes, dropout, training mode and reduction
mode, then checks the forward and the backward against the fp64 oracle. The
draws are fixed by the case index, so every run checks the same cases. A
second set draws from the reference's six hidden sizes only, with a random
`threads` (the reference's dropout stream of a 128-, 192- or 256-thread
launch) and a random generator offset. A third set draws large launches
(2^22 to 2^26 elements, any hidden size), where the grid and schedule rules
of large launches apply, and checks every element of every output
(parity.check_full_tensor) and the weight/bias sums against a float64
reduction.
"""

import numpy as np
import pytest
import torch

from gfx1010_kernels import _C
from gfx1010_kernels._normalization_native import NATIVE_HIDDEN_SIZES
from parity import (
    SPECIALIZED_HIDDEN_SIZES,
    check_backward,
    check_forward,
    generator_state,
    make_grads,
    make_inputs,
)
from parity import check_full_tensor
from test_gpu_backward import deterministic_algorithms, raw_backward
from test_gpu_configs import check_parameter_gradients, device_inputs

pytestmark = pytest.mark.gpu
EPS = 1e-5
DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def draw(case, sizes=NATIVE_HIDDEN_SIZES):
    rng = np.random.default_rng(1000 + case)
    hidden = int(rng.choice(sizes))
    max_rows = max(1, (1 << 20) // hidden)
    rows = int(min(max_rows, rng.choice([1, 2, 3, 7, 31, 64, 255, 513, 1024, 2047, 4099])))
    return dict(
        hidden=hidden,
        rows=rows,
        branch=DTYPES[int(rng.integers(3))],
        normalized=DTYPES[int(rng.integers(3))],
        dropout_p=float(rng.choice([0.0, 0.1, 0.5])),
        training=bool(rng.integers(4) != 0),
        deterministic=bool(rng.integers(2)),
        x_mean=float(rng.choice([0.0, 3.0, 100.0])),
        threads=int(rng.choice([128, 192, 256])),
        offset_steps=int(rng.integers(0, 1 << 20)),
    )


@pytest.mark.parametrize("case", range(128))
def test_random_configuration_matches_oracle(case):
    c = draw(case)
    print(f"[random] case {case}: {c}", flush=True)
    inputs = make_inputs((c["rows"], c["hidden"]), c["branch"], seed=case, x_mean=c["x_mean"])
    grad_updated, grad_normalized = make_grads((c["rows"], c["hidden"]), seed=case + 500)
    grad_normalized = grad_normalized.to(c["normalized"])
    torch.cuda.manual_seed(case)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, c["dropout_p"], EPS, c["training"], 128,
                                             normalized_dtype=c["normalized"])
    keep, scale = check_forward(outputs, inputs, c["dropout_p"], c["training"], EPS, seed,
                                offset, f"case {case}")
    with deterministic_algorithms(c["deterministic"]):
        gradients = raw_backward(grad_updated, grad_normalized, outputs, inputs[2],
                                 c["dropout_p"], c["branch"], training=c["training"])
    check_backward(gradients, grad_updated, grad_normalized, outputs[0], inputs[2], EPS, keep,
                   scale, f"case {case}")


@pytest.mark.parametrize("case", [*range(100, 124), *range(200, 240)])
def test_random_reference_stream_configuration_matches_oracle(case):
    c = draw(case, SPECIALIZED_HIDDEN_SIZES)
    c["dropout_p"] = c["dropout_p"] or 0.25
    c["training"] = True
    print(f"[random-reference] case {case}: {c}", flush=True)
    inputs = make_inputs((c["rows"], c["hidden"]), c["branch"], seed=case, x_mean=c["x_mean"])
    grad_updated, grad_normalized = make_grads((c["rows"], c["hidden"]), seed=case + 500)
    grad_normalized = grad_normalized.to(c["normalized"])
    torch.cuda.manual_seed(case)
    generator = torch.cuda.default_generators[0]
    generator.set_offset(4 * c["offset_steps"])
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, c["dropout_p"], EPS, True, c["threads"],
                                             normalized_dtype=c["normalized"])
    keep, scale = check_forward(outputs, inputs, c["dropout_p"], True, EPS, seed, offset,
                                f"case {case}", threads=c["threads"])
    with deterministic_algorithms(c["deterministic"]):
        gradients = raw_backward(grad_updated, grad_normalized, outputs, inputs[2],
                                 c["dropout_p"], c["branch"], training=True)
    check_backward(gradients, grad_updated, grad_normalized, outputs[0], inputs[2], EPS, keep,
                   scale, f"case {case}")


@pytest.mark.parametrize("case", range(300, 316))
def test_random_large_configuration_matches_oracle(case):
    rng = np.random.default_rng(1000 + case)
    hidden = int(rng.integers(2, 129)) * 64
    rows = max(1, int(2 ** rng.uniform(22, 26)) // hidden + int(rng.integers(-3, 4)))
    branch_dtype = DTYPES[int(rng.integers(3))]
    dropout_p = float(rng.choice([0.1, 0.15, 0.5]))
    deterministic = bool(rng.integers(2))
    threads = 192 if hidden == 1024 else 128
    print(f"[random-large] case {case}: rows={rows} H={hidden} {branch_dtype} p={dropout_p} "
          f"deterministic={deterministic}", flush=True)
    inputs, grads = device_inputs(rows, hidden, branch_dtype, seed=case)
    torch.cuda.manual_seed(case)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, dropout_p, EPS, True, threads)
    with deterministic_algorithms(deterministic):
        gradients = raw_backward(grads[0], grads[1], outputs, inputs[2], dropout_p, branch_dtype)
    check_full_tensor(inputs, grads, outputs, gradients, dropout_p, EPS, seed, offset,
                      threads=threads, what=f"case {case}: {rows} x {hidden}")
    check_parameter_gradients(outputs[0], grads[1], gradients)
