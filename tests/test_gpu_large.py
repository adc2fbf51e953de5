"""Launches beyond 2^31 elements: every index is 64-bit.

One call over more than 2^31 elements per tensor (8.6 GB fp32 each, ~60 GB in
all, well inside MI355X's 288 GB), for a specialized and a multi-wave row
shape: every row matches the oracle (parity.check_full_tensor: the whole
mask bit for bit, `updated` bitwise, the rest against float64 on the device),
and the weight/bias gradients match a float64 reduction over all rows.
"""

import pytest
import torch

from gfx1010_kernels import _C
from parity import check_full_tensor, generator_state
from test_gpu_configs import check_parameter_gradients, device_inputs, raw_backward

pytestmark = pytest.mark.gpu
EPS = 1e-5


@pytest.mark.parametrize("hidden", [1024, 4096])
def test_more_than_2_31_elements(hidden):
    rows = (1 << 31) // hidden + 3
    print(f"[large] rows={rows} H={hidden} elements={rows * hidden}", flush=True)
    inputs, grads = device_inputs(rows, hidden, torch.float16, seed=31 + hidden)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, 0.1, EPS, True, 128)
    gradients = raw_backward(grads, outputs, inputs[2], 0.1, True)
    torch.cuda.synchronize()
    check_full_tensor(inputs, grads, outputs, gradients, 0.1, EPS, seed, offset,
                      chunk=(1 << 24) // hidden, what=f"2^31+ H={hidden}")
    check_parameter_gradients(outputs[0], grads[1], gradients)
