"""The pre-norm integration helpers on the native MI355X path.

A stack driven by ``prenorm_forward`` (every residual add fused into the
LayerNorm after it) against the unfused PyTorch stack with the same weights:
outputs and all gradients agree to fp32 rounding at p = 0, eval mode equals
p = 0, dropout replays bit for bit from the same RNG state, and bf16
sublayers get bf16 normalized inputs.
"""

import warnings

import pytest
import torch

from parity import assert_normwise, host
from prenorm_models import Fused, Unfused, randomize

pytestmark = pytest.mark.gpu

# Tolerance for a 3-block stack: the native LayerNorm and torch's differ in
# fp32 rounding (~1e-7 relative), amplified a little by the sublayers.
TOL_STACK = 1e-4


def make_pair(hidden, depth=3, dropout_p=0.0, seed=0):
    torch.manual_seed(seed)
    unfused = randomize(Unfused(hidden, depth, dropout_p), seed).cuda()
    fused = Fused(hidden, depth, dropout_p, implementation="gfx950").cuda()
    fused.load_state_dict(unfused.state_dict())
    return unfused, fused


def run(model, x):
    model.zero_grad()
    leaf = x.clone().requires_grad_(True)
    residual, out = model(leaf)
    (residual.square().mean() + out.sin().sum()).backward()
    return residual, out, leaf.grad, [p.grad for p in model.parameters()]


@pytest.mark.parametrize("hidden", [768, 1600])
def test_native_stack_matches_unfused(hidden):
    unfused, fused = make_pair(hidden)
    x = torch.randn(4, 33, hidden, device="cuda")
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        got = run(fused, x)
    expected = run(unfused, x)
    for name, a, b in zip(("residual", "out", "grad_x"), got[:3], expected[:3]):
        assert_normwise(host(a), host(b), TOL_STACK, name)
    for (name, _), a, b in zip(fused.named_parameters(), got[3], expected[3]):
        assert_normwise(host(a), host(b), TOL_STACK, name)


def test_eval_equals_p0_and_dropout_replays():
    unfused, fused = make_pair(768, dropout_p=0.1)
    x = torch.randn(2, 64, 768, device="cuda")
    fused.eval()
    with torch.no_grad():
        eval_out = fused(x)
        fused.dropout_p = 0.0
        fused.train()
        p0_out = fused(x)
    assert torch.equal(eval_out[0], p0_out[0]) and torch.equal(eval_out[1], p0_out[1])

    fused.dropout_p = 0.1
    state = torch.cuda.get_rng_state()
    first = run(fused, x)
    torch.cuda.set_rng_state(state)
    second = run(fused, x)
    for a, b in zip(first[:3], second[:3]):
        assert torch.equal(a, b)
    assert not torch.equal(first[0], p0_out[0])


def test_bfloat16_sublayers_get_bfloat16_inputs():
    from gfx1010_kernels import prenorm_forward

    unfused, _ = make_pair(512, depth=2)
    reference = unfused(torch.zeros(1, 512, device="cuda"))  # warm the modules
    del reference
    blocks = [block.to(torch.bfloat16) for block in unfused.h]
    for block in blocks:
        block.ln_1.float()
        block.ln_2.float()
    seen = []

    def attention(block, h):
        seen.append(h.dtype)
        return block.attn(h)

    x = torch.randn(3, 40, 512, device="cuda")
    residual, out = prenorm_forward(x, blocks, unfused.ln_f, attention=attention,
                                    implementation="gfx950", normalized_dtype=torch.bfloat16)
    assert seen == [torch.bfloat16, torch.bfloat16]
    assert residual.dtype == torch.float32 and out.dtype == torch.bfloat16
    assert torch.isfinite(out.float()).all()
