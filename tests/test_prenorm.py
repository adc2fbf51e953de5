"""The pre-norm integration helpers on the CPU (PyTorch implementation).

With ``implementation="torch"`` the fused steps run the reference's
decomposition, so a stack driven by ``prenorm_forward`` must equal the
unfused stack bit for bit (values and gradients), use each LayerNorm where the
recipe puts it (docs/residual_layer_norm.md:51-83 of the reference), and keep
the model's ``state_dict`` keys.
"""

import pytest
import torch
from torch import nn

from gfx1010_kernels import prenorm_forward, residual_norm
from prenorm_models import Fused, Unfused, randomize


def make_pair(hidden=64, depth=3, seed=0):
    torch.manual_seed(seed)
    unfused = randomize(Unfused(hidden, depth), seed)
    fused = Fused(hidden, depth, implementation="torch")
    fused.load_state_dict(unfused.state_dict())
    return unfused, fused


def test_stack_equals_unfused_bitwise_with_gradients():
    unfused, fused = make_pair()
    x = torch.randn(5, 7, 64)
    outputs = []
    for model in (unfused, fused):
        model.zero_grad()
        leaf = x.clone().requires_grad_(True)
        residual, out = model(leaf)
        (residual.square().mean() + out.sin().sum()).backward()
        grads = [p.grad.clone() for p in model.parameters()]
        outputs.append((residual, out, leaf.grad, grads))
    (r0, o0, g0, p0), (r1, o1, g1, p1) = outputs
    assert torch.equal(r0, r1) and torch.equal(o0, o1) and torch.equal(g0, g1)
    assert all(torch.equal(a, b) for a, b in zip(p0, p1))


def test_state_dict_keys_are_unchanged():
    unfused, fused = make_pair()
    assert list(unfused.state_dict()) == list(fused.state_dict())


def test_each_norm_is_used_where_the_recipe_puts_it():
    """Perturbing one LayerNorm changes the output exactly as in the unfused stack."""
    unfused, fused = make_pair(depth=2)
    x = torch.randn(3, 64)
    for name in ("h.0.ln_1", "h.0.ln_2", "h.1.ln_1", "h.1.ln_2", "ln_f"):
        for model in (unfused, fused):
            with torch.no_grad():
                model.get_submodule(name).bias.add_(0.5)
        assert torch.equal(unfused(x)[1], fused(x)[1]), name


def test_accessor_functions_and_eval_mode():
    unfused, fused = make_pair(depth=2)
    unfused.eval()
    x = torch.randn(4, 64)
    residual, out = prenorm_forward(
        x, list(unfused.h), unfused.ln_f, dropout_p=0.5, training=False,
        attention=lambda block, h: block.attn(h), mlp=lambda block, h: block.mlp(h),
        ln1=lambda block: block.ln_1, ln2=lambda block: block.ln_2, implementation="torch")
    expected = unfused(x)
    assert torch.equal(residual, expected[0]) and torch.equal(out, expected[1])


def test_residual_norm_reads_the_module_parameters():
    norm = randomize(nn.LayerNorm(32, eps=1e-3), 3)
    x, branch = torch.randn(2, 6, 32), torch.randn(2, 6, 32)
    updated, normalized = residual_norm(x, branch, norm, implementation="torch")
    assert torch.equal(updated, x + branch)
    assert torch.equal(normalized, norm(x + branch))


def test_rejections():
    x = torch.randn(2, 32)
    with pytest.raises(TypeError, match="LayerNorm"):
        residual_norm(x, x, nn.Linear(32, 32), implementation="torch")
    with pytest.raises(ValueError, match="hidden size 32"):
        residual_norm(x, x, nn.LayerNorm(16), implementation="torch")
    with pytest.raises(ValueError, match="elementwise affine"):
        residual_norm(x, x, nn.LayerNorm(32, elementwise_affine=False), implementation="torch")
    with pytest.raises(ValueError, match="at least one block"):
        prenorm_forward(x, [], nn.LayerNorm(32))
