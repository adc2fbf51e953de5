"""Small pre-norm transformer stacks shared by the pre-norm helper tests."""

import torch
from torch import nn
from torch.nn import functional as F

from gfx1010_kernels import prenorm_forward


class Block(nn.Module):
    """GPT-2-style pre-norm block; `attn` is a token-mixing stand-in (a
    linear map), `mlp` the usual two-layer MLP without its final dropout."""

    def __init__(self, hidden):
        super().__init__()
        self.ln_1 = nn.LayerNorm(hidden)
        self.attn = nn.Linear(hidden, hidden)
        self.ln_2 = nn.LayerNorm(hidden)
        self.mlp = nn.Sequential(nn.Linear(hidden, 2 * hidden), nn.GELU(),
                                 nn.Linear(2 * hidden, hidden))


class Unfused(nn.Module):
    """The unfused stack: `x = x + drop(sublayer(ln(x)))` per sublayer."""

    def __init__(self, hidden, depth, dropout_p=0.0):
        super().__init__()
        self.h = nn.ModuleList(Block(hidden) for _ in range(depth))
        self.ln_f = nn.LayerNorm(hidden)
        self.dropout_p = dropout_p

    def forward(self, x):
        for block in self.h:
            x = x + F.dropout(block.attn(block.ln_1(x)), self.dropout_p, self.training)
            x = x + F.dropout(block.mlp(block.ln_2(x)), self.dropout_p, self.training)
        return x, self.ln_f(x)


class Fused(Unfused):
    """Same modules (and state_dict keys); forward through prenorm_forward."""

    def __init__(self, hidden, depth, dropout_p=0.0, implementation="auto"):
        super().__init__(hidden, depth, dropout_p)
        self.implementation = implementation

    def forward(self, x):
        return prenorm_forward(x, self.h, self.ln_f, dropout_p=self.dropout_p,
                               training=self.training, implementation=self.implementation)


def randomize(model, seed):
    """Non-trivial LayerNorm parameters, so a mix-up of norms shows."""
    generator = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for module in model.modules():
            if isinstance(module, nn.LayerNorm):
                module.weight.copy_(1 + 0.1 * torch.randn(module.weight.shape, generator=generator))
                module.bias.copy_(0.1 * torch.randn(module.bias.shape, generator=generator))
    return model
