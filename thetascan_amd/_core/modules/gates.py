"""Per-head gates (src/thetascan/_core/modules/gates.py:8-40): the data-dependent
EMA decay log(alpha) = -softplus(W x + b) with bias -4, and the SiLU output
gate with bias 1.  Weights start at zero as in the reference."""
from __future__ import annotations

import torch.nn as nn
import torch.nn.functional as F

from ..ops.linear import linear


class _HeadLinear(nn.Module):
    def __init__(self, d_model: int, n_heads: int, out: int, bias_init: float):
        super().__init__()
        self.h, self.o = n_heads, out
        self.lin = nn.Linear(d_model, n_heads * out, bias=True)
        nn.init.zeros_(self.lin.weight)
        nn.init.constant_(self.lin.bias, bias_init)

    def forward(self, x):
        B, T, _ = x.shape
        # split-K weight gradient and HIP bias column sums on the GPU
        return linear(x, self.lin.weight, self.lin.bias).view(B, T, self.h, self.o).transpose(1, 2)


class DecayGate(nn.Module):
    def __init__(self, d_model, n_heads):
        super().__init__()
        self.g = _HeadLinear(d_model, n_heads, 1, bias_init=-4.0)

    def forward(self, x):
        la = -F.softplus(self.g(x))
        return la, la


class OutGate(nn.Module):
    def __init__(self, d_model, n_heads, d):
        super().__init__()
        self.g = _HeadLinear(d_model, n_heads, d, bias_init=1.0)

    def forward(self, x):
        return F.silu(self.g(x))

    def preactivation(self, x):
        """[B,T,H*d] gate logits (the fused read applies the SiLU itself)."""
        return self.g.lin(x)
