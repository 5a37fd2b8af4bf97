"""Multi-head RBF (spatial) attention: the eager site the backend rewrites.

  weights = softmax_j(-||q_i - k_j||^2 / (2 sigma_h^2) + key_bias_j)

with a learned bandwidth per head, written as the plain eager chain on
purpose (reference: models/price_transformer/spatial_attention.py:68-88) so
that torch.compile(backend='vectra') finds it and substitutes
torch.ops.vectra.rbf_attention.
"""

import math

import torch
from torch import nn


class SpatialAttention(nn.Module):
    def __init__(self, d_model: int, num_heads: int):
        super().__init__()
        if d_model % num_heads:
            raise ValueError(f'd_model {d_model} not divisible by num_heads {num_heads}')
        self.num_heads = num_heads
        self.head_dim = d_model // num_heads
        self.qkv = nn.Linear(d_model, 3 * d_model)
        self.out = nn.Linear(d_model, d_model)
        # sigma^2 starts at the head width, near the typical squared distance.
        self.log_sigma = nn.Parameter(
            torch.full((1, num_heads, 1, 1), 0.5 * math.log(self.head_dim))
        )

    def forward(self, x: torch.Tensor, key_bias: torch.Tensor) -> torch.Tensor:
        """x [B, N, d_model], key_bias [B, 1, 1, N] (0 or -inf) -> [B, N, d_model]."""
        batch, tokens, width = x.shape
        q, k, v = (
            t.view(batch, tokens, self.num_heads, self.head_dim).transpose(1, 2)
            for t in self.qkv(x).split(width, dim=-1)
        )
        sq_dist = (q.unsqueeze(-2) - k.unsqueeze(-3)).pow(2).sum(-1)
        logits = -sq_dist / (2 * self.log_sigma.exp() ** 2) + key_bias
        mixed = torch.softmax(logits, dim=-1) @ v
        return self.out(mixed.transpose(1, 2).reshape(batch, tokens, width))
