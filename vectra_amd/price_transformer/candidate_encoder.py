"""Token encoders for the subject property and its comparables.

Same inputs and widths as the reference's
models/price_transformer/candidate_encoder.py: a two-layer GELU MLP over the
embedding and attributes (plus, for comparables, normalised log price, years
since sale, radius-scaled offsets and distance, and the cell flags).
"""

import torch
from torch import nn

LOG_PRICE_CENTER = 13.12  # log of $500,000
LOG_PRICE_SCALE = 0.6
DAYS_PER_YEAR = 365.25
_EXTRA_FEATURES = 1 + 1 + 3 + 3  # price, age, geometry (east, north, distance), cell flags


def _mlp(n_in: int, hidden: int, n_out: int) -> nn.Sequential:
    return nn.Sequential(nn.Linear(n_in, hidden), nn.GELU(), nn.Linear(hidden, n_out))


class QueryEncoder(nn.Module):
    """[B, E], [B, A] -> [B, d_model]."""

    def __init__(self, embedding_dim: int, attribute_dim: int, d_model: int):
        super().__init__()
        self.mlp = _mlp(embedding_dim + attribute_dim, 2 * d_model, d_model)
        self.role = nn.Parameter(torch.zeros(d_model))

    def forward(self, embedding, attributes):
        return self.mlp(torch.cat([embedding, attributes], dim=-1)) + self.role


class CandidateEncoder(nn.Module):
    """[B, K, ...] comparable features -> [B, K, d_model]."""

    def __init__(self, embedding_dim: int, attribute_dim: int, d_model: int):
        super().__init__()
        self.mlp = _mlp(embedding_dim + attribute_dim + _EXTRA_FEATURES, 2 * d_model, d_model)

    def forward(self, embedding, attributes, log_price, sale_age_days, offsets_km, distance_km,
                radius_km, cell_flags):
        radius = radius_km[:, None, None]
        features = torch.cat(
            [
                embedding,
                attributes,
                ((log_price - LOG_PRICE_CENTER) / LOG_PRICE_SCALE).unsqueeze(-1),
                (sale_age_days / DAYS_PER_YEAR).unsqueeze(-1),
                offsets_km / radius,
                distance_km.unsqueeze(-1) / radius,
                cell_flags,
            ],
            dim=-1,
        )
        return self.mlp(features)
