"""The price Transformer.

The subject property and its K comparables become K + 1 tokens; pre-norm
Transformer blocks with spatial (RBF) attention mix them, and the subject
token is read out as a correction to the comparables' mean log price.  Same
architecture and forward semantics as the reference's
models/price_transformer/model.py:39-282; trimming comparables to the search
radius (with a nearest-neighbour fallback) is branch-free tensor code, so
TorchDynamo captures the forward pass as a single graph, every attention
site stays visible to the rewrite, and a forward pass never waits for the
GPU.
"""

import dataclasses
import math
import typing
from collections.abc import Mapping

import torch
from torch import nn

from vectra_amd.price_transformer import candidate_encoder
from vectra_amd.price_transformer import microhood
from vectra_amd.price_transformer import spatial_attention


@dataclasses.dataclass(frozen=True)
class ModelConfig:
    embedding_dim: int = 128
    attribute_dim: int = 5
    d_model: int = 128
    num_heads: int = 4
    num_layers: int = 2
    ffn_dim: int = 256
    num_candidates: int = 64
    min_candidates: int = 4  # kept when no comparable lies inside the radius

    @classmethod
    def from_dict(cls, values: Mapping[str, typing.Any]) -> 'ModelConfig':
        names = {f.name for f in dataclasses.fields(cls)}
        return cls(**{k: v for k, v in values.items() if k in names})


class PricingInputs(typing.NamedTuple):
    """One batch of requests, in forward-argument order."""

    query_embedding: torch.Tensor  # [B, E]
    query_attributes: torch.Tensor  # [B, A]
    query_location: torch.Tensor  # [B, 2] lat, lon degrees
    query_cell6: torch.Tensor  # [B] int64
    valuation_day: torch.Tensor  # [B] days since epoch
    radius_km: torch.Tensor  # [B]
    cand_embedding: torch.Tensor  # [B, K, E]
    cand_attributes: torch.Tensor  # [B, K, A]
    cand_log_price: torch.Tensor  # [B, K]
    cand_sale_day: torch.Tensor  # [B, K]
    cand_location: torch.Tensor  # [B, K, 2]
    cand_cell6: torch.Tensor  # [B, K] int64
    cand_valid: torch.Tensor  # [B, K] bool

    def to(self, device) -> 'PricingInputs':
        return PricingInputs(*(t.to(device) for t in self))  # pylint: disable=not-an-iterable


def trim_to_radius(distance_km, radius_km, valid, min_keep: int) -> torch.Tensor:
    """Comparables inside the radius; rows with none keep their `min_keep` nearest.

    The reference (models/price_transformer/model.py:96-138) picks between an
    inside-only branch and this nearest-neighbour fallback with a torch.cond
    on "every row has a comparable inside".  Both give the same mask on every
    row the inside-only branch covers, so here the fallback is always taken
    and selected per row: the same mask with no data-dependent branch.  The
    cond's predicate is a device-to-host read on every forward pass, which
    stalls the host until the GPU has caught up, so the model could not be
    launched ahead of the GPU, overlapped with the next batch's copy, or
    captured in a HIP graph.
    """
    inside = valid & (distance_km <= radius_km.unsqueeze(-1))
    nearest = distance_km.masked_fill(~valid, float('inf')).topk(min_keep, dim=-1, largest=False).indices
    fallback = torch.zeros_like(valid).scatter(-1, nearest, True) & valid
    return torch.where(inside.any(-1, keepdim=True), inside, fallback)


class Block(nn.Module):
    """Pre-norm Transformer block with spatial attention."""

    def __init__(self, config: ModelConfig):
        super().__init__()
        self.norm1 = nn.LayerNorm(config.d_model)
        self.attention = spatial_attention.SpatialAttention(config.d_model, config.num_heads)
        self.norm2 = nn.LayerNorm(config.d_model)
        self.ffn = nn.Sequential(
            nn.Linear(config.d_model, config.ffn_dim),
            nn.GELU(),
            nn.Linear(config.ffn_dim, config.d_model),
        )

    def forward(self, x, key_bias):
        x = x + self.attention(self.norm1(x), key_bias)
        return x + self.ffn(self.norm2(x))


class PriceTransformer(nn.Module):
    def __init__(self, config: ModelConfig):
        super().__init__()
        self.config = config
        self.query_encoder = candidate_encoder.QueryEncoder(
            config.embedding_dim, config.attribute_dim, config.d_model
        )
        self.candidate_encoder = candidate_encoder.CandidateEncoder(
            config.embedding_dim, config.attribute_dim, config.d_model
        )
        self.blocks = nn.ModuleList([Block(config) for _ in range(config.num_layers)])
        self.norm = nn.LayerNorm(config.d_model)
        self.head = nn.Linear(config.d_model, 1)
        self._block_dtype = torch.float32

    def set_block_dtype(self, dtype: torch.dtype) -> 'PriceTransformer':
        """Runs the Transformer blocks in `dtype`; encoders, geometry and the
        read-out stay fp32 (coordinates in half precision would lose km)."""
        self.blocks.to(dtype)
        self._block_dtype = dtype
        return self

    def forward(self, query_embedding, query_attributes, query_location, query_cell6,
                valuation_day, radius_km, cand_embedding, cand_attributes, cand_log_price,
                cand_sale_day, cand_location, cand_cell6, cand_valid) -> torch.Tensor:
        """Predicted natural-log prices [B]."""
        distance = microhood.haversine_km(query_location, cand_location)
        valid = trim_to_radius(
            distance, radius_km, cand_valid, min(self.config.min_candidates, cand_valid.shape[-1])
        )
        candidates = self.candidate_encoder(
            cand_embedding,
            cand_attributes,
            cand_log_price,
            valuation_day.unsqueeze(-1) - cand_sale_day,
            microhood.relative_offsets_km(query_location, cand_location),
            distance,
            radius_km,
            microhood.same_cell_flags(query_cell6, cand_cell6),
        )
        query = self.query_encoder(query_embedding, query_attributes)
        tokens = torch.cat([query.unsqueeze(1), candidates], dim=1).to(self._block_dtype)
        token_valid = torch.cat([torch.ones_like(valid[:, :1]), valid], dim=1)
        key_bias = torch.zeros_like(token_valid, dtype=tokens.dtype).masked_fill(
            ~token_valid, float('-inf')
        )[:, None, None, :]
        for block in self.blocks:
            tokens = block(tokens, key_bias)
        weights = valid.to(cand_log_price.dtype)
        baseline = (cand_log_price * weights).sum(-1) / weights.sum(-1).clamp_min(1.0)
        readout = self.head(self.norm(tokens[:, 0].float()))
        return baseline + readout.squeeze(-1)


def example_inputs(config: ModelConfig, batch_size: int, device='cpu', seed: int = 0) -> PricingInputs:
    """Random inputs of the serving shape around one city (reference model.py:247-282):
    comparables within ~2 km of the subject, the last K/8 of them padding."""
    gen = torch.Generator().manual_seed(seed)
    k = config.num_candidates

    def randn(*shape):
        return torch.randn(*shape, generator=gen)

    center = torch.tensor([37.7749, -122.4194])
    query_location = center + 0.02 * randn(batch_size, 2)
    cand_location = query_location[:, None, :] + 0.02 * randn(batch_size, k, 2)
    cells = torch.randint(0, 1 << 30, (batch_size,), generator=gen)
    valid = torch.ones(batch_size, k, dtype=torch.bool)
    valid[:, k - k // 8 :] = False
    return PricingInputs(
        query_embedding=torch.tanh(randn(batch_size, config.embedding_dim)),
        query_attributes=randn(batch_size, config.attribute_dim),
        query_location=query_location,
        query_cell6=cells,
        valuation_day=torch.full((batch_size,), 20000.0),
        radius_km=torch.full((batch_size,), 5.0),
        cand_embedding=torch.tanh(randn(batch_size, k, config.embedding_dim)),
        cand_attributes=randn(batch_size, k, config.attribute_dim),
        cand_log_price=13.0 + 0.5 * randn(batch_size, k),
        cand_sale_day=20000.0 - 900.0 * randn(batch_size, k).abs(),
        cand_location=cand_location,
        cand_cell6=cells[:, None] + torch.randint(0, 3, (batch_size, k), generator=gen),
        cand_valid=valid,
    ).to(device)


def box_inputs(config: ModelConfig, batch_size: int, device='cpu', seed: int = 0,
               box_km: float = 50.0, max_age_days: float = 730.0) -> PricingInputs:
    """Inputs of the full-model benchmark configuration: attributes ~ N(0, 1),
    subjects and comparables uniform over a `box_km` square, sale dates
    uniform over the `max_age_days` before valuation, embeddings tanh(N(0,1)),
    every comparable valid and a radius covering the box."""
    gen = torch.Generator().manual_seed(seed)
    k = config.num_candidates
    south_west = torch.tensor([37.55, -122.55])
    deg_lat = box_km / (microhood.EARTH_RADIUS_KM * math.pi / 180.0)
    deg_lon = deg_lat / math.cos(math.radians(float(south_west[0]) + deg_lat / 2))
    span = torch.tensor([deg_lat, deg_lon])

    def uniform(*shape):
        return torch.rand(*shape, generator=gen)

    query_location = south_west + span * uniform(batch_size, 2)
    cand_location = south_west + span * uniform(batch_size, k, 2)
    cells = torch.randint(0, 1 << 30, (batch_size,), generator=gen)
    valuation = torch.full((batch_size,), 20000.0)
    return PricingInputs(
        query_embedding=torch.tanh(torch.randn(batch_size, config.embedding_dim, generator=gen)),
        query_attributes=torch.randn(batch_size, config.attribute_dim, generator=gen),
        query_location=query_location,
        query_cell6=cells,
        valuation_day=valuation,
        radius_km=torch.full((batch_size,), box_km * math.sqrt(2.0)),
        cand_embedding=torch.tanh(torch.randn(batch_size, k, config.embedding_dim, generator=gen)),
        cand_attributes=torch.randn(batch_size, k, config.attribute_dim, generator=gen),
        cand_log_price=13.0 + 0.5 * torch.randn(batch_size, k, generator=gen),
        cand_sale_day=valuation[:, None] - max_age_days * uniform(batch_size, k),
        cand_location=cand_location,
        cand_cell6=cells[:, None] + torch.randint(0, 3, (batch_size, k), generator=gen),
        cand_valid=torch.ones(batch_size, k, dtype=torch.bool),
    ).to(device)
