"""Geometry and micro-neighbourhood features of query/comparable pairs.

Same features as the reference's models/price_transformer/microhood.py:
great-circle distance (haversine), local east/north offsets, and flags for
comparables sharing the subject's 6-, 5- and 4-character GeoHash cell.  All
branch-free tensor arithmetic, so the forward pass captures as one graph.
"""

import math

import torch

EARTH_RADIUS_KM = 6371.0088
_RAD = math.pi / 180.0


def haversine_km(query_location: torch.Tensor, candidate_location: torch.Tensor) -> torch.Tensor:
    """[B, 2] and [B, K, 2] (lat, lon degrees) -> [B, K] km."""
    lat_q = query_location[:, None, 0] * _RAD
    lon_q = query_location[:, None, 1] * _RAD
    lat_c = candidate_location[..., 0] * _RAD
    lon_c = candidate_location[..., 1] * _RAD
    a = torch.sin((lat_c - lat_q) / 2) ** 2 + torch.cos(lat_q) * torch.cos(lat_c) * torch.sin(
        (lon_c - lon_q) / 2
    ) ** 2
    return 2.0 * EARTH_RADIUS_KM * torch.asin(torch.sqrt(a.clamp(0.0, 1.0)))


def relative_offsets_km(query_location: torch.Tensor, candidate_location: torch.Tensor) -> torch.Tensor:
    """East and north offsets [B, K, 2] km (local equirectangular projection)."""
    km_per_degree = EARTH_RADIUS_KM * _RAD
    delta = candidate_location - query_location[:, None, :]
    east = delta[..., 1] * km_per_degree * torch.cos(query_location[:, None, 0] * _RAD)
    north = delta[..., 0] * km_per_degree
    return torch.stack([east, north], dim=-1)


def same_cell_flags(query_cell6: torch.Tensor, candidate_cell6: torch.Tensor) -> torch.Tensor:
    """[B] and [B, K] integer cells -> [B, K, 3] float flags (6-, 5-, 4-char match)."""
    q = query_cell6[:, None]
    flags = [
        (torch.bitwise_right_shift(candidate_cell6, bits) == torch.bitwise_right_shift(q, bits))
        for bits in (0, 5, 10)
    ]
    return torch.stack(flags, dim=-1).to(torch.float32)
