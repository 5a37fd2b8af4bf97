"""Analytic HBM traffic, FLOPs and roofline placement of RBF attention.

The byte and FLOP models restate the reference's
kernels/benchmarks/roofline.py:87-139 (fused_bytes, eager_bytes,
fused_flops, eager_flops), so measured figures are divided by the same
algorithmic work the reference budgets against.  The hardware figures are
MI355X's published ones instead of the H100's.
"""

import dataclasses


@dataclasses.dataclass(frozen=True)
class GpuSpec:
    """Peak figures used for roofline placement."""

    name: str
    compute_units: int
    xcds: int
    lds_bytes_per_cu: int
    l2_bytes_per_xcd: int
    infinity_cache_bytes: int
    hbm_bytes: int
    hbm_bytes_per_s: float
    bf16_mfma_flops: float  # dense, fp32 accumulate
    fp32_mfma_flops: float

    @property
    def ridge_flop_per_byte(self) -> float:
        return self.bf16_mfma_flops / self.hbm_bytes_per_s


MI355X = GpuSpec(
    name='AMD Instinct MI355X (gfx950)',
    compute_units=256,
    xcds=8,
    lds_bytes_per_cu=160 * 1024,
    l2_bytes_per_xcd=4 * 1024 * 1024,
    infinity_cache_bytes=256 * 1024 * 1024,
    hbm_bytes=288 * 10**9,
    hbm_bytes_per_s=8.0e12,
    bf16_mfma_flops=2.5e15,
    fp32_mfma_flops=157.3e12,
)


@dataclasses.dataclass(frozen=True)
class Shape:
    """One attention problem: [B, H, Nq, D] x [B, H, Nk, D] (roofline.py:56-73)."""

    batch: int
    heads: int
    n_q: int
    n_k: int
    head_dim: int
    value_dim: int
    element_bytes: int

    @property
    def planes(self) -> int:
        return self.batch * self.heads


def fused_bytes(s: Shape) -> int:
    """q, k, v, the per-head coefficient and the per-key bias read once; the
    output written once (roofline.py:87-95)."""
    reads = (
        s.planes
        * (s.n_q * s.head_dim + s.n_k * s.head_dim + s.n_k * s.value_dim)
        * s.element_bytes
    )
    reads += s.heads * 4 + s.batch * s.n_k * s.element_bytes
    return reads + s.planes * s.n_q * s.value_dim * s.element_bytes


def eager_bytes(s: Shape) -> dict[str, int]:
    """Per-operator HBM traffic of the eager chain (roofline.py:98-117)."""
    e = s.element_bytes
    q = s.planes * s.n_q * s.head_dim * e
    k = s.planes * s.n_k * s.head_dim * e
    v = s.planes * s.n_k * s.value_dim * e
    diff = s.planes * s.n_q * s.n_k * s.head_dim * e
    scores = s.planes * s.n_q * s.n_k * e
    bias = s.batch * s.n_k * e
    out = s.planes * s.n_q * s.value_dim * e
    return {
        'sub': q + k + diff,
        'pow': 2 * diff,
        'sum': diff + scores,
        'neg': 2 * scores,
        'scale': 2 * scores,
        'bias': 2 * scores + bias,
        'softmax': 2 * scores,
        'bmm': scores + v + out,
    }


def fused_flops(s: Shape) -> int:
    """QK^T and PV products, norms and the online softmax (roofline.py:120-128)."""
    per_plane = (
        2 * s.n_q * s.n_k * s.head_dim
        + 2 * s.n_q * s.n_k * s.value_dim
        + 2 * (s.n_q + s.n_k) * s.head_dim
        + 6 * s.n_q * s.n_k
    )
    return s.planes * per_plane


def eager_flops(s: Shape) -> int:
    """Difference, square and reduction, then softmax and PV (roofline.py:131-139)."""
    per_plane = (
        3 * s.n_q * s.n_k * s.head_dim
        + 3 * s.n_q * s.n_k
        + 5 * s.n_q * s.n_k
        + 2 * s.n_q * s.n_k * s.value_dim
    )
    return s.planes * per_plane


def matrix_flops(s: Shape) -> int:
    """The two products only (what MFMA executes): 2 Nq Nk (D + Dv) per plane."""
    return s.planes * 2 * s.n_q * s.n_k * (s.head_dim + s.value_dim)


def analyze(s: Shape, spec: GpuSpec = MI355X) -> dict:
    """Budgets and roofline placement of both formulations at `s`."""
    eager = eager_bytes(s)
    eager_total = sum(eager.values())
    fused = fused_bytes(s)
    fused_ai = fused_flops(s) / fused
    return {
        'shape': dataclasses.asdict(s),
        'eager_bytes': eager_total,
        'eager_bytes_by_op': eager,
        'fused_bytes': fused,
        'bytes_ratio': fused / eager_total,
        'eager_intensity_flop_per_byte': eager_flops(s) / eager_total,
        'fused_intensity_flop_per_byte': fused_ai,
        'ridge_flop_per_byte': spec.ridge_flop_per_byte,
        'fused_is_memory_bound': fused_ai < spec.ridge_flop_per_byte,
        'fused_hbm_floor_us': fused / spec.hbm_bytes_per_s * 1e6,
        'matrix_flops': matrix_flops(s),
        'fused_mfma_floor_us': matrix_flops(s) / spec.bf16_mfma_flops * 1e6,
        'fused_working_set_fits_infinity_cache': fused < spec.infinity_cache_bytes,
    }
