"""The benchmark configurations and their seeded synthetic inputs.

Each configuration is one of the operator workloads the headline metric and
the parity gates are quoted on.  Inputs are drawn on the CPU from
``torch.Generator().manual_seed(seed)`` in the order q, k, v, gamma, valid
counts, as fp32 ``randn`` then cast and moved, as the reference's parity
tests draw theirs (kernels/tests/test_parity.py:49-61).  A valid count c_b
masks keys j >= c_b of batch b with a -inf key bias.

A configuration with `fused_qkv` draws one [B, N, 3 H D] tensor instead, and
q, k and v are head-transposed views of its three thirds, [B, N, H, D] ->
[B, H, N, D] (rows of D elements, 3 H D apart): the layout the price
model's attention sites hand the operator, a slice of one qkv projection
(models/price_transformer/spatial_attention.py:80-87 of the reference).
"""

import dataclasses

import torch

from vectra_amd.benchmarks import roofline


@dataclasses.dataclass(frozen=True)
class Config:
    """One operator workload."""

    name: str
    batch: int
    heads: int
    n_q: int
    n_k: int
    head_dim: int
    dtype: torch.dtype
    # gamma: a constant, or per head uniform in [lo, hi].
    gamma: float | tuple[float, float]
    # Valid key counts uniform in [lo, hi] (inclusive), or None for no mask.
    valid: tuple[int, int] | None
    qk_std: float = 1.0
    bias_dtype: torch.dtype | None = None  # default: the input dtype
    fused_qkv: bool = False  # q, k, v as head-transposed views of one projection

    @property
    def value_dim(self) -> int:
        return self.head_dim

    def shape(self) -> roofline.Shape:
        return roofline.Shape(
            self.batch,
            self.heads,
            self.n_q,
            self.n_k,
            self.head_dim,
            self.value_dim,
            torch.empty((), dtype=self.dtype).element_size(),
        )

    def with_dtype(self, dtype: torch.dtype) -> 'Config':
        return dataclasses.replace(self, dtype=dtype, name=f'{self.name}_{_short(dtype)}')


def _short(dtype: torch.dtype) -> str:
    return {torch.float32: 'fp32', torch.float16: 'fp16', torch.bfloat16: 'bf16'}[dtype]


CPU_EAGER = Config('cpu_eager', 64, 4, 1, 32, 16, torch.float32, 0.5 / 16, (4, 32))
SERVING = Config('serving', 1024, 8, 1, 64, 32, torch.bfloat16, (0.01, 0.1), (8, 64))
SELF_ATTENTION = Config('self_attention', 1024, 8, 65, 65, 32, torch.bfloat16, 1.0 / 32, (16, 65))
LONG_KEY = Config('long_key', 16, 16, 4096, 4096, 64, torch.bfloat16, (0.005, 0.05), None, qk_std=0.5)
# The reference's bandwidth-proof workload (kernels/benchmarks/bandwidth.py:44-57,
# throughput.py:97-111): fp16, gamma = 1/(2D) in every head, the last 8 keys padded.
BANDWIDTH = Config('bandwidth', 1024, 4, 65, 65, 32, torch.float16, (1.0 / 64, 1.0 / 64), (57, 57))
# One attention site of the config-5 price model (d_model 128, 8 heads of 16
# dims, 1024 subjects x (1 + 64 comparables)) with fp16 blocks: q, k, v as
# views of the qkv projection; gamma = 1 / (2 sigma^2) at the model's initial
# sigma^2 = 16 (the head width); the subject and 8-64 comparables valid.
MODEL_SITE = Config('model_site', 1024, 8, 65, 65, 16, torch.float16, 1.0 / 32, (9, 65), fused_qkv=True)

CONFIGS = {c.name: c for c in (CPU_EAGER, SERVING, SELF_ATTENTION, LONG_KEY, BANDWIDTH, MODEL_SITE)}


@dataclasses.dataclass
class Inputs:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    scale: torch.Tensor
    key_bias: torch.Tensor | None
    counts: torch.Tensor | None

    def args(self):
        return self.q, self.k, self.v, self.scale, self.key_bias

    def to(self, device) -> 'Inputs':
        def move(t):
            return None if t is None else t.to(device)

        base = self.q._base  # pylint: disable=protected-access
        shared = base is not None and all(t._base is base for t in (self.k, self.v))  # pylint: disable=protected-access
        if shared and base.is_contiguous():
            # Views of one projection: move it once and view it the same way
            # there (moving each view alone would make it contiguous).
            moved = base.to(device)
            q, k, v = (moved.as_strided(t.shape, t.stride(), t.storage_offset() - base.storage_offset())
                       for t in (self.q, self.k, self.v))
            return Inputs(q, k, v, move(self.scale), move(self.key_bias), move(self.counts))
        return Inputs(*(move(getattr(self, f.name)) for f in dataclasses.fields(self)))

    def nbytes(self) -> int:
        return sum(
            t.numel() * t.element_size()
            for t in (self.q, self.k, self.v, self.scale, self.key_bias)
            if t is not None
        )


def make_inputs(config: Config, seed: int = 0, device='cpu', batch: int | None = None) -> Inputs:
    """Seeded inputs of `config` (optionally only its first `batch` batches)."""
    gen = torch.Generator().manual_seed(seed)
    b = config.batch if batch is None else batch
    h, d = config.heads, config.head_dim

    def randn(*size, std=1.0):
        x = torch.randn(*size, generator=gen)
        return (x * std if std != 1.0 else x).to(config.dtype)

    if config.fused_qkv:
        if config.n_q != config.n_k or config.value_dim != d or config.qk_std != 1.0:
            raise ValueError('a fused projection has one token axis, one head width and unit values')
        qkv = randn(b, config.n_q, 3 * h * d)
        q, k, v = (t.view(b, config.n_q, h, d).transpose(1, 2) for t in qkv.split(h * d, dim=-1))
    else:
        q = randn(b, h, config.n_q, d, std=config.qk_std)
        k = randn(b, h, config.n_k, d, std=config.qk_std)
        v = randn(b, h, config.n_k, config.value_dim)
    if isinstance(config.gamma, tuple):
        lo, hi = config.gamma
        scale = lo + (hi - lo) * torch.rand(1, h, 1, 1, generator=gen)
    else:
        scale = torch.tensor(config.gamma, dtype=torch.float32)
    key_bias = counts = None
    if config.valid is not None:
        lo, hi = config.valid
        counts = torch.randint(lo, hi + 1, (b,), generator=gen)
        keys = torch.arange(config.n_k)
        bias = torch.zeros(b, 1, 1, config.n_k)
        bias[(keys[None, :] >= counts[:, None])[:, None, None, :]] = float('-inf')
        key_bias = bias.to(config.bias_dtype or config.dtype)
    return Inputs(q, k, v, scale, key_bias, counts).to(device)
