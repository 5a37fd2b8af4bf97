"""Shared pieces of the compiler tests.

* `operands`: seeded q, k, v and a per-head bandwidth sigma.
* `run_vectra`: compiles a callable with the `vectra` backend (one graph, no
  dynamic shapes), runs it once without autograd, and returns the output
  and the CompileReport counting the rewritten sites.
* Parts of an RBF-attention spelling (a squared distance, a logit, a
  normaliser), so the tests can compose many spellings of one computation.
"""

import dataclasses

import torch

from vectra_amd.compiler import backend

F = torch.nn.functional


@dataclasses.dataclass
class Operands:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    sigma: torch.Tensor

    def __iter__(self):
        return iter((self.q, self.k, self.v, self.sigma))


def operands(batch=2, heads=3, n_q=6, n_k=9, dim=8, dim_v=None, dtype=torch.float32, seed=0) -> Operands:
    gen = torch.Generator().manual_seed(seed)

    def normal(*shape):
        return torch.randn(*shape, generator=gen).to(dtype)

    q = normal(batch, heads, n_q, dim)
    k = normal(batch, heads, n_k, dim)
    v = normal(batch, heads, n_k, dim if dim_v is None else dim_v)
    sigma = (1.0 + torch.rand(1, heads, 1, 1, generator=gen)).to(dtype)
    return Operands(q, k, v, sigma)


def run_vectra(fn, *args):
    torch._dynamo.reset()  # pylint: disable=protected-access
    report = backend.CompileReport()
    compiled = torch.compile(fn, backend=backend.make_backend(report), fullgraph=True, dynamic=False)
    with torch.no_grad():
        return compiled(*args), report


# ------------------------------------------------ parts of a spelling

def distance_broadcast_pow(q, k):
    return (q.unsqueeze(-2) - k.unsqueeze(-3)).pow(2).sum(-1)


def distance_indexed_self_product(q, k):
    gap = q[:, :, :, None, :] - k[:, :, None, :, :]
    return (gap * gap).sum(dim=4)


def distance_functional_square(q, k):
    return torch.sum(torch.square(torch.sub(torch.unsqueeze(q, 3), torch.unsqueeze(k, 2))), dim=-1)


def logit_over_two_sigma_squared(sq, sigma):
    return -sq / (2 * sigma**2)


def logit_times_negative_reciprocal(sq, sigma):
    return torch.mul(sq, -torch.reciprocal(2.0 * sigma * sigma))


def logit_negated_product(sq, sigma):
    return -(sq * (0.5 / sigma**2))


def logit_fixed_temperature(sq, sigma):
    del sigma
    return sq * -0.125


def normalise_softmax(x):
    return torch.softmax(x, dim=-1)


def normalise_functional(x):
    return F.softmax(x, -1)


def normalise_exp_over_sum(x):
    e = torch.exp(x)
    return e / e.sum(dim=-1, keepdim=True)


def spelling(distance, logit, normalise):
    """q, k, v, sigma -> normalise(logit(distance(q, k), sigma)) @ v."""

    def attention(q, k, v, sigma):
        return normalise(logit(distance(q, k), sigma)) @ v

    attention.__name__ = f'{distance.__name__}+{logit.__name__}+{normalise.__name__}'
    return attention
