"""Helpers for the compiler suites: compile a function, count rewrites."""

import torch

from vectra_amd.compiler import backend


def compile_and_run(fn, *inputs):
    """Compiles `fn` with the vectra backend and runs it once.

    Returns (output, backend.CompileReport).
    """
    torch._dynamo.reset()  # pylint: disable=protected-access
    report = backend.CompileReport()
    compiled = torch.compile(fn, backend=backend.make_backend(report), fullgraph=True, dynamic=False)
    with torch.no_grad():
        out = compiled(*inputs)
    return out, report


def attention_inputs(batch=2, heads=3, n_q=6, n_k=9, dim=8, dim_v=None, dtype=torch.float32,
                     seed=0, device='cpu'):
    """Random q [B,H,Nq,D], k [B,H,Nk,D], v [B,H,Nk,Dv] and a per-head sigma."""
    gen = torch.Generator().manual_seed(seed)
    dim_v = dim if dim_v is None else dim_v
    q = torch.randn(batch, heads, n_q, dim, generator=gen)
    k = torch.randn(batch, heads, n_k, dim, generator=gen)
    v = torch.randn(batch, heads, n_k, dim_v, generator=gen)
    sigma = torch.rand(1, heads, 1, 1, generator=gen) + 1.0
    return tuple(t.to(device=device, dtype=dtype) for t in (q, k, v, sigma))
