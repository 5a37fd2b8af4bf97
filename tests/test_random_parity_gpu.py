"""Seeded random parity cases over shapes, layouts, dtypes, scales, masks and
every kernel variant the library accepts, and over the engine's top-k search
(GPU, through the C ABI).

The RBF cases stay in the regime the gates are stated for (q, k ~ N(0, s^2)
with s <= 1, values ~ N(0, t^2) with t <= 4, gamma <= 0.11, head dims up to
80; for fp32 inputs gamma D s^2 <= 1.5, as at config 3): each output is
held to the gate of its input dtype around the float64 value on the same
rounded inputs, with the absolute term scaled by the
values' spread (the operator is linear in v) and widened by four times the
eager fp32 chain's own error there (the expansion |q|^2 + |k|^2 - 2 q.k that
every matrix-core formulation uses, the reference's Triton kernel included,
carries two to three times the direct chain's rounding).  Top-k results must
equal the oracle's bit for bit in every entry point's form.
"""

import numpy as np
import pytest
import torch

from oracle import rbf as oracle
from oracle import scan as scan_oracle
from vectra_amd.index import scan
from vectra_amd.kernels import capi
from vectra_amd.kernels import custom_ops  # noqa: F401  (registers the op)

pytestmark = pytest.mark.gpu

GATES = {torch.float32: (1e-5, 1e-6), torch.bfloat16: (1e-3, 1e-4), torch.float16: (1e-3, 1e-4)}
SIZES = [1, 2, 3, 5, 16, 17, 31, 33, 64, 65, 80, 81, 127, 129, 200]


def _case(seed):
    rng = np.random.default_rng(seed)
    g = torch.Generator().manual_seed(seed)
    dtype = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(3))]
    B, H = int(rng.integers(1, 4)), int(rng.integers(1, 5))
    nq, nk = int(rng.choice(SIZES)), int(rng.choice(SIZES))
    if rng.random() < 0.1:
        B, H, nq, nk = 1, 2, int(rng.choice([16, 65])), int(rng.choice([1024, 1100]))
    D = int(rng.choice([16, 32, 64, 8, 24, 48, 80]))
    Dv = D if rng.random() < 0.8 else int(rng.choice([8, 16, 32, 40]))
    s, t = float(rng.choice([0.5, 1.0])), float(rng.choice([1.0, 4.0]))
    layout = ['contiguous', 'transposed', 'fused'][int(rng.integers(3))]
    if layout == 'fused' and nq == nk and D == Dv:
        proj = torch.cat([torch.randn(B, nq, H * D, generator=g) * s, torch.randn(B, nq, H * D, generator=g) * s,
                          torch.randn(B, nq, H * D, generator=g) * t], -1).to(dtype)
        q, k, v = (x.view(B, nq, H, D).transpose(1, 2) for x in proj.split(H * D, dim=-1))
    elif layout == 'transposed':
        q = (torch.randn(B, nq, H, D, generator=g) * s).to(dtype).transpose(1, 2)
        k = (torch.randn(B, nk, H, D, generator=g) * s).to(dtype).transpose(1, 2)
        v = (torch.randn(B, nk, H, Dv, generator=g) * t).to(dtype).transpose(1, 2)
    else:
        q = (torch.randn(B, H, nq, D, generator=g) * s).to(dtype)
        k = (torch.randn(B, H, nk, D, generator=g) * s).to(dtype)
        v = (torch.randn(B, H, nk, Dv, generator=g) * t).to(dtype)
    form = int(rng.integers(3))
    base = 0.01 + 0.1 * torch.rand((1,) if form == 0 else ((1, H, 1, 1) if form == 1 else (B, H, 1, 1)), generator=g)
    if dtype == torch.float32:
        # The fp32 gate (rtol 1e-5) is stated at gamma |k|^2 of order 1 (config 3:
        # D = 32, gamma = 1/32): larger exponents leave it for any fp32 chain.
        base = base * min(1.0, 1.5 / (0.11 * D * s * s))
    scale = base.reshape(()) if form == 0 else base
    kind = int(rng.integers(4))
    bias = None
    if kind == 1:  # key padding per batch entry, some rows fully masked
        counts = torch.randint(0, nk + 1, (B,), generator=g)
        bias = torch.zeros(B, 1, 1, nk).masked_fill((torch.arange(nk)[None, :] >= counts[:, None])[:, None, None, :],
                                                     float('-inf'))
    elif kind == 2:  # per-head padding
        counts = torch.randint(1, nk + 1, (B, H), generator=g)
        bias = torch.zeros(B, H, 1, nk).masked_fill((torch.arange(nk) >= counts[..., None])[:, :, None, :],
                                                    float('-inf'))
    elif kind == 3:
        bias = torch.randn(B, 1, 1, nk, generator=g)
    if bias is not None and dtype != torch.float32:
        bias = bias.to([torch.float32, torch.bfloat16, torch.float16][int(rng.integers(3))])
    return q, k, v, scale, bias


def _variants(q, k, v, scale, bias):
    scale4, bias4 = capi.broadcast_operands(q, k, scale, bias)
    out = torch.empty((*q.shape[:-1], v.shape[-1]), device='cuda')
    names = ['auto']
    for name in ('generic', 'stream', 'mfma', 'plane', 'tile'):
        if capi.select_variant(capi.make_args(q, k, v, out, scale4, bias4, name)) > 0:
            names.append(name)
    return names


@pytest.mark.parametrize('seed', range(48))
def test_random_rbf_cases_on_every_variant(seed):
    q, k, v, scale, bias = _case(1000 + seed)
    rtol, atol = GATES[q.dtype]
    ref = oracle.direct_fp64(q, k, v, scale, bias)
    eager = oracle.eager_fp32(q, k, v, scale, bias, batch_chunk=1).double().numpy()
    spread = max(1.0, float(v.float().abs().max()) / 3.0)
    with np.errstate(invalid='ignore'):
        allow = atol * spread + rtol * np.abs(ref) + np.nan_to_num(4.0 * np.abs(eager - ref), nan=0.0, posinf=0.0)
    dev = [None if x is None else x.cuda() for x in (q, k, v, scale, bias)]
    for variant in _variants(*dev):
        got = capi.forward(*dev, out_dtype=torch.float32, variant=variant)
        torch.cuda.synchronize()
        got = got.cpu().double().numpy()
        assert np.array_equal(np.isnan(got), np.isnan(ref)), variant
        finite = ~np.isnan(ref)
        worst = np.max(np.abs(got - ref)[finite] - allow[finite], initial=-np.inf)
        assert worst <= 0, f'{variant}: worst excess {worst:.3g} over the gate'
    out = torch.ops.vectra.rbf_attention(*dev)
    fp32 = capi.forward(*dev, out_dtype=torch.float32)
    torch.cuda.synchronize()
    # The operator's output is the fp32 result rounded once (fully masked rows: NaN in both).
    torch.testing.assert_close(out.cpu(), fp32.cpu().to(out.dtype), rtol=0, atol=0, equal_nan=True)


@pytest.mark.parametrize('seed', range(24))
def test_random_top_k_cases_in_every_form(seed):
    rng = np.random.default_rng(2000 + seed)
    g = torch.Generator().manual_seed(2000 + seed)
    n_rows = int(rng.choice([1, 7, 100, 1030, 2060]))
    dim = int(rng.choice([8, 32, 100, 128]))
    n_q = int(rng.choice([1, 3, 64, 65]))
    k = int(rng.choice([1, 10, 100, 1000, 1024]))
    rows = torch.randn(n_rows, dim, generator=g)
    if rng.random() < 0.2:
        rows[int(rng.integers(n_rows))] = float('nan')
    queries = torch.randn(n_q, dim, generator=g)
    kind = int(rng.integers(4))
    ids = None
    if kind == 1:  # ids past the row count are skipped, duplicates kept
        ids = torch.randint(0, n_rows + 40, (int(rng.integers(1, 2 * n_rows + 10)),), generator=g).to(torch.int32)
    elif kind == 2:
        ids = torch.randperm(n_rows, generator=g)[: max(1, n_rows // 2)].to(torch.int32)
    elif kind == 3:
        ids = torch.zeros(0, dtype=torch.int32)
    want_d, want_n = scan_oracle.nearest(queries.numpy(), rows.numpy(), k, None if ids is None else ids.numpy())
    for form in scan.TOP_K_FORMS:
        d, n = scan.nearest(queries.cuda(), rows.cuda(), k, None if ids is None else ids.cuda(), form=form)
        torch.cuda.synchronize()
        assert np.array_equal(d.cpu().numpy().view(np.uint32), want_d.view(np.uint32)), form
        assert np.array_equal(n.cpu().numpy(), want_n), form
