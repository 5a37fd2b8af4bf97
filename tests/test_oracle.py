"""Pins the CPU oracle before anything is checked against it.

Each oracle function (oracle/rbf.py) is checked against:
* the brute-force golden fixtures (tests/golden/make_golden.py);
* library identities: torch's scaled_dot_product_attention with the
  expansion folded into q and the mask, and torch.cdist (the form the
  reference pins its model with, models/tests/test_model.py:88-100);
* closed-form special cases (kernels/tests/test_edges.py:59-101);
and a set of planted mistakes shows that each plausible error fails a pin.
"""

import math

import numpy as np
import pytest
import torch

from oracle import rbf as oracle
from tests import _golden

F = torch.nn.functional

ORACLES = {
    'direct_fp64': oracle.direct_fp64,
    'expanded_fp64': oracle.expanded_fp64,
    'tiled_fp64': lambda *a: oracle.tiled(*a, block_q=4, block_k=8),
    'tiled_fp64_big_tiles': oracle.tiled,
}


def _args(case):
    return case['q'], case['k'], case['v'], case['scale'], case['bias']


@pytest.mark.parametrize('name', sorted(_golden.cases()))
@pytest.mark.parametrize('which', sorted(ORACLES))
def test_fp64_oracles_match_brute_force_fixtures(name, which):
    case = _golden.cases()[name]
    got = np.asarray(ORACLES[which](*_args(case)))
    want = case['expected'].numpy()
    np.testing.assert_allclose(got, want, rtol=1e-9, atol=1e-9, equal_nan=True)


@pytest.mark.parametrize('name', sorted(_golden.cases()))
def test_eager_fp32_chain_matches_fixtures(name):
    case = _golden.cases()[name]
    got = oracle.eager_fp32(*_args(case)).double().numpy()
    want = case['expected'].numpy()
    # Far points: fp32 sums of squares of ~1e3 lose ~1e-4 of the logit.
    atol = 2e-3 if name == 'far_points' else 2e-5
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=atol, equal_nan=True)


def test_tiled_fp32_tracks_fp64():
    gen = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(2, 3, 37, 16, generator=gen) for _ in range(3))
    scale = torch.rand(1, 3, 1, 1, generator=gen) * 0.1
    bias = torch.zeros(2, 1, 1, 37)
    bias[1, ..., 30:] = -math.inf
    want = oracle.direct_fp64(q, k, v, scale, bias)
    got = oracle.tiled(q, k, v, scale, bias, block_q=16, block_k=16, dtype=np.float32)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


def _random_problem(seed, b=2, h=3, n_q=7, n_k=11, d=8, dv=5, bias_heads=1):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(b, h, n_q, d, generator=gen, dtype=torch.float64)
    k = torch.randn(b, h, n_k, d, generator=gen, dtype=torch.float64)
    v = torch.randn(b, h, n_k, dv, generator=gen, dtype=torch.float64)
    scale = 0.02 + 0.1 * torch.rand(1, h, 1, 1, generator=gen, dtype=torch.float64)
    bias = torch.zeros(b, bias_heads, 1, n_k, dtype=torch.float64)
    bias[0, ..., n_k - 3 :] = -math.inf
    return q, k, v, scale, bias


def _sdpa_pin(q, k, v, scale, bias):
    """-s|q-k|^2 = 2s q.k - s|k|^2 - s|q|^2; the last term is constant per row."""
    k_norm = (k * k).sum(-1)[..., None, :]
    mask = -scale * k_norm + bias
    return F.scaled_dot_product_attention(2 * scale * q, k, v, attn_mask=mask, scale=1.0)


def _cdist_pin(q, k, v, scale, bias):
    d2 = torch.cdist(q, k) ** 2
    return torch.softmax(-d2 * scale + bias, dim=-1) @ v


@pytest.mark.parametrize('seed', range(4))
@pytest.mark.parametrize('pin', [_sdpa_pin, _cdist_pin], ids=['sdpa', 'cdist'])
def test_library_identities(seed, pin):
    args = _random_problem(seed, bias_heads=1 + 2 * (seed % 2))
    want = pin(*args).numpy()
    for fn in ORACLES.values():
        np.testing.assert_allclose(np.asarray(fn(*args)), want, rtol=1e-9, atol=1e-10)
    np.testing.assert_allclose(
        oracle.eager_fp32(*args).double().numpy(), want, rtol=1e-4, atol=1e-5
    )


@pytest.mark.parametrize('fn', list(ORACLES.values()) + [oracle.eager_fp32])
def test_closed_form_special_cases(fn):
    gen = torch.Generator().manual_seed(11)
    q = torch.randn(2, 2, 3, 8, generator=gen)
    k = torch.randn(2, 2, 9, 8, generator=gen)
    v = torch.randn(2, 2, 9, 6, generator=gen)
    s = torch.tensor(0.07)

    def run(*a):
        return torch.as_tensor(np.asarray(fn(*a))).double()

    # One live key: every query returns that key's value.
    one = torch.full((2, 1, 1, 9), -math.inf)
    one[..., 4] = 0.0
    torch.testing.assert_close(run(q, k, v, s, one), v[:, :, 4:5].double().expand(2, 2, 3, 6))
    # Zero scale: the masked mean of v.
    counts = torch.tensor([3, 9])
    bias = torch.zeros(2, 1, 1, 9)
    bias[0, ..., 3:] = -math.inf
    mean = torch.stack([v[0, :, :3].mean(1), v[1].mean(1)]).double()
    torch.testing.assert_close(
        run(q, k, v, torch.tensor(0.0), bias), mean[:, :, None].expand(2, 2, 3, 6)
    )
    assert counts.sum() == 12
    # A single key.
    torch.testing.assert_close(
        run(q, k[:, :, :1], v[:, :, :1], s, None), v[:, :, :1].double().expand(2, 2, 3, 6)
    )
    # Fully masked rows are NaN, as eager softmax gives.
    assert torch.isnan(run(q, k, v, s, torch.full((2, 1, 1, 9), -math.inf))).all()
    # A constant added to every key's bias changes nothing.
    torch.testing.assert_close(
        run(q, k, v, s, bias + 3.5), run(q, k, v, s, bias), rtol=1e-5, atol=1e-6
    )


# --- Planted mistakes: each must fail at least one pin. ---------------------


def _mistake_sign(q, k, v, s, b):
    return oracle.expanded_fp64(q, k, v, -s, b)


def _mistake_dropped_k_norm(q, k, v, s, b):
    q, k, v = (t.double() for t in (q, k, v))
    sq = (q * q).sum(-1, keepdim=True) - 2 * q @ k.transpose(-1, -2)
    logits = -sq * s.double() + (0 if b is None else b.double())
    return (torch.softmax(logits, -1) @ v).numpy()


def _mistake_wrong_axis(q, k, v, s, b):
    q, k, v = (t.double() for t in (q, k, v))
    sq = ((q.unsqueeze(-2) - k.unsqueeze(-3)) ** 2).sum(-1)
    logits = -sq * s.double() + (0 if b is None else b.double())
    return (torch.softmax(logits, -2) @ v).numpy()


def _mistake_divisor(q, k, v, s, b):
    return oracle.expanded_fp64(q, k, v, 1.0 / s.double(), b)


def _mistake_transposed_k(q, k, v, s, b):
    # Keys and values swapped (same shapes when D == Dv).
    return oracle.direct_fp64(q, v, k, s, b)


def _mistake_bias_off_by_one(q, k, v, s, b):
    # Key j reads the bias of key j - 1.
    return oracle.direct_fp64(q, k, v, s, None if b is None else b.roll(1, -1))


def _mistake_no_max_guard(q, k, v, s, b):
    # Softmax without subtracting the row maximum: far points underflow.
    q, k, v = (t.double() for t in (q, k, v))
    sq = ((q.unsqueeze(-2) - k.unsqueeze(-3)) ** 2).sum(-1)
    e = torch.exp((-sq * s.double() + (0 if b is None else b.double())).float()).double()
    return (e / e.sum(-1, keepdim=True) @ v).numpy()


MISTAKES = [
    _mistake_sign,
    _mistake_dropped_k_norm,
    _mistake_wrong_axis,
    _mistake_divisor,
    _mistake_transposed_k,
    _mistake_bias_off_by_one,
    _mistake_no_max_guard,
]


def _passes_all_pins(fn) -> bool:
    try:
        for case in _golden.cases().values():
            if case['k'].shape[2] == 0:
                continue
            if case['v'].shape != case['k'].shape and fn is _mistake_transposed_k:
                continue
            got = np.asarray(fn(*_args(case)))
            if not np.allclose(got, case['expected'].numpy(), rtol=1e-6, atol=1e-7, equal_nan=True):
                return False
        for seed in range(2):
            args = _random_problem(seed, n_q=5, n_k=5, d=5, dv=5)
            if not np.allclose(np.asarray(fn(*args)), _sdpa_pin(*args).numpy(), rtol=1e-6, atol=1e-7):
                return False
    except (RuntimeError, ValueError):
        return False
    return True


@pytest.mark.parametrize('mistake', MISTAKES, ids=lambda f: f.__name__)
def test_planted_mistakes_fail_a_pin(mistake):
    assert not _passes_all_pins(mistake)


def test_pins_accept_the_oracle():
    assert _passes_all_pins(oracle.expanded_fp64)
    assert _passes_all_pins(oracle.direct_fp64)
