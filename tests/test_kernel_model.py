"""The plane and tile kernels' own numerics, modelled on the CPU
(tests/kernel_model.py), against the fp64 oracle.

The kernels replace the reference's online softmax with unshifted exp2 and a
range check, feed the weights as 16-bit hi + lo pairs and drop the clamp of
the expanded distance at 0.  These tests run that design on the CPU over the
16-bit edge cases and over the regime where dropping the clamp matters most
(large norms with a large gamma), so its error is bounded before any GPU
run; tests/test_kernel_model_gpu.py then holds the kernels to the model.
"""

import zlib

import numpy as np
import pytest
import torch

from oracle import rbf as oracle
from tests import kernel_model as km
from tests.half_cases import HALF_CASES, HALF_KERNEL_SHAPES, half_case

HALF_TOL = {'rtol': 1e-3, 'atol': 1e-4}
KINDS = {'bf16': torch.bfloat16, 'fp16': torch.float16}


def _case(case, shape, kind):
    n_q, n_k, dim = HALF_KERNEL_SHAPES[shape]
    gen = torch.Generator().manual_seed(zlib.crc32(f'{case}/{shape}'.encode()) % 1000)
    q, k, v, scale, bias = half_case(case, n_q, n_k, dim, gen)
    dt = KINDS[kind]
    return q.to(dt).float(), k.to(dt).float(), v.to(dt).float(), scale, bias


@pytest.mark.parametrize('kind', sorted(KINDS))
@pytest.mark.parametrize('shape', sorted(HALF_KERNEL_SHAPES))
@pytest.mark.parametrize('case', HALF_CASES)
def test_the_design_meets_the_gate_on_the_edge_cases(case, shape, kind):
    q, k, v, scale, bias = _case(case, shape, kind)
    model = 'plane' if shape.startswith('plane') else 'tile'
    got, _ = km.run(model, q, k, v, scale, bias, kind)
    want = oracle.expanded_fp64(q, k, v, scale, bias)
    np.testing.assert_allclose(got, want, equal_nan=True, **HALF_TOL)


def test_both_branches_are_taken():
    """The shifted recompute runs exactly where the unshifted weights leave
    the accurate range, and not on ordinary inputs."""
    seen = {}
    for kind in KINDS:
        for case in HALF_CASES:
            for shape in ('plane32', 'tile32'):
                q, k, v, scale, bias = _case(case, shape, kind)
                _, path = km.run(shape[:-2], q, k, v, scale, bias, kind)
                seen[(kind, case, shape)] = (path == km.SHIFTED).mean()
    for kind in KINDS:
        # Far points: the weights underflow unshifted (a block is recomputed
        # when any of its 16 queries leaves the range).
        assert seen[(kind, 'far_points', 'plane32')] >= 0.9
        assert seen[(kind, 'far_points', 'tile32')] == 1.0
        # Biases of +-40: far outside both ranges.
        assert seen[(kind, 'large_biases', 'plane32')] == 1.0
        # Fully masked rows (sum 0) are recomputed, to NaN; the others not.
        assert seen[(kind, 'fully_masked', 'plane32')] == 0.5
        # Ordinary inputs stay unshifted in the plane kernel.
        for case in ('negative_scale', 'zero_scale', 'one_live_key', 'ragged_mask'):
            assert seen[(kind, case, 'plane32')] == 0.0, case
        # The tile kernel's single pass needs no bias and gamma >= 0.
        for case in ('negative_scale', 'zero_scale', 'ragged_mask'):
            assert seen[(kind, case, 'tile32')] == 1.0, case
        q, k, v, _, _ = _case('ragged_mask', 'tile32', kind)
        assert (km.run('tile', q, k, v, torch.tensor(0.01), None, kind)[1] == km.SPLIT).all()


# Cases where one unshifted pass misses the gate: weights that overflow
# (biases of +-40) or underflow to a 0 / 0 sum (far points in the tile kernel,
# whose logits are <= 0 by construction).
ONE_PASS_FAILS = {
    'bf16': [('large_biases', 'plane16'), ('large_biases', 'tile32'), ('far_points', 'tile64')],
    'fp16': [('large_biases', 'plane16'), ('large_biases', 'plane32'), ('large_biases', 'tile64'),
             ('far_points', 'plane32'), ('far_points', 'tile32')],
}


@pytest.mark.parametrize('kind', sorted(KINDS))
def test_the_range_check_is_needed(kind):
    """Where the model recomputes, one unshifted pass would miss the gate on
    these cases, so the check is not decorative."""
    for case, shape in ONE_PASS_FAILS[kind]:
        q, k, v, scale, bias = _case(case, shape, kind)
        model = 'plane' if shape.startswith('plane') else 'tile'
        want = oracle.expanded_fp64(q, k, v, scale, bias)
        one, _ = km.run(model, q, k, v, scale, bias, kind, one_pass=True)
        with np.errstate(invalid='ignore'):
            bad = ~np.isclose(one, want, equal_nan=True, **HALF_TOL)
        assert bad.mean() > 0.1, (case, shape)


def test_split_precision():
    """hi + lo keeps ~2^-17 of a bf16-split weight anywhere in fp32's range;
    fp16 keeps 2^-20 of weights in [2^-3, 2^15) and an absolute 2^-24 below
    (its subnormal step), which the range check's sum >= 2^-3 makes
    relative 2^-21 of the sum."""
    rng = np.random.default_rng(0)
    w = np.exp2(rng.uniform(-100, 30, 200000)).astype(np.float32)
    hi, lo = km.split(w, 'bf16')
    assert (np.abs((hi.astype(np.float64) + lo) - w) / w).max() <= 2.0 ** -16
    w = np.exp2(rng.uniform(-30, 14.9, 200000)).astype(np.float32)
    hi, lo = km.split(w, 'fp16')
    err = np.abs((hi.astype(np.float64) + lo) - w)
    normal = w >= 2.0 ** -3
    assert (err[normal] / w[normal]).max() <= 2.0 ** -20
    assert err[~normal].max() <= 2.0 ** -24
    # Round toward zero: hi never exceeds w, and lo >= 0.
    assert (hi <= w).all() and (lo >= 0).all()


def _large_norm_case(seed, norm, gamma, n_q=40, n_k=65, dim=32, kind='bf16'):
    """A cluster of keys of radius ~1 around a centre of norm `norm`, and
    queries inside it: the distances are O(1), so the weights are spread
    (gamma d of a few units), while |q|^2 + |k|^2 is ~2 norm^2, so the
    expansion |q|^2 + |k|^2 - 2 q.k cancels ~2 norm^2 down to O(1)."""
    gen = torch.Generator().manual_seed(seed)
    centre = torch.randn(dim, generator=gen)
    centre = centre / centre.norm() * norm
    k = centre + torch.randn(1, 1, n_k, dim, generator=gen) / dim ** 0.5
    q = centre + torch.randn(1, 1, n_q, dim, generator=gen) / dim ** 0.5
    v = torch.randn(1, 1, n_k, dim, generator=gen)
    dt = KINDS[kind]
    return q.to(dt).float(), k.to(dt).float(), v.to(dt).float(), torch.tensor(gamma), None


@pytest.mark.parametrize('kind', sorted(KINDS))
@pytest.mark.parametrize('norm,gamma', [(3.0, 2.0), (10.0, 2.0), (30.0, 2.0), (100.0, 2.0), (100.0, 0.5)])
def test_dropping_the_clamp_costs_no_more_than_the_expansion_error(kind, norm, gamma):
    """Large norms with a large gamma, where the clamp's effect is largest.

    Without the clamp the kernels' logit for key j differs from the
    reference's clamped one only where the rounded expansion is negative,
    and then by gamma |d~| with |d~| <= (D + 2) u (|q|^2 + |k|^2) (u = 2^-24,
    the standard bound of a D-term fp32 dot product): the same size as the
    expansion's own rounding error, which the reference's fp32 kernel
    (reproduced by oracle.tiled in fp32, with its clamp) carries as well.  So
    the model's error against fp64 is held to that of the reference's
    algorithm in fp32, plus the 16-bit split's share."""
    q, k, v, scale, bias = _large_norm_case(int(norm * 7 + gamma * 100), norm, gamma, kind=kind)
    want = oracle.direct_fp64(q, k, v, scale, bias)
    ref32 = oracle.tiled(q, k, v, scale, bias, dtype=np.float32)
    ref_err = np.abs(ref32 - want).max()
    for model in ('plane', 'tile'):
        got, _ = km.run(model, q, k, v, scale, bias, kind)
        err = np.abs(got - want).max()
        assert err <= 2 * ref_err + 1e-5, (model, err, ref_err)
    # The bound itself, per logit, on these inputs.
    dim = q.shape[-1]
    qn = (q.double() ** 2).sum(-1)[..., :, None]
    kn = (k.double() ** 2).sum(-1)[..., None, :]
    bound = gamma * (dim + 2) * 2.0 ** -24 * (qn + kn)
    d32 = (qn.float() + kn.float() - 2 * q @ k.transpose(-1, -2)).double()
    d64 = ((q.double()[..., :, None, :] - k.double()[..., None, :, :]) ** 2).sum(-1)
    assert (gamma * (d32 - d64).abs() <= bound).all()


# The tile kernel's fast pass (fp16 weights, no split) on long key axes.

def _long_keys(seed, kind, n_k=1280, n_q=320, dim=64, gamma=0.03, v_scale=0.25):
    """A plane like config 4's (q, k ~ 0.5 N(0, 1)) with values v_scale N(0, 1)
    and a key axis long enough for the fast pass; 320 queries are two work
    items of 64-dim heads (256 and 64 rows).  (At 1280 keys the fast pass holds for values of a quarter of
    config 4's; config 4's own values need its 4096 keys.)"""
    gen = torch.Generator().manual_seed(seed)
    q = 0.5 * torch.randn(1, 1, n_q, dim, generator=gen)
    k = 0.5 * torch.randn(1, 1, n_k, dim, generator=gen)
    v = v_scale * torch.randn(1, 1, n_k, dim, generator=gen)
    dt = KINDS[kind]
    return q.to(dt).float(), k.to(dt).float(), v.to(dt).float(), torch.tensor(gamma), None


def _concentrated(seed, n_live, kind, n_k=1024, n_q=32, dim=64):
    """Weights held by `n_live` keys (each in (1/2, 1]) against values of +-4,
    the rest of the keys far away: the fewer live keys, the less the fp16
    rounding errors of the weights average out."""
    gen = torch.Generator().manual_seed(seed)
    q = 0.02 * torch.randn(1, 1, n_q, dim, generator=gen)
    u = torch.randn(n_k, dim, generator=gen)
    u = u / u.norm(dim=-1, keepdim=True)
    dist = torch.full((n_k,), 40.0)
    dist[:n_live] = 0.69 * torch.rand(n_live, generator=gen)
    k = (u * dist.sqrt()[:, None])[None, None]
    v = torch.randn(1, 1, n_k, dim, generator=gen)
    v[..., :n_live, :] = 4 * torch.sign(torch.randn(n_live, dim, generator=gen))
    dt = KINDS[kind]
    return q.to(dt).float(), k.to(dt).float(), v.to(dt).float(), torch.tensor(1.0), None


@pytest.mark.parametrize('kind', sorted(KINDS))
def test_the_fast_pass_runs_where_it_holds(kind):
    q, k, v, scale, bias = _long_keys(1, kind)
    assert (km.run('tile', q, k, v, scale, bias, kind)[1] == km.FAST).all()
    # Shorter key axes, a bias, or gamma < 0 never try it.
    short = _long_keys(1, kind, n_k=km.FAST_KEYS - 24)
    assert (km.run('tile', *short, kind)[1] == km.SPLIT).all()
    assert (km.run('tile', q, k, v, scale, torch.zeros(1, 1, 1, k.shape[2]), kind)[1] == km.SHIFTED).all()
    assert (km.run('tile', q, k, v, torch.tensor(-0.01), bias, kind)[1] == km.SHIFTED).all()
    # Weight sums below FAST_SUM (a large gamma) send the item to the split.
    assert (km.run('tile', q, k, v, torch.tensor(0.3), bias, kind)[1] != km.FAST).all()
    # Per work item: queries far from the keys in the second item only.
    item = km.TILE_ITEM_ROWS[64]
    far = q.clone()
    far[..., item:, :] += 1.5
    far = far.to(KINDS[kind]).float()
    path = km.run('tile', far, k, v, scale, bias, kind)[1][0, 0]
    assert (path[:item] == km.FAST).all() and (path[item:] != km.FAST).all()
    # Values 16 times larger: the bound misses the contract, the item splits.
    big = (v * 16).to(KINDS[kind]).float()
    assert (km.run('tile', q, k, big, scale, bias, kind)[1] == km.SPLIT).all()


def test_values_fp16_cannot_hold_send_the_item_to_the_split():
    q, k, v, scale, bias = _long_keys(2, 'bf16')
    v[..., 7, 3] = 2.0 ** 17  # a bf16 value beyond fp16's range
    got, path = km.run('tile', q, k, v, scale, bias, 'bf16')
    assert (path == km.SPLIT).all()
    want = oracle.expanded_fp64(q, k, v, scale, bias)
    np.testing.assert_allclose(got, want, **HALF_TOL)


def _config4_plane(seed, kind, gamma, v_scale, n_q=128):
    """One plane of config 4 (q, k ~ 0.5 N(0, 1), v ~ N(0, 1), 4096 keys of 64
    dims), 128 queries (part of one work item), values scaled by v_scale."""
    return _long_keys(seed, kind, n_k=4096, n_q=n_q, gamma=gamma, v_scale=v_scale)


@pytest.mark.parametrize('kind', sorted(KINDS))
@pytest.mark.parametrize('gamma', [0.005, 0.03, 0.05])
def test_the_fast_pass_meets_the_gate_on_config_4(kind, gamma):
    """Config 4's key axis and range of gamma with its own values: the fast
    pass holds for every query, stays within the reference's fp16 bound
    (2^-11 of the spread of the values, kernels/tests/test_parity.py:16-23)
    and within the 1e-3 / 1e-4 gate."""
    q, k, v, scale, bias = _config4_plane(int(gamma * 1000), kind, gamma, 1.0)
    got, path = km.run('tile', q, k, v, scale, bias, kind)
    assert (path == km.FAST).all()
    want = oracle.expanded_fp64(q, k, v, scale, bias)
    vv = v.double().numpy()[0, 0]
    spread = vv.max(0) - vv.min(0)
    assert (np.abs(got - want) <= 2.0 ** -11 * spread + 1e-6).all()
    np.testing.assert_allclose(got, want, **HALF_TOL)


@pytest.mark.parametrize('kind', sorted(KINDS))
@pytest.mark.parametrize('v_scale', [1.0, 16.0, 256.0])
def test_the_default_path_holds_the_gate_at_any_value_scale(kind, v_scale):
    """Config 4's q, k and gamma range with the values scaled by 1, 16 and
    256: the default path (fast pass where its bound allows, the split
    otherwise) stays inside the gate.  Unit values keep the fast pass; larger
    ones are sent to the split.  With the check reduced to its old form
    (weight sums of at least FAST_SUM and finite outputs, no bound), the
    fast pass is kept at x16 and x256 and misses the gate."""
    for gamma in (0.005, 0.05):
        q, k, v, scale, bias = _config4_plane(7 + int(v_scale), kind, gamma, v_scale)
        want = oracle.expanded_fp64(q, k, v, scale, bias)
        got, path = km.run('tile', q, k, v, scale, bias, kind)
        np.testing.assert_allclose(got, want, err_msg=f'gamma={gamma}', **HALF_TOL)
        assert (path == (km.FAST if v_scale == 1.0 else km.SPLIT)).all()
        if v_scale > 1.0:
            old = _without_the_bound(q, k, v, scale, bias, kind)
            assert not np.allclose(old, want, **HALF_TOL), gamma


def _without_the_bound(q, k, v, scale, bias, kind):
    """The model with the fast pass's check reduced to its old form."""
    saved = km.fast_misses
    def old(acc, total, wsq, vmax, seen, n_k, slack=1.0):
        return ~(np.isfinite(acc).all(-1) & (total * (n_k / seen) * slack >= km.FAST_SUM))
    km.fast_misses = old
    try:
        return km.run('tile', q, k, v, scale, bias, kind)[0]
    finally:
        km.fast_misses = saved


def _walk_bound(x, v16):
    """Per output, the check's bound on the deviation of the fast pass's
    rounding walk (one deviation: FAST_WALK / FAST_SIGMAS), from the fp16
    weights' own sums."""
    acc, total, wsq = km._weighted_fast(x, v16)
    o = np.abs(acc.astype(np.float64) / total.astype(np.float64)[:, None])
    per = km.FAST_WALK / km.FAST_SIGMAS * np.sqrt(wsq.astype(np.float64)) / total
    return per[:, None] * (np.abs(v16).max() + o), acc, total


def _fast_logits(q, k, v, scale):
    """The tile kernel's unshifted logits for one plane, and its fp16 values."""
    qq, kk, vv = (t.numpy()[0, 0].astype(np.float32) for t in (q, k, v))
    coef, c = km._folded_keys(kk, km.F32(scale), None)
    half_q = (km.F32(-0.5) * (qq.astype(np.float64) ** 2).sum(-1).astype(np.float32)).astype(np.float32)
    s = ((qq.astype(np.float64) @ kk.astype(np.float64).T) + half_q[:, None]).astype(np.float32)
    return km.fma32(coef, s, c[None, :]), vv.astype(np.float16).astype(np.float32)


@pytest.mark.parametrize('values', ['normal', 'two_valued', 'offset'])
def test_the_bound_covers_the_walk(values):
    """Across value distributions the fast pass's error against the exact
    weights, in units of the check's bound on the walk's deviation, has a
    root mean square of at most 1 (the bound is at least the deviation) and
    stays below the FAST_SIGMAS units the check allows at every output.
    Values of +-4 on every key make max|v - o| equal the typical |v - o|, the
    hardest case for a bound taken from max|v| (measured: rms 0.8, worst 3.4
    over 16K outputs); normal values sit far inside (rms ~0.2), and values
    offset by 100 farther still (the bound takes max|v| + |o|, not the
    spread: safe, and the relative allowance keeps such items on the fast
    pass).  Weights rounded to bf16 (2^-9, as the reference rounds them for
    bf16 inputs) leave the bound for normal and two-valued values."""
    ratios, coarse_ratios = [], []
    for seed in range(4):
        q, k, v, scale, bias = _long_keys(40 + seed, 'bf16', n_k=2048, n_q=64, gamma=0.02, v_scale=1.0)
        if values == 'two_valued':
            v = 4 * torch.sign(v)
        elif values == 'offset':
            v = (100 + v).to(torch.bfloat16).float()
        x, v16 = _fast_logits(q, k, v, scale)
        bound, acc, total = _walk_bound(x, v16)
        exact = oracle.expanded_fp64(q, k, v, scale, bias)[0, 0]
        err = np.abs(acc / total[:, None].astype(np.float64) - exact)
        ratios.append((err / bound).ravel())
        coarse, ctot = _bf16_weights(x, v16)
        cerr = np.abs(coarse / ctot[:, None].astype(np.float64) - exact)
        coarse_ratios.append((cerr / bound).ravel())
    ratio, coarse_ratio = np.concatenate(ratios), np.concatenate(coarse_ratios)
    assert np.sqrt((ratio ** 2).mean()) <= 1.0 and ratio.max() < km.FAST_SIGMAS, (ratio.max(), values)
    if values == 'offset':
        assert ratio.max() < 0.1
    else:
        assert np.sqrt((coarse_ratio ** 2).mean()) > 1.0 and coarse_ratio.max() > km.FAST_SIGMAS


def _bf16_weights(x, v16):
    """The fast pass with the weights rounded to bf16 (2^-9) instead."""
    w = km.to_bf16(km.exp2_32(x)).astype(np.float64)
    return (w @ v16.astype(np.float64)).astype(km.F32), w.sum(-1).astype(km.F32)


@pytest.mark.parametrize('kind', sorted(KINDS))
def test_the_fast_pass_check_is_needed(kind):
    """Weights held by a few keys, or many keys against values of +-4 (the
    check's edge): the model takes the split pass and meets the gate; the
    fast pass kept regardless would miss it."""
    for n_live in (4, 16, 64, 380):
        q, k, v, scale, bias = _concentrated(n_live, n_live, kind)
        want = oracle.expanded_fp64(q, k, v, scale, bias)
        got, path = km.run('tile', q, k, v, scale, bias, kind)
        assert (path == km.SPLIT).all()
        np.testing.assert_allclose(got, want, **HALF_TOL)
        saved = km.fast_misses
        km.fast_misses = lambda acc, *rest, **kw: np.zeros(acc.shape[0], dtype=bool)
        try:
            forced, path = km.run('tile', q, k, v, scale, bias, kind)
        finally:
            km.fast_misses = saved
        assert (path == km.FAST).all()
        assert not np.allclose(forced, want, **HALF_TOL), n_live


def test_the_pass_is_abandoned_early_where_the_bound_fails_early():
    """Values 16 times config 4's: the check's course after an eighth of the
    keys already misses twice over, so the pass stops there (the split runs);
    large values only past that point are caught by the final check."""
    q, k, v, scale, bias = _config4_plane(3, 'bf16', 0.03, 16.0, n_q=32)
    x, v16 = _fast_logits(q, k, v, scale)
    acc, total, kept = km.fast_pass(x, v16, 4096)
    assert acc is None and not kept  # abandoned at the probe
    q, k, v, scale, bias = _config4_plane(3, 'bf16', 0.03, 1.0, n_q=32)
    v[..., 2048:, :] *= 64
    v = v.to(torch.bfloat16).float()
    x, v16 = _fast_logits(q, k, v, scale)
    acc, total, kept = km.fast_pass(x, v16, 4096)
    assert acc is not None and not kept  # ran to the end, then failed the check
    got, path = km.run('tile', q, k, v, scale, bias, 'bf16')
    assert (path == km.SPLIT).all()
    np.testing.assert_allclose(got, oracle.expanded_fp64(q, k, v, scale, bias), **HALF_TOL)
