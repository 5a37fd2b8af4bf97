"""The plane and tile kernels against the CPU model of their own numerics
(tests/kernel_model.py), on the GPU.

The model takes its sums in float64 and rounds once, while the matrix cores
accumulate in their own order; with logits of a few hundred (far points) a
float32 ulp of q.k moves a weight by ~2e-5 of itself.  So the two agree to
rtol 1e-4 / atol 2e-5: ten times inside the 1e-3 / 1e-4 gate, and twenty
times below what a dropped lo part (2^-9 of every weight), a missed
recompute (0 / 0 or overflow) or a wrong folded key value would change.  The
cases are the 16-bit edge cases, which drive both kernels through both
branches, and, against fp64, the large-norm cases where dropping the clamp matters
most; and the tile kernel's long-key paths, config 4's values scaled by 1, 16
and 256 among them.
"""

import zlib

import numpy as np
import pytest
import torch

from oracle import rbf as oracle
from tests import kernel_model as km
from tests.half_cases import HALF_CASES, HALF_KERNEL_SHAPES, half_case
from tests.test_kernel_model import _concentrated, _config4_plane, _large_norm_case, _long_keys
from vectra_amd.kernels import capi

pytestmark = pytest.mark.gpu

MODEL_TOL = {'rtol': 1e-4, 'atol': 2e-5}
KINDS = {'bf16': torch.bfloat16, 'fp16': torch.float16}


def _kernel(q, k, v, scale, bias, dtype, variant, split_weights=False):
    out = capi.forward(q.to('cuda', dtype), k.to('cuda', dtype), v.to('cuda', dtype), scale.cuda(),
                       None if bias is None else bias.cuda(), out_dtype=torch.float32, variant=variant,
                       split_weights=split_weights)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize('kind', sorted(KINDS))
@pytest.mark.parametrize('shape', sorted(HALF_KERNEL_SHAPES))
@pytest.mark.parametrize('case', HALF_CASES)
def test_kernels_follow_the_model(case, shape, kind):
    n_q, n_k, dim = HALF_KERNEL_SHAPES[shape]
    gen = torch.Generator().manual_seed(zlib.crc32(f'{case}/{shape}'.encode()) % 1000)
    q, k, v, scale, bias = half_case(case, n_q, n_k, dim, gen)
    dt = KINDS[kind]
    q, k, v = q.to(dt).float(), k.to(dt).float(), v.to(dt).float()
    variant = 'plane' if shape.startswith('plane') else 'tile'
    print(f'case={case} shape={shape} kind={kind} variant={variant}', flush=True)
    want, _ = km.run(variant, q, k, v, scale, bias, kind)
    got = _kernel(q, k, v, scale, bias, dt, variant)
    np.testing.assert_allclose(got, want, equal_nan=True, **MODEL_TOL)


@pytest.mark.parametrize('kind', sorted(KINDS))
@pytest.mark.parametrize('norm,gamma', [(10.0, 2.0), (30.0, 2.0), (100.0, 2.0), (100.0, 0.5)])
def test_large_norms_without_the_clamp(kind, norm, gamma):
    """Where the dropped clamp matters most, the kernels err against fp64 no
    more than the reference's algorithm does in fp32 (oracle.tiled, with its
    clamp).  (Here the logits are differences of terms ~2 norm^2 apart, so
    float32 accumulation order alone moves them by ~1e-3: the kernels are
    held to the error bound, not to the model's float64 sums.)"""
    q, k, v, scale, bias = _large_norm_case(int(norm * 7 + gamma * 100), norm, gamma, kind=kind)
    want = oracle.direct_fp64(q, k, v, scale, bias)
    ref_err = np.abs(oracle.tiled(q, k, v, scale, bias, dtype=np.float32) - want).max()
    for variant in ('plane', 'tile'):
        got = _kernel(q, k, v, scale, bias, KINDS[kind], variant)
        err = np.abs(got - want).max()
        print(f'norm={norm} gamma={gamma} kind={kind} variant={variant}: error {err:.3g}, '
              f'reference algorithm in fp32 {ref_err:.3g}', flush=True)
        assert err <= 2 * ref_err + 1e-5


def _long_key_cases(kind):
    """Long key axes through each of the tile kernel's paths: (name, inputs,
    split_weights flag, number of leading queries on the fast pass)."""
    q, k, v, scale, bias = _long_keys(1, kind)
    item = km.TILE_ITEM_ROWS[64]
    far = q.clone()
    far[..., item:, :] += 1.5
    far = far.to(KINDS[kind]).float()  # the model takes the inputs the kernel sees
    yield 'fast', (q, k, v, scale, bias), False, q.shape[2]
    yield 'second_item_below_the_guard', (far, k, v, scale, bias), False, item
    yield 'large_gamma', (q, k, v, torch.tensor(0.3), bias), False, 0
    yield 'few_live_keys', _concentrated(16, 16, kind), False, 0
    yield 'bound_edge', _concentrated(0, 380, kind), False, 0
    yield 'split_flag', (q, k, v, scale, bias), True, 0
    # Values 16 times larger: abandoned at the course check.
    yield 'values_x16', (q, k, (v * 16).to(KINDS[kind]).float(), scale, bias), False, 0
    # Large values past the course check only: the final check sends it on.
    late = v.clone()
    late[..., 640:, :] *= 64
    yield 'late_large_values', (q, k, late.to(KINDS[kind]).float(), scale, bias), False, 0
    if kind == 'bf16':
        big = v.clone()
        big[..., 7, 3] = 2.0 ** 17
        yield 'value_beyond_fp16', (q, k, big, scale, bias), False, 0


@pytest.mark.parametrize('kind', sorted(KINDS))
def test_the_tile_kernel_follows_the_model_on_long_keys(kind):
    for name, (q, k, v, scale, bias), split, n_fast in _long_key_cases(kind):
        print(f'long keys: case={name} kind={kind} split_weights={split}', flush=True)
        want, path = km.run('tile', q, k, v, scale, bias, kind, split_weights=split)
        fast = (path[0, 0] == km.FAST)
        assert fast[:n_fast].all() and not fast[n_fast:].any(), name
        got = _kernel(q, k, v, scale, bias, KINDS[kind], 'tile', split_weights=split)
        np.testing.assert_allclose(got, want, err_msg=name, **MODEL_TOL)


@pytest.mark.parametrize('kind', sorted(KINDS))
def test_the_default_long_key_path_holds_the_gate_at_any_value_scale(kind):
    """Config 4's q, k and gamma range on one plane of its 4096 keys, with
    the values scaled by 1, 16 and 256: the default path (the fast pass where
    its bound allows, the split otherwise) stays inside the 1e-3 / 1e-4 gate
    against fp64, and follows the model's choice of path."""
    for v_scale in (1.0, 16.0, 256.0):
        for gamma in (0.005, 0.05):
            q, k, v, scale, bias = _config4_plane(7 + int(v_scale), kind, gamma, v_scale)
            print(f'config-4 plane: kind={kind} gamma={gamma} values x{v_scale:g}', flush=True)
            want, path = km.run('tile', q, k, v, scale, bias, kind)
            assert (path == (km.FAST if v_scale == 1.0 else km.SPLIT)).all()
            got = _kernel(q, k, v, scale, bias, KINDS[kind], 'tile')
            np.testing.assert_allclose(got, want, **MODEL_TOL)
            exact = oracle.expanded_fp64(q, k, v, scale, bias)
            np.testing.assert_allclose(got, exact, rtol=1e-3, atol=1e-4)
