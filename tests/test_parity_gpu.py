"""Parity of the HIP kernels with the oracle, through the C ABI (GPU).

Gates (from the operator's acceptance targets):
* bf16 / fp16 inputs: the fp32 output of the kernel within rtol 1e-3 /
  atol 1e-4 of the eager chain evaluated in fp32 on the same rounded inputs;
* fp32 inputs: within rtol 1e-5 (atol 1e-6) of the float64 oracle.
The operator itself returns v.dtype; its output must be exactly the kernel's
fp32 result rounded once (test_operator_output_is_the_rounded_fp32_result).
"""

import math
import zlib

import numpy as np
import pytest
import torch

from oracle import rbf as oracle
from tests import _golden
from tests.half_cases import HALF_CASES, HALF_KERNEL_SHAPES, half_case as _half_case
from vectra_amd.benchmarks import configs
from vectra_amd.kernels import _native
from vectra_amd.kernels import capi
from vectra_amd.kernels import custom_ops  # noqa: F401  (registers the op)

pytestmark = pytest.mark.gpu

HALF_TOL = {'rtol': 1e-3, 'atol': 1e-4}
FP32_TOL = {'rtol': 1e-5, 'atol': 1e-6}


def _cuda(t):
    return None if t is None else t.cuda()


def _variants(q, k, v, scale, bias):
    """Every variant the library accepts for these inputs, plus 'auto'."""
    q, k, v, scale = _cuda(q), _cuda(k), _cuda(v), _cuda(scale)
    bias = _cuda(bias)
    scale4, bias4 = capi.broadcast_operands(q, k, scale, bias)
    out = torch.empty((*q.shape[:-1], v.shape[-1]), device='cuda')
    found = ['auto']
    for name in ('generic', 'stream', 'mfma', 'plane', 'tile'):
        if capi.select_variant(capi.make_args(q, k, v, out, scale4, bias4, name)) > 0:
            found.append(name)
    return found


def run(q, k, v, scale, bias=None, variant='auto', out_dtype=torch.float32, split_weights=False):
    out = capi.forward(_cuda(q), _cuda(k), _cuda(v), _cuda(scale), _cuda(bias),
                       out_dtype=out_dtype, variant=variant, split_weights=split_weights)
    torch.cuda.synchronize()
    return out.cpu()


def _golden_params():
    params = []
    for name, case in sorted(_golden.cases().items()):
        args = (case['q'], case['k'], case['v'], case['scale'], case['bias'])
        if torch.cuda.is_available():
            variants = _variants(*args)
        else:
            variants = ['auto']
        params += [(name, variant) for variant in variants]
    return params


@pytest.mark.parametrize('name,variant', _golden_params())
def test_golden_fixtures(name, variant):
    case = _golden.cases()[name]
    print(f'golden case={name} variant={variant}', flush=True)
    got = run(case['q'], case['k'], case['v'], case['scale'], case['bias'], variant)
    want = case['expected'].numpy()
    if case['dtype'] == torch.float32:
        tol = {'rtol': 1e-4, 'atol': 1e-4} if name == 'far_points' else FP32_TOL
    else:
        tol = HALF_TOL
    np.testing.assert_allclose(got.double().numpy(), want, equal_nan=True, **tol)


# (config, batch subset for the oracle)
CONFIG_CASES = [
    (configs.CPU_EAGER, None),
    (configs.SERVING, None),
    (configs.SELF_ATTENTION, 48),
    (configs.SELF_ATTENTION.with_dtype(torch.float32), 48),
    (configs.SERVING.with_dtype(torch.float16), 128),
]


@pytest.mark.parametrize('config,batch', CONFIG_CASES, ids=lambda c: getattr(c, 'name', str(c)))
def test_config_parity(config, batch):
    inputs = configs.make_inputs(config, seed=0, batch=batch)
    for variant in _variants(*inputs.args()):
        print(f'config={config.name} batch={batch} variant={variant}', flush=True)
        got = run(*inputs.args(), variant=variant).double().numpy()
        if config.dtype == torch.float32:
            want = oracle.direct_fp64(*inputs.args())
            np.testing.assert_allclose(got, want, **FP32_TOL)
        else:
            want = oracle.eager_fp32(*inputs.args(), batch_chunk=16).double().numpy()
            np.testing.assert_allclose(got, want, **HALF_TOL)


def test_long_key_rows_against_the_expansion():
    # Config 4's full key axis (4096) for a slice of query rows and planes.
    config = configs.LONG_KEY
    gen = torch.Generator().manual_seed(0)
    q = (0.5 * torch.randn(2, 16, 24, 64, generator=gen)).bfloat16()
    k = (0.5 * torch.randn(2, 16, 4096, 64, generator=gen)).bfloat16()
    v = torch.randn(2, 16, 4096, 64, generator=gen).bfloat16()
    scale = 0.005 + 0.045 * torch.rand(1, 16, 1, 1, generator=gen)
    assert config.head_dim == 64
    want = oracle.expanded_fp64(q, k, v, scale)
    for variant in _variants(q, k, v, scale, None):
        for split in (False, True):  # the tile kernel's fp16-weight pass, then the split kept
            print(f'long_key slice variant={variant} split_weights={split}', flush=True)
            got = run(q, k, v, scale, None, variant, split_weights=split).double().numpy()
            np.testing.assert_allclose(got, want, **HALF_TOL)


@pytest.mark.parametrize('n_q', [1, 17, 255, 257, 300])
@pytest.mark.parametrize('dim', [32, 64])
def test_long_keys_with_partial_work_items(n_q, dim):
    # Query counts around the tile kernel's work items (128 rows for 32-dim
    # heads, 256 for 64-dim), on a key axis long enough for its fp16-weight
    # pass: the default output, both head-dim kernels, against the expansion.
    gen = torch.Generator().manual_seed(n_q * 3 + dim)
    q = (0.5 * torch.randn(1, 2, n_q, dim, generator=gen)).bfloat16()
    k = (0.5 * torch.randn(1, 2, 1100, dim, generator=gen)).bfloat16()
    v = (0.25 * torch.randn(1, 2, 1100, dim, generator=gen)).bfloat16()
    scale = torch.tensor([0.02, 0.04]).reshape(1, 2, 1, 1)
    want = oracle.expanded_fp64(q, k, v, scale)
    print(f'long keys n_q={n_q} dim={dim}', flush=True)
    got = run(q, k, v, scale, None, 'tile').double().numpy()
    np.testing.assert_allclose(got, want, **HALF_TOL)


def test_operator_output_is_the_rounded_fp32_result():
    inputs = configs.make_inputs(configs.SERVING, seed=1).to('cuda')
    out = torch.ops.vectra.rbf_attention(*inputs.args())
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16 and out.is_cuda and out.is_contiguous()
    fp32 = capi.forward(*inputs.args(), out_dtype=torch.float32)
    assert torch.equal(out, fp32.to(torch.bfloat16))
    loaded = _native.loaded_libraries()
    assert _native.HIP_LIBRARY in loaded and _native.TORCH_LIBRARY in loaded


@pytest.mark.parametrize('config', [configs.SERVING, configs.SELF_ATTENTION], ids=lambda c: c.name)
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16], ids=str)
def test_every_variant_rounds_its_fp32_result_once(config, dtype):
    """A 16-bit output is the kernel's fp32 result rounded once (no fused
    multiply-convert), for every variant that runs the shape."""
    inputs = configs.make_inputs(config.with_dtype(dtype), seed=3, batch=64).to('cuda')
    for variant in _variants(*inputs.args()):
        print(f'config={config.name} dtype={dtype} variant={variant}', flush=True)
        fp32 = capi.forward(*inputs.args(), out_dtype=torch.float32, variant=variant)
        half = capi.forward(*inputs.args(), out_dtype=dtype, variant=variant)
        torch.cuda.synchronize()
        assert torch.equal(half, fp32.to(dtype)), variant


def test_full_serving_size_properties():
    config = configs.SERVING
    inputs = configs.make_inputs(config, seed=2).to('cuda')
    q, k, v, scale, bias = inputs.args()
    base = capi.forward(q, k, v, scale, bias, out_dtype=torch.float32)
    # Rows are independent: a sub-batch reproduces its rows bit for bit.
    part = capi.forward(q[100:300], k[100:300], v[100:300], scale, bias[100:300],
                        out_dtype=torch.float32)
    assert torch.equal(part, base[100:300])
    # Key order does not matter (up to fp32 summation order).
    perm = torch.randperm(config.n_k, generator=torch.Generator().manual_seed(0)).cuda()
    permuted = capi.forward(q, k[:, :, perm], v[:, :, perm], scale, bias[..., perm],
                            out_dtype=torch.float32)
    torch.testing.assert_close(permuted, base, rtol=1e-5, atol=1e-6)
    # A constant added to every key's bias changes nothing.
    shifted = capi.forward(q, k, v, scale, bias.float() + 2.5, out_dtype=torch.float32)
    torch.testing.assert_close(shifted, base, rtol=1e-5, atol=1e-6)
    # Outputs are convex combinations of the live values.
    live = torch.isfinite(bias.float())[:, :, 0, :, None]  # [B,1,Nk,1]
    vf = v.float()
    lo = torch.where(live, vf, torch.inf).amin(2, keepdim=True)
    hi = torch.where(live, vf, -torch.inf).amax(2, keepdim=True)
    assert bool(((base >= lo - 1e-5) & (base <= hi + 1e-5)).all())
    # The bf16 operator output is the rounded fp32 one.
    assert torch.equal(torch.ops.vectra.rbf_attention(q, k, v, scale, bias), base.to(torch.bfloat16))


def test_full_long_key_size_properties():
    """Config 4 at its full size (16 x 16 planes of 4096 x 4096, D = 64),
    through properties the operator must have whatever the size."""
    inputs = configs.make_inputs(configs.LONG_KEY, seed=4).to('cuda')
    q, k, v, scale, bias = inputs.args()
    assert bias is None
    base = capi.forward(q, k, v, scale, None, out_dtype=torch.float32)
    # Scaling V by a power of two scales every output exactly with the split
    # weights.
    split = capi.forward(q, k, v, scale, None, out_dtype=torch.float32, split_weights=True)
    split2 = capi.forward(q, k, v * 2, scale, None, out_dtype=torch.float32, split_weights=True)
    assert torch.equal(split2, split * 2)
    # The default path keeps the fp16-weight pass per work item where its
    # error bound (which grows with |v|) fits the absolute allowance, so at
    # 2V more items take the split: every output at 2V is then either twice
    # the split's, or twice the default's at V (where both kept the fast pass;
    # bf16 values below 2^-14 round to fp16's subnormal steps of 2^-24, so to
    # that step and an ulp of the output).
    doubled = capi.forward(q, k, v * 2, scale, None, out_dtype=torch.float32)
    from_split = doubled == split2
    from_fast = torch.isclose(doubled, base * 2, rtol=2.0 ** -22, atol=2.0 ** -22)
    assert bool((from_split | from_fast).all())
    print(f'fast pass kept at V: {(base != split).float().mean().item():.3f} of outputs, '
          f'at 2V: {(~from_split).float().mean().item():.3f}', flush=True)
    # The default and the split agree within the gate: the fp16 weights'
    # rounding errors add up like a random walk of ~2^-12 / sqrt(3 sum) of
    # the values' spread (sums of 400-3500 weights here: ~2e-5 at most over
    # the 67M outputs), and the kernel keeps the fast result only where four
    # times its bound on that walk fits the gate.
    torch.testing.assert_close(base, split, **HALF_TOL)
    torch.testing.assert_close(doubled, split2, **HALF_TOL)
    # Planes and query rows are independent: a sub-batch of planes and a
    # permutation of the query rows reproduce their outputs.
    part = capi.forward(q[3:5, 7:9], k[3:5, 7:9], v[3:5, 7:9], scale[:, 7:9], None, out_dtype=torch.float32)
    torch.testing.assert_close(part, base[3:5, 7:9], rtol=1e-6, atol=1e-7)
    perm = torch.randperm(q.shape[2], generator=torch.Generator().manual_seed(1)).cuda()
    permuted = capi.forward(q[:, :, perm], k, v, scale, None, out_dtype=torch.float32)
    torch.testing.assert_close(permuted, base[:, :, perm], rtol=1e-6, atol=1e-7)
    # Outputs are convex combinations of each plane's values.
    vf = v.float()
    lo, hi = vf.amin(2, keepdim=True), vf.amax(2, keepdim=True)
    assert bool(((base >= lo - 1e-5) & (base <= hi + 1e-5)).all())
    assert bool(torch.isfinite(base).all())


def test_variants_agree_at_full_self_attention_size():
    inputs = configs.make_inputs(configs.SELF_ATTENTION, seed=3).to('cuda')
    results = {}
    for variant in _variants(*inputs.args()):
        if variant == 'generic':
            continue  # slow at this size; covered at reduced size above
        results[variant] = capi.forward(*inputs.args(), out_dtype=torch.float32, variant=variant)
    ref = results.pop('auto')
    # The MFMA kernel feeds P to the second product as a 16-bit hi + lo pair
    # (~2^-17 relative), the stream kernel in fp32: they agree to ~1e-5.
    for variant, out in results.items():
        err = (out - ref).abs().max().item()
        torch.testing.assert_close(out, ref, rtol=1e-4, atol=2e-5, msg=f'{variant}: max |diff| {err}')


# --- Edge shapes and values (kernels/tests/test_edges.py:37-114). ----------


def _check(q, k, v, scale, bias=None, tol=None):
    want = oracle.expanded_fp64(q, k, v, scale, bias)
    for variant in _variants(q, k, v, scale, bias):
        got = run(q, k, v, scale, bias, variant).double().numpy()
        np.testing.assert_allclose(got, want, equal_nan=True, err_msg=variant, **(tol or FP32_TOL))


@pytest.mark.parametrize('n_q,n_k', [(1, 1), (1, 65), (17, 3), (63, 65), (65, 63), (129, 1), (130, 200)])
def test_tails_not_multiple_of_tiles(n_q, n_k):
    gen = torch.Generator().manual_seed(n_q * 1000 + n_k)
    q = torch.randn(2, 3, n_q, 32, generator=gen)
    k = torch.randn(2, 3, n_k, 32, generator=gen)
    v = torch.randn(2, 3, n_k, 32, generator=gen)
    _check(q, k, v, torch.tensor(0.02))
    _check(q.bfloat16(), k.bfloat16(), v.bfloat16(), torch.tensor(0.02), tol=HALF_TOL)


@pytest.mark.parametrize('dim,value_dim', [(8, 8), (16, 16), (48, 48), (64, 64), (80, 24), (100, 128),
                                           (128, 7), (128, 128), (300, 300)])
def test_head_dims(dim, value_dim):
    gen = torch.Generator().manual_seed(dim)
    q = torch.randn(1, 2, 40, dim, generator=gen)
    k = torch.randn(1, 2, 70, dim, generator=gen)
    v = torch.randn(1, 2, 70, value_dim, generator=gen)
    _check(q, k, v, torch.tensor(1.0 / (4.0 * dim)), tol={'rtol': 1e-5, 'atol': 2e-6})
    _check(q.half(), k.half(), v.half(), torch.tensor(1.0 / (4.0 * dim)), tol=HALF_TOL)


def test_all_but_one_key_masked():
    gen = torch.Generator().manual_seed(5)
    q = torch.randn(3, 2, 9, 16, generator=gen)
    k = torch.randn(3, 2, 70, 16, generator=gen)
    v = torch.randn(3, 2, 70, 16, generator=gen)
    bias = torch.full((3, 1, 1, 70), -math.inf)
    bias[..., 0] = 0.0
    for variant in _variants(q, k, v, torch.tensor(0.05), bias):
        out = run(q, k, v, torch.tensor(0.05), bias, variant)
        torch.testing.assert_close(out, v[:, :, :1].expand_as(out), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize('n_k', [20, 64, 130])
def test_fully_masked_rows_are_nan(n_k):
    q, k, v = torch.randn(2, 1, 4, 16), torch.randn(2, 1, n_k, 16), torch.randn(2, 1, n_k, 16)
    bias = torch.zeros(2, 1, 1, n_k)
    bias[1] = -math.inf
    for variant in _variants(q, k, v, torch.tensor(0.1), bias):
        out = run(q, k, v, torch.tensor(0.1), bias, variant)
        assert torch.isnan(out[1]).all() and torch.isfinite(out[0]).all(), variant


# (Nq, Nk, D): the stream kernel (one query row), the plane kernel (both axes
# one tile, D = 32 and 16), streamed key tiles; fp32 reaches the MFMA kernel.
MASKED_ROW_SHAPES = [(1, 64, 32), (65, 65, 32), (24, 70, 16), (40, 200, 32)]


@pytest.mark.parametrize('shape', MASKED_ROW_SHAPES, ids=str)
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32], ids=str)
def test_non_finite_values_in_masked_rows_propagate(shape, dtype):
    """A key masked by a -inf bias still reaches the output through 0 * x:
    NaN in its K row makes every output of the query row NaN, and inf or NaN
    in its V row makes that value dim NaN, as in the eager chain.  Kernels
    that skip the products of masked key blocks must keep these."""
    n_q, n_k, dim = shape
    gen = torch.Generator().manual_seed(11)
    q = torch.randn(3, 2, n_q, dim, generator=gen)
    k = torch.randn(3, 2, n_k, dim, generator=gen)
    v = torch.randn(3, 2, n_k, dim, generator=gen)
    bias = torch.zeros(3, 1, 1, n_k)
    bias[..., n_k // 2:] = -math.inf  # a masked suffix, as padding gives
    k[0, 1, n_k - 1, 3] = math.nan
    v[1, 0, n_k - 2, 5] = math.inf
    v[1, 1, n_k // 2, 7] = math.nan
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    scale = torch.tensor(0.05)
    want = oracle.expanded_fp64(q, k, v, scale, bias)
    assert np.isnan(want[0, 1]).all() and np.isfinite(want[0, 0]).all() and np.isfinite(want[2]).all()
    assert np.isnan(want[1, 0, :, 5]).all() and np.isnan(want[1, 1, :, 7]).all()
    assert np.isfinite(np.delete(want[1, 0], 5, axis=-1)).all()
    tol = FP32_TOL if dtype == torch.float32 else HALF_TOL
    for variant in _variants(q, k, v, scale, bias):
        print(f'shape={shape} dtype={dtype} variant={variant}', flush=True)
        got = run(q, k, v, scale, bias, variant).double().numpy()
        np.testing.assert_allclose(got, want, equal_nan=True, err_msg=variant, **tol)


@pytest.mark.parametrize('shape', [(65, 65, 32), (24, 70, 16), (33, 128, 16), (40, 64, 32)], ids=str)
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16, torch.float32], ids=str)
def test_skipped_masked_blocks_are_bit_exact(shape, dtype):
    """The plane kernels skip the products of 16-key blocks (and the fp32
    kernel its tail keys) whose keys are all masked with finite K and V
    rows.  A finite bias of -1e30 masks the same keys (their weights are
    exactly 0) but keeps their blocks, so the two give bit-identical outputs."""
    n_q, n_k, dim = shape
    gen = torch.Generator().manual_seed(12)
    q = torch.randn(4, 2, n_q, dim, generator=gen).to(dtype)
    k = torch.randn(4, 2, n_k, dim, generator=gen).to(dtype)
    v = torch.randn(4, 2, n_k, dim, generator=gen).to(dtype)
    counts = torch.tensor([1, n_k, 17, n_k // 2])  # live keys per batch entry
    masked = (torch.arange(n_k)[None, :] >= counts[:, None])[:, None, None, :]
    skip_bias = torch.zeros(4, 1, 1, n_k).masked_fill(masked, -math.inf)
    keep_bias = torch.zeros(4, 1, 1, n_k).masked_fill(masked, -1e30)
    scale = torch.tensor(0.04)
    for out_dtype in (dtype, torch.float32):
        print(f'shape={shape} dtype={dtype} out={out_dtype}', flush=True)
        skipped = run(q, k, v, scale, skip_bias, 'plane', out_dtype=out_dtype)
        kept = run(q, k, v, scale, keep_bias, 'plane', out_dtype=out_dtype)
        assert torch.equal(skipped, kept)
    want = oracle.expanded_fp64(q, k, v, scale, skip_bias)
    tol = FP32_TOL if dtype == torch.float32 else HALF_TOL
    np.testing.assert_allclose(skipped.double().numpy(), want, **tol)  # the fp32 output


def test_far_points_do_not_underflow():
    gen = torch.Generator().manual_seed(6)
    q = torch.randn(2, 2, 10, 32, generator=gen) * 20
    k = torch.randn(2, 2, 50, 32, generator=gen) * 20
    v = torch.randn(2, 2, 50, 32, generator=gen)
    _check(q, k, v, torch.tensor(0.1), tol={'rtol': 1e-4, 'atol': 1e-4})


@pytest.mark.parametrize('scale', [0.0, -0.01, 3.0])
def test_degenerate_and_negative_scales(scale):
    gen = torch.Generator().manual_seed(7)
    q = torch.randn(1, 2, 12, 16, generator=gen)
    k = torch.randn(1, 2, 30, 16, generator=gen)
    v = torch.randn(1, 2, 30, 16, generator=gen)
    _check(q, k, v, torch.tensor(scale), tol={'rtol': 1e-5, 'atol': 1e-5})


def test_head_transposed_views_and_per_head_bias():
    gen = torch.Generator().manual_seed(8)
    projected = torch.randn(4, 65, 3 * 4 * 32, generator=gen)
    for dtype in (torch.float32, torch.bfloat16):
        proj = projected.to(dtype).cuda()
        q, k, v = (t.view(4, 65, 4, 32).transpose(1, 2) for t in proj.split(4 * 32, dim=-1))
        assert not q.is_contiguous()
        bias = torch.zeros(4, 4, 1, 65)
        bias[1, 2, 0, 40:] = -math.inf
        _check(q, k, v, torch.full((1, 4, 1, 1), 0.02), bias,
               tol=FP32_TOL if dtype == torch.float32 else HALF_TOL)


@pytest.mark.parametrize('bias_dtype', [torch.float32, torch.float16, torch.bfloat16, torch.float64])
@pytest.mark.parametrize('scale_dtype', [torch.float32, torch.bfloat16, torch.float64])
def test_bias_and_scale_dtypes(bias_dtype, scale_dtype):
    gen = torch.Generator().manual_seed(9)
    q, k, v = (torch.randn(2, 3, n, 32, generator=gen) for n in (2, 40, 40))
    scale = (0.02 + 0.05 * torch.rand(2, 3, 1, 1, generator=gen)).to(scale_dtype)
    bias = torch.randn(2, 1, 1, 40, generator=gen).to(bias_dtype)
    bias[0, ..., 30:] = -math.inf
    _check(q, k, v, scale.float(), bias.double(), tol=FP32_TOL)  # oracle on converted values
    for variant in _variants(q, k, v, scale, bias):
        got = run(q, k, v, scale, bias, variant).double().numpy()
        want = oracle.expanded_fp64(q, k, v, scale.float(), bias.float())
        np.testing.assert_allclose(got, want, **FP32_TOL)


@pytest.mark.parametrize('n_q', [1, 40])
@pytest.mark.parametrize('bias_dtype', [torch.float16, torch.bfloat16])
def test_two_byte_bias_planes_at_any_alignment(bias_dtype, n_q):
    # An odd key count puts every other (b, h) plane of a 2-byte bias at an
    # address = 2 (mod 4); a view one element into a buffer does the same for
    # the base pointer.  The kernels read biases as aligned 32-bit words.
    gen = torch.Generator().manual_seed(13)
    batch, heads, n_k = 3, 2, 41
    q = torch.randn(batch, heads, n_q, 32, generator=gen).bfloat16()
    k = torch.randn(batch, heads, n_k, 32, generator=gen).bfloat16()
    v = torch.randn(batch, heads, n_k, 32, generator=gen).bfloat16()
    flat = (2.0 * torch.randn(batch * heads * n_k + 1, generator=gen)).to(bias_dtype)
    flat[::7] = -math.inf
    flat_gpu = flat.cuda()
    for offset in (0, 1):
        bias_gpu = flat_gpu[offset:offset + batch * heads * n_k].view(batch, heads, 1, n_k)
        assert (bias_gpu.data_ptr() % 4 == 0) == (offset == 0)
        bias = flat[offset:offset + batch * heads * n_k].view(batch, heads, 1, n_k)
        want = oracle.expanded_fp64(q, k, v, torch.tensor(0.05), bias.float())
        for variant in _variants(q, k, v, torch.tensor(0.05), bias):
            got = capi.forward(q.cuda(), k.cuda(), v.cuda(), torch.tensor(0.05).cuda(), bias_gpu,
                               out_dtype=torch.float32, variant=variant)
            np.testing.assert_allclose(got.cpu().double().numpy(), want, err_msg=f'{variant} offset {offset}',
                                       **HALF_TOL)


# Shapes that reach the 16-bit query-tile kernels: one plane tile per wave
# (head dims 16 and 32, <= 80 rows) and streamed key tiles (more keys, or
# 64-dim heads).
@pytest.mark.parametrize('case', HALF_CASES)
@pytest.mark.parametrize('shape', sorted(HALF_KERNEL_SHAPES))
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16], ids=str)
def test_16bit_edge_cases(case, shape, dtype):
    """Edge cases through the 16-bit kernels, including their exact-maximum
    passes (far queries, gamma < 0, biases, fully masked rows)."""
    n_q, n_k, dim = HALF_KERNEL_SHAPES[shape]
    gen = torch.Generator().manual_seed(zlib.crc32(f'{case}/{shape}'.encode()) % 1000)
    q, k, v, scale, bias = _half_case(case, n_q, n_k, dim, gen)
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    want = oracle.expanded_fp64(q, k, v, scale, bias)
    variants = _variants(q, k, v, scale, bias)
    assert ('plane' if shape.startswith('plane') else 'tile') in variants, variants
    for variant in variants:
        print(f'case={case} shape={shape} dtype={dtype} variant={variant}', flush=True)
        got = run(q, k, v, scale, bias, variant).double().numpy()
        np.testing.assert_allclose(got, want, equal_nan=True, err_msg=variant, **HALF_TOL)


def test_empty_key_set_gives_zeros():
    q = torch.randn(1, 2, 3, 32)
    k, v = torch.empty(1, 2, 0, 32), torch.empty(1, 2, 0, 32)
    for variant in _variants(q, k, v, torch.tensor(0.1), None):
        assert torch.equal(run(q, k, v, torch.tensor(0.1), None, variant), torch.zeros(1, 2, 3, 32))


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16, torch.float32], ids=str)
@pytest.mark.parametrize('dim', [16, 32, 64, 128])
def test_every_variant_over_a_grid_of_shapes(dtype, dim):
    """Every variant that accepts the shape, over key and query counts on
    both sides of the kernels' tile, slot and wave-count boundaries (1, 16,
    17, 64, 65, 80, 81, 129 keys; 1, 16, 65, 81, 127 queries), against the
    float64 chain at the dtype's gate."""
    gen = torch.Generator().manual_seed(dim)
    tol = FP32_TOL if dtype == torch.float32 else HALF_TOL
    for n_k in (1, 16, 17, 64, 65, 80, 81, 129):
        for n_q in (1, 16, 65, 81, 127):
            q = (0.5 * torch.randn(2, 3, n_q, dim, generator=gen)).to(dtype)
            k = (0.5 * torch.randn(2, 3, n_k, dim, generator=gen)).to(dtype)
            v = torch.randn(2, 3, n_k, dim, generator=gen).to(dtype)
            scale = torch.tensor(0.5 / dim)
            want = oracle.direct_fp64(q, k, v, scale)
            for variant in _variants(q, k, v, scale, None):
                print(f'grid dtype={dtype} dim={dim} n_k={n_k} n_q={n_q} variant={variant}', flush=True)
                got = run(q, k, v, scale, None, variant).double().numpy()
                np.testing.assert_allclose(got, want, err_msg=f'{variant} n_k={n_k} n_q={n_q}', **tol)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16])
@pytest.mark.parametrize('n_q,n_k', [(81, 65), (127, 65), (127, 80), (200, 80), (80, 65), (127, 64), (127, 81)])
def test_mfma_variant_64_dim_heads_around_80_keys(dtype, n_q, n_k):
    """The MFMA kernel at 64-dim 16-bit heads, key axes of 64 to 81 and query
    counts on both sides of five 16-row tiles (where the launch changes its
    wave count and key tile), every output against the float64 chain."""
    gen = torch.Generator().manual_seed(n_q * 1000 + n_k)
    q, k, v = (torch.randn(2, 4, n, 64, generator=gen).to(dtype) for n in (n_q, n_k, n_k))
    scale = torch.tensor(0.5 / 64)
    want = oracle.direct_fp64(q, k, v, scale)
    np.testing.assert_allclose(run(q, k, v, scale, variant='mfma').double().numpy(), want, **HALF_TOL)


@pytest.mark.parametrize('n_q,n_k', [(1, 64), (65, 65), (100, 100)])
def test_key_rows_walked_backwards(n_q, n_k):
    """Negative key-row strides (K, V and the bias addressed from their last
    key row), which the ABI accepts: the result is that of the reversed keys,
    from the kernel with signed 64-bit addressing (the shapes are the stream,
    plane and tile kernels' with forward strides)."""
    gen = torch.Generator().manual_seed(21 + n_k)
    q = torch.randn(2, 4, n_q, 32, generator=gen).to(torch.bfloat16)
    k = torch.randn(2, 4, n_k, 32, generator=gen).to(torch.bfloat16)
    v = torch.randn(2, 4, n_k, 32, generator=gen).to(torch.bfloat16)
    bias = torch.randn(2, 1, 1, n_k, generator=gen)
    scale = torch.tensor(0.05)
    want = oracle.direct_fp64(q, k.flip(2), v.flip(2), scale, bias.flip(3))
    qd, kd, vd, sd, bd = (x.cuda() for x in (q, k, v, scale, bias))
    scale4, bias4 = capi.broadcast_operands(qd, kd, sd, bd)
    out = torch.full((2, 4, n_q, 32), float('nan'), device='cuda')
    a = capi.make_args(qd, kd, vd, out, scale4, bias4)
    a.k, a.v = kd[:, :, n_k - 1].data_ptr(), vd[:, :, n_k - 1].data_ptr()
    a.k_stride[2], a.v_stride[2] = -kd.stride(2), -vd.stride(2)
    a.key_bias, a.bias_stride_n = bias4[:, :, :, n_k - 1].data_ptr(), -bias4.stride(3)
    assert capi.VARIANT_NAMES[capi.select_variant(a)] == 'generic'
    capi.launch(a)
    torch.cuda.synchronize()
    np.testing.assert_allclose(out.cpu().double().numpy(), want, **HALF_TOL)


def test_operator_with_a_cpu_scalar_scale_and_outputs_in_every_dtype():
    gen = torch.Generator().manual_seed(10)
    q, k, v = (torch.randn(2, 3, n, 32, generator=gen) for n in (4, 50, 50))
    want = oracle.expanded_fp64(q, k, v, torch.tensor(0.03))
    for dtype in (torch.float32, torch.float16, torch.bfloat16):
        out = torch.ops.vectra.rbf_attention(q.to('cuda', dtype), k.to('cuda', dtype),
                                             v.to('cuda', dtype), torch.tensor(0.03))
        assert out.dtype == dtype
        ref = oracle.expanded_fp64(q.to(dtype), k.to(dtype), v.to(dtype), torch.tensor(0.03))
        np.testing.assert_allclose(out.double().cpu().numpy(), ref, rtol=1e-2, atol=1e-2)
    assert want.shape == (2, 3, 4, 32)


def test_squared_norms():
    gen = torch.Generator().manual_seed(12)
    x = torch.randn(3, 4, 77, 40, generator=gen)
    for dtype in (torch.float32, torch.float16, torch.bfloat16):
        xd = x.to('cuda', dtype).transpose(1, 2).contiguous().transpose(1, 2)  # strided
        got = capi.squared_norms(xd).cpu()
        want = (x.to(dtype).double() ** 2).sum(-1)
        np.testing.assert_allclose(got.double().numpy(), want.numpy(), rtol=1e-5, atol=1e-5)


GRAPH_CASES = [(configs.SERVING, 256, 'stream'), (configs.SELF_ATTENTION, 64, 'plane'),
               (configs.SELF_ATTENTION.with_dtype(torch.float32), 64, 'plane'), (configs.LONG_KEY, 1, 'tile')]


@pytest.mark.parametrize('config,batch,kernel', GRAPH_CASES,
                         ids=lambda c: f'{c.name}-{c.dtype}'.replace('torch.', '') if hasattr(c, 'name') else str(c))
def test_graph_replays_match_eager(config, batch, kernel):
    """Graph replays of the operator (the stream, plane, fp32 plane and tile
    kernels) give the eager result on every replay."""
    inputs = configs.make_inputs(config, seed=4, batch=batch).to('cuda')
    eager = torch.ops.vectra.rbf_attention(*inputs.args())
    q, k, v, scale, bias = inputs.args()
    scale4, bias4 = capi.broadcast_operands(q, k, scale, bias)
    chosen = capi.select_variant(capi.make_args(q, k, v, eager, scale4, bias4, 'auto'))
    assert capi.VARIANT_NAMES[chosen] == kernel
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(2):
            torch.ops.vectra.rbf_attention(*inputs.args())
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = torch.ops.vectra.rbf_attention(*inputs.args())
    for i in range(4):
        static_out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_out, eager), f'replay {i}'
        torch.ops.vectra.rbf_attention(*inputs.args())  # eager work between replays
        torch.cuda.synchronize()


# --- A seeded sweep over the operator's input space. -------------------------

def _sweep_cases(count=48):
    """(seed, n_q, n_k, dim, value_dim, dtype, bias kind, layout) drawn from a
    fixed seed, so the sweep is the same on every run."""
    rng = np.random.default_rng(20261202)
    n_qs = [1, 2, 5, 15, 16, 17, 33, 64, 65, 80, 81, 130]
    n_ks = [1, 7, 16, 31, 64, 65, 80, 81, 128, 129, 200, 257]
    dims = [8, 16, 32, 48, 64, 128]
    dtypes = [torch.bfloat16, torch.float16, torch.float32]
    cases = []
    for i in range(count):
        dim = int(rng.choice(dims))
        value_dim = dim if rng.random() < 0.75 else int(rng.choice(dims))
        cases.append((i, int(rng.choice(n_qs)), int(rng.choice(n_ks)), dim, value_dim,
                      dtypes[int(rng.integers(3))], ['none', 'ragged', 'per_head'][int(rng.integers(3))],
                      ['contiguous', 'transposed'][int(rng.integers(2))]))
    return cases


@pytest.mark.parametrize('case', _sweep_cases(), ids=lambda c: '-'.join(str(x).replace('torch.', '') for x in c))
def test_seeded_sweep(case):
    """Random shapes, dtypes, masks and layouts through every variant that
    accepts them, against the float64 oracle."""
    seed, n_q, n_k, dim, value_dim, dtype, bias_kind, layout = case
    gen = torch.Generator().manual_seed(1000 + seed)
    batch, heads = 2, 3
    if layout == 'transposed':
        # Head-transposed views of one [B, N, H * 3 * D] projection, as the model's sites.
        def project(n, d):
            return torch.randn(batch, n, heads * d, generator=gen).view(batch, n, heads, d).transpose(1, 2)
        q, k, v = project(n_q, dim), project(n_k, dim), project(n_k, value_dim)
    else:
        q = torch.randn(batch, heads, n_q, dim, generator=gen)
        k = torch.randn(batch, heads, n_k, dim, generator=gen)
        v = torch.randn(batch, heads, n_k, value_dim, generator=gen)
    scale = 0.5 / dim + 0.2 / dim * torch.rand(1, heads, 1, 1, generator=gen)
    bias = None
    if bias_kind == 'ragged':
        bias = torch.zeros(batch, 1, 1, n_k)
        bias[0, ..., max(1, n_k // 2):] = -math.inf
    elif bias_kind == 'per_head':
        bias = torch.randn(batch, heads, 1, n_k, generator=gen)
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    if bias is not None:
        bias = bias.to(dtype)
    want = oracle.expanded_fp64(q, k, v, scale, bias)
    tol = FP32_TOL if dtype == torch.float32 else HALF_TOL
    for variant in _variants(q, k, v, scale, bias):
        print(f'sweep case={case} variant={variant}', flush=True)
        got = run(q, k, v, scale, bias, variant).double().numpy()
        np.testing.assert_allclose(got, want, equal_nan=True, err_msg=variant, **tol)


def _strided_copy(small, strides, device='cuda'):
    """`small` placed in a large zeroed buffer under the given element strides
    (a view whose offsets need more than 32 bits)."""
    span = 1 + sum((n - 1) * s for n, s in zip(small.shape, strides))
    big = torch.zeros(span, dtype=small.dtype, device=device)
    view = big.as_strided(small.shape, strides)
    view.copy_(small.to(device))
    return view


def test_offsets_beyond_32_bits():
    """Keys 1 GB apart inside a plane (per-lane 32-bit offsets would wrap: the
    kernels that use them must decline), and planes 4 GB apart (64-bit plane
    bases), against the float64 oracle."""
    gen = torch.Generator().manual_seed(32)
    q = torch.randn(2, 2, 3, 32, generator=gen).bfloat16()
    k = torch.randn(2, 2, 3, 32, generator=gen).bfloat16()
    v = torch.randn(2, 2, 3, 32, generator=gen).bfloat16()
    scale = torch.tensor(0.05)
    want = oracle.expanded_fp64(q, k, v, scale)
    # Keys 2^29 elements (1 GB of bf16) apart within each plane.
    far_keys = _strided_copy(k, (6 * 32, 3 * 32, 1 << 29, 1))
    variants = _variants(q, far_keys, v, scale, None)
    assert 'stream' not in variants, variants
    for variant in variants:
        got = run(q, far_keys, v, scale, None, variant).double().numpy()
        np.testing.assert_allclose(got, want, err_msg=f'far keys {variant}', **HALF_TOL)
    del far_keys
    # Batch entries 2^31 elements (4 GB) apart; each plane itself is compact.
    far_planes = _strided_copy(v, (1 << 31, 3 * 32, 32, 1))
    variants = _variants(q, k, far_planes, scale, None)
    assert 'stream' in variants, variants
    for variant in variants:
        got = run(q, k, far_planes, scale, None, variant).double().numpy()
        np.testing.assert_allclose(got, want, err_msg=f'far planes {variant}', **HALF_TOL)
    del far_planes
    torch.cuda.empty_cache()


# fp32 planes: key counts with 0-4 keys past a whole 16-key block (those keys
# take the VALU in the fp32 plane kernel, key blocks past Nk are skipped) and
# more than 4 (a block of products), with and without a masked tail key.
FP32_TAIL_CASES = [(n_q, n_k, dim) for n_q in (16, 65) for n_k in (1, 2, 4, 5, 17, 20, 33, 36, 64, 65, 68)
                   for dim in (16, 32)]


@pytest.mark.parametrize('shape', FP32_TAIL_CASES, ids=str)
def test_fp32_plane_tail_keys(shape):
    n_q, n_k, dim = shape
    gen = torch.Generator().manual_seed(31 + n_k + 7 * n_q + dim)
    q = torch.randn(2, 3, n_q, dim, generator=gen)
    k = torch.randn(2, 3, n_k, dim, generator=gen)
    v = torch.randn(2, 3, n_k, dim, generator=gen)
    scale = torch.full((1, 3, 1, 1), 1.0 / dim)
    bias = torch.zeros(2, 1, 1, n_k)
    if n_k > 1:
        bias[1, ..., n_k - 1] = -math.inf  # the last (tail) key masked in one batch entry
        bias[0, ..., 0] = 0.75
    variants = _variants(q, k, v, scale, bias)
    assert 'plane' in variants, variants
    print(f'shape={shape}', flush=True)
    _check(q, k, v, scale, bias)
    # Negative gamma (the shifted second pass, tail keys included) and a
    # fully masked row.
    _check(q, k, v, -scale, bias)
    masked = bias.clone()
    masked[0] = -math.inf
    got = run(q, k, v, scale, masked, 'plane')
    assert torch.isnan(got[0]).all() and torch.isfinite(got[1]).all()


def test_fp32_plane_large_values_do_not_overflow():
    """Queries on top of keys with gamma*|q|^2 = 60: the fp32 plane kernel's
    unshifted weight for the matching key is e^60 (about 2^87), and with
    |v| near 2^50 the unshifted value products would pass fp32's 2^128.  The
    kernel must take its max-subtracted pass for such queries and return v of
    the matching key, as the float64 oracle does."""
    gen = torch.Generator().manual_seed(53)
    b, h, n, dim = 2, 3, 65, 32
    gamma = 1.0 / dim
    k = torch.randn(b, h, n, dim, generator=gen, dtype=torch.float64)
    k = k / k.norm(dim=-1, keepdim=True) * math.sqrt(60.0 / gamma)
    k = k.float()
    q = k.clone()
    v = (torch.randn(b, h, n, dim, generator=gen) * 2.0 ** 50).float()
    scale = torch.full((1, h, 1, 1), gamma)
    assert 'plane' in _variants(q, k, v, scale, None)
    got = run(q, k, v, scale, None, 'plane').double()
    assert torch.isfinite(got).all()
    want = oracle.direct_fp64(q, k, v, scale)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-5, atol=0)


# Preallocated outputs under strides the operator's callers hand in: heads
# inside rows (a [B, Nq, H, Dv] buffer viewed as [B, H, Nq, Dv]), every other
# element, and rows one element longer than Dv (unaligned rows).
OUT_LAYOUTS = ('heads_inner', 'every_other', 'odd_rows')
OUT_LAYOUT_SHAPES = [(1, 64, 32, torch.bfloat16), (65, 65, 16, torch.bfloat16), (65, 65, 32, torch.float16),
                     (65, 65, 32, torch.float32), (40, 200, 32, torch.bfloat16), (40, 100, 64, torch.float32),
                     (20, 70, 128, torch.bfloat16), (20, 70, 48, torch.bfloat16)]


def _out_view(layout, b, h, n_q, dv, dtype, sentinel):
    if layout == 'heads_inner':
        buf = torch.full((b, n_q, h, dv), sentinel, dtype=dtype, device='cuda')
        return buf, buf.permute(0, 2, 1, 3)
    if layout == 'every_other':
        buf = torch.full((b, h, n_q, 2 * dv), sentinel, dtype=dtype, device='cuda')
        return buf, buf[..., ::2]
    buf = torch.full((b, h, n_q, dv + 1), sentinel, dtype=dtype, device='cuda')
    return buf, buf[..., :dv]


@pytest.mark.parametrize('layout', OUT_LAYOUTS)
@pytest.mark.parametrize('shape', OUT_LAYOUT_SHAPES, ids=str)
def test_preallocated_strided_outputs(shape, layout):
    """Every variant that accepts the output view writes exactly the values
    it writes into a contiguous output, and nothing outside the view."""
    n_q, n_k, dim, dtype = shape
    gen = torch.Generator().manual_seed(41 + n_q + n_k + dim)
    b, h = 3, 4
    q = torch.randn(b, h, n_q, dim, generator=gen).to(dtype).cuda()
    k = torch.randn(b, h, n_k, dim, generator=gen).to(dtype).cuda()
    v = torch.randn(b, h, n_k, dim, generator=gen).to(dtype).cuda()
    scale = torch.full((1, h, 1, 1), 1.0 / dim, device='cuda')
    bias = torch.zeros(b, 1, 1, n_k, device='cuda')
    for i in range(b):
        bias[i, ..., n_k - i:] = -math.inf  # ragged key counts
    bias[0, ..., 0] = 0.5
    scale4, bias4 = capi.broadcast_operands(q, k, scale, bias)
    sentinel = 7.0
    checked = set()
    for out_dtype in {torch.float32, dtype}:
        buf, view = _out_view(layout, b, h, n_q, dim, out_dtype, sentinel)
        for variant in ('auto', 'generic', 'stream', 'mfma', 'plane', 'tile'):
            chosen = capi.select_variant(capi.make_args(q, k, v, view, scale4, bias4, variant))
            if chosen <= 0:
                continue
            checked.add(variant)
            print(f'shape={shape} layout={layout} out={out_dtype} variant={variant}', flush=True)
            buf.fill_(sentinel)
            # 'auto' against the kernel it picks for this view (a contiguous
            # output may pick another one).
            want = capi.forward(q, k, v, scale, bias, out_dtype=out_dtype, variant=capi.VARIANT_NAMES[chosen])
            capi.forward(q, k, v, scale, bias, out=view, variant=variant)
            torch.cuda.synchronize()
            assert torch.equal(view, want), variant
            rest = buf.clone()
            rest.as_strided(view.shape, view.stride()).fill_(sentinel)
            assert rest.eq(sentinel).all(), f'{variant} wrote outside the view'
    # Query blocks of 16-, 32-, 64- and 128-dim heads reach a matrix-core
    # kernel under every layout; single queries reach the stream kernel only
    # under 16-byte aligned rows.
    if (n_q >= 16 and dim != 48) or (layout == 'heads_inner' and n_q == 1):
        assert checked - {'auto', 'generic'}, checked
