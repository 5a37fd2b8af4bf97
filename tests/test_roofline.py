"""The analytic traffic and FLOP model (CPU).

Known answers: the per-config budgets restated from the reference's
kernels/benchmarks/roofline.py:87-139 formulas (fused_bytes, eager_bytes,
fused_flops) at every benchmark configuration, and the reference's own
harness check (benchmark/harness_test.py:244-252).  The byte budget is also
pinned against the tensors the benchmarks actually allocate.
"""

import pytest
import torch

from vectra_amd.benchmarks import configs
from vectra_amd.benchmarks import roofline

# (config, dtype) -> fused bytes, reference FLOPs, matrix FLOPs, eager bytes
KNOWN = {
    ('cpu_eager', torch.float32): (1_089_552, 843_776, 524_288, 3_514_368),
    ('serving', torch.bfloat16): (68_288_544, 104_333_312, 67_108_864, 212_992_000),
    ('self_attention', torch.bfloat16): (136_448_032, 4_706_058_240, 4_430_233_600, 9_689_139_200),
    ('self_attention', torch.float32): (272_896_032, 4_706_058_240, 4_430_233_600, 19_378_278_400),
    ('long_key', torch.bfloat16): (537_002_048, 1_125_549_867_008, 1_099_511_627_776, 2_285_459_603_456),
}


def _shape(name, dtype):
    c = configs.CONFIGS[name]
    return (c if c.dtype == dtype else c.with_dtype(dtype)).shape()


@pytest.mark.parametrize('key', sorted(KNOWN, key=str))
def test_budgets_at_every_configuration(key):
    s = _shape(*key)
    fused, flops, matrix, eager = KNOWN[key]
    assert roofline.fused_bytes(s) == fused
    assert roofline.fused_flops(s) == flops
    assert roofline.matrix_flops(s) == matrix
    assert sum(roofline.eager_bytes(s).values()) == eager


def test_serving_eager_chain_by_operator():
    by_op = roofline.eager_bytes(configs.SERVING.shape())
    assert by_op == {
        'sub': 67_633_152, 'pow': 67_108_864, 'sum': 34_603_008, 'neg': 2_097_152,
        'scale': 2_097_152, 'bias': 2_228_224, 'softmax': 2_097_152, 'bmm': 35_127_296,
    }
    # Per subject query: q, k, v and out of 8 heads plus the bias row.
    assert roofline.fused_bytes(configs.SERVING.shape()) / 1024 == 8 * (64 + 4096 + 4096 + 64) + 128 + 32 / 1024


@pytest.mark.parametrize('name', ['cpu_eager', 'serving', 'self_attention'])
def test_fused_bytes_are_the_allocated_operands(name):
    """q, k, v, scale and bias as the benchmarks allocate them, plus the
    output: the budget the kernels are measured against."""
    c = configs.CONFIGS[name]
    inputs = configs.make_inputs(c)
    out_bytes = inputs.q.shape[0] * inputs.q.shape[1] * inputs.q.shape[2] * inputs.v.shape[-1] * inputs.v.element_size()
    scale_bytes = c.heads * 4  # the model budgets one fp32 coefficient per head
    held = inputs.nbytes() - inputs.scale.numel() * inputs.scale.element_size() + scale_bytes
    assert roofline.fused_bytes(c.shape()) == held + out_bytes


def test_long_key_budget_counts_a_bias_row_it_does_not_have():
    s = configs.LONG_KEY.shape()
    inputs = configs.make_inputs(configs.LONG_KEY, batch=1)
    assert inputs.key_bias is None
    operands = 4 * s.batch * s.heads * s.n_q * s.head_dim * s.element_bytes
    assert roofline.fused_bytes(s) == operands + s.batch * s.n_k * s.element_bytes + s.heads * 4


def test_reference_harness_traffic_model():
    """harness_test.py:244-252 at its own shape (B=64, H=4, Lq=Lk=65, D=32,
    16-bit): the fused kernel moves under 2 % of the eager chain's bytes and
    stays below the ridge point; the B=1024 working set does not fit one
    XCD's L2 (nor would it fit the reference GPU's 50 MB L2)."""
    small = roofline.analyze(roofline.Shape(64, 4, 65, 65, 32, 32, 2))
    assert small['bytes_ratio'] < 0.02
    assert small['fused_is_memory_bound']
    big = roofline.Shape(1024, 4, 65, 65, 32, 32, 2)
    assert roofline.fused_bytes(big) > roofline.MI355X.l2_bytes_per_xcd
    assert roofline.fused_bytes(big) > 50 * 2**20


def test_placement_of_each_configuration():
    for name in ('cpu_eager', 'serving', 'self_attention'):
        assert roofline.analyze(configs.CONFIGS[name].shape())['fused_is_memory_bound'], name
    long_key = roofline.analyze(configs.LONG_KEY.shape())
    assert not long_key['fused_is_memory_bound']
    assert long_key['fused_intensity_flop_per_byte'] > roofline.MI355X.ridge_flop_per_byte
    # The serving floor at 8 TB/s.
    assert roofline.analyze(configs.SERVING.shape())['fused_hbm_floor_us'] == pytest.approx(8.536, abs=1e-3)
