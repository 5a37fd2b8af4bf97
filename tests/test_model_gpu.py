"""The price model compiled with the `vectra` backend on the GPU (config 5).

Every spatial-attention site is rewritten to torch.ops.vectra.rbf_attention
(the HIP kernels) and the compiled model matches eager: tightly against the
same model run eagerly in the same precision, and within bf16 accuracy
against the eager fp32 model.
"""

import pytest
import torch

from vectra_amd.compiler import backend
from vectra_amd.kernels import _native
from vectra_amd.price_transformer import model as model_lib

pytestmark = pytest.mark.gpu


class Autocast(torch.nn.Module):
    """Runs the wrapped model under torch.autocast(bfloat16)."""

    def __init__(self, inner):
        super().__init__()
        self.inner = inner

    def forward(self, *inputs):
        with torch.autocast('cuda', dtype=torch.bfloat16):
            return self.inner(*inputs)


def _config(layers):
    return model_lib.ModelConfig(d_model=128, num_heads=8, num_layers=layers, attribute_dim=16,
                                 ffn_dim=256, num_candidates=64)


@pytest.fixture(autouse=True)
def _fresh_dynamo():
    torch._dynamo.reset()  # pylint: disable=protected-access
    yield
    torch._dynamo.reset()  # pylint: disable=protected-access


@pytest.mark.timeout(900)
@pytest.mark.parametrize('layers', [3, 4])
def test_autocast_model_has_every_site_on_the_hip_operator(layers):
    config = _config(layers)
    torch.manual_seed(0)
    model = model_lib.PriceTransformer(config).eval().cuda()
    # Config 5's own batch: 1024 subjects x 64 comparables.
    inputs = tuple(model_lib.box_inputs(config, 1024, device='cuda', seed=0))
    wrapped = Autocast(model)
    compiled, report = backend.compile_for_serving(wrapped, inputs, expected_sites=layers)
    print(f'layers={layers} report={report}', flush=True)
    assert report.sites == layers and report.graph_break_count == 0
    assert all(name.endswith('[autocast]') for name in report.matches), report.matches
    assert _native.HIP_LIBRARY in _native.loaded_libraries()
    with torch.no_grad():
        fresh = tuple(model_lib.box_inputs(config, 1024, device='cuda', seed=1))
        got = compiled(*fresh)
        same_precision = wrapped(*fresh)
        fp32 = model(*fresh)
    assert got.dtype == torch.float32
    # The fused operator is more accurate than autocast's eager chain (it does
    # not round the difference tensor or the weights to bf16), so the two
    # differ by bf16 rounding of the attention, not more.  The sites
    # themselves are checked against the oracle at rtol 1e-3 / atol 1e-4 in
    # test_model_sites_gpu.py.
    torch.testing.assert_close(got, same_precision, rtol=0, atol=3e-2)
    torch.testing.assert_close(got, fp32, rtol=0, atol=5e-2)


@pytest.mark.timeout(900)
def test_bf16_blocks_are_rewritten_and_match():
    config = _config(3)
    torch.manual_seed(0)
    model = model_lib.PriceTransformer(config).eval().cuda()
    inputs = tuple(model_lib.box_inputs(config, 256, device='cuda', seed=2))
    with torch.no_grad():
        fp32 = model(*inputs)
    model.set_block_dtype(torch.bfloat16)
    compiled, report = backend.compile_for_serving(model, inputs, expected_sites=3)
    assert report.matches == {'rbf_divisor_bias_softmax[half]': 3}
    with torch.no_grad():
        got = compiled(*inputs)
        eager_bf16 = model(*inputs)
    torch.testing.assert_close(got, eager_bf16, rtol=0, atol=3e-2)
    torch.testing.assert_close(got, fp32, rtol=0, atol=5e-2)


@pytest.mark.timeout(900)
def test_deployment_bundle_on_the_gpu(tmp_path):
    # Export, reload and serve with the reference's GPU default (float16
    # blocks): the numerics gate (rtol 1e-3 vs the eager model in the same
    # precision) runs on the HIP operator at export and again at load.
    from vectra_amd.export import compile_entry
    from vectra_amd.price_transformer import checkpoint

    config = _config(3)
    torch.manual_seed(0)
    model = model_lib.PriceTransformer(config).eval()
    checkpoint.save(str(tmp_path / 'ckpt'), model)
    spec = compile_entry.ServingSpec('cuda', batch_size=64, block_dtype='float16')
    manifest = compile_entry.export_bundle(str(tmp_path / 'ckpt'), str(tmp_path / 'bundle'), spec,
                                           numerics_batches=2)
    print(f"manifest compile={manifest['compile']} numerics={manifest['numerics']}", flush=True)
    assert manifest['compile']['sites'] == 3 and manifest['compile']['graph_break_count'] == 0
    assert manifest['numerics']['max_abs_error_vs_eager'] < 1.4e-2
    torch._dynamo.reset()  # pylint: disable=protected-access
    serving = compile_entry.load_bundle(str(tmp_path / 'bundle'))
    assert _native.HIP_LIBRARY in _native.loaded_libraries()
    eager = compile_entry.prepare(checkpoint.load(str(tmp_path / 'ckpt')), spec)
    for count in (1, 64, 100):
        inputs = model_lib.example_inputs(config, count, seed=70 + count)
        got = serving.predict(inputs)
        with torch.no_grad():
            want = eager(*inputs.to('cuda')).float()
        assert got.shape == (count,)
        torch.testing.assert_close(got, want, rtol=1e-3, atol=1e-3)
