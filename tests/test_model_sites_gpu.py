"""The config-5 model's attention sites at their own shape, against the oracle (GPU).

The price model (d_model 128, 8 heads of 16 dims, 3 blocks, 1024 subjects x
64 comparables + the subject = 65 tokens) is run eagerly with a hook on each
block's SpatialAttention.  Each site's operands are rebuilt exactly as the
compiled graph hands them to vectra::rbf_attention
(models/price_transformer/spatial_attention.py:68-88 of the reference):

* q, k, v: head-transposed views of the qkv projection's output (rows of
  16 elements, 3 * 128 elements apart), in the block precision, not copied;
* the coefficient 1 / (2 sigma^2) per head ([1, H, 1, 1]; the rewrite turns
  the divisor into a reciprocal), in the parameters' dtype;
* the key bias [B, 1, 1, 65] in the block dtype, -inf for padded comparables.

The kernel's fp32 output on those operands must lie within rtol 1e-3 /
atol 1e-4 of the eager chain evaluated in fp32 on the same values
(oracle.eager_fp32), for every row of every site: bf16 under autocast,
fp16 blocks and bf16 blocks.
"""

import numpy as np
import pytest
import torch

from oracle import rbf as oracle
from vectra_amd.kernels import capi
from vectra_amd.kernels import custom_ops  # noqa: F401  (registers the op)
from vectra_amd.price_transformer import model as model_lib

pytestmark = pytest.mark.gpu

BATCH = 1024
CONFIG = model_lib.ModelConfig(d_model=128, num_heads=8, num_layers=3, attribute_dim=16, ffn_dim=256,
                               num_candidates=64)


def _inputs(seed):
    """Config-5 inputs with ragged valid comparables (8 to 64 per subject)."""
    inputs = model_lib.box_inputs(CONFIG, BATCH, seed=seed)
    gen = torch.Generator().manual_seed(seed + 1)
    counts = torch.randint(8, CONFIG.num_candidates + 1, (BATCH,), generator=gen)
    valid = torch.arange(CONFIG.num_candidates)[None, :] < counts[:, None]
    return inputs._replace(cand_valid=valid).to('cuda')


def _site_operands(attention, x, key_bias, autocast):
    """q, k, v, coefficient and bias of one site, as the compiled graph has them."""
    batch, tokens, width = x.shape
    with torch.no_grad(), torch.autocast('cuda', dtype=torch.bfloat16, enabled=autocast):
        qkv = attention.qkv(x)
        q, k, v = (t.view(batch, tokens, attention.num_heads, attention.head_dim).transpose(1, 2)
                   for t in qkv.split(width, dim=-1))
        coefficient = torch.reciprocal(2 * attention.log_sigma.exp() ** 2)
    return q, k, v, coefficient, key_bias


@pytest.mark.timeout(600)
@pytest.mark.parametrize('precision', ['autocast_bf16', 'float16_blocks', 'bfloat16_blocks'])
def test_every_site_of_the_model_matches_the_oracle(precision):
    torch.manual_seed(0)
    model = model_lib.PriceTransformer(CONFIG).eval().cuda()
    autocast = precision == 'autocast_bf16'
    if not autocast:
        model.set_block_dtype(getattr(torch, precision.split('_')[0]))
    captured = []
    hooks = [block.attention.register_forward_pre_hook(
        lambda module, args: captured.append((module, args[0].detach(), args[1].detach())))
        for block in model.blocks]
    try:
        with torch.no_grad(), torch.autocast('cuda', dtype=torch.bfloat16, enabled=autocast):
            model(*_inputs(seed=3))
    finally:
        for hook in hooks:
            hook.remove()
    assert len(captured) == CONFIG.num_layers
    for site, (attention, x, key_bias) in enumerate(captured):
        q, k, v, coefficient, bias = _site_operands(attention, x, key_bias, autocast)
        assert q.shape == (BATCH, 8, 65, 16) and not q.is_contiguous() and q.stride(2) == 3 * 128
        assert bias.shape == (BATCH, 1, 1, 65) and torch.isinf(bias).any()
        scale4, bias4 = capi.broadcast_operands(q, k, coefficient, bias)
        out = torch.empty(q.shape, device='cuda')
        variant = capi.VARIANT_NAMES[capi.select_variant(capi.make_args(q, k, v, out, scale4, bias4))]
        print(f'{precision} site {site}: q {q.dtype} coefficient {coefficient.dtype} bias {bias.dtype} '
              f'kernel {variant}', flush=True)
        assert variant == 'plane'
        got = capi.forward(q, k, v, coefficient, bias, out_dtype=torch.float32)
        torch.cuda.synchronize()
        want = oracle.eager_fp32(q.cpu(), k.cpu(), v.cpu(), coefficient.cpu(), bias.cpu(), batch_chunk=64)
        np.testing.assert_allclose(got.cpu().double().numpy(), want.double().numpy(), rtol=1e-3, atol=1e-4)
        # The operator returns v.dtype: the same result rounded once.
        op = torch.ops.vectra.rbf_attention(q, k, v, coefficient, bias)
        assert torch.equal(op, got.to(op.dtype))
