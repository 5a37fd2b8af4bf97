"""The price model harness around the attention sites (CPU).

The behaviours the reference's model tests hold (models/tests/test_model.py:
35-86), checked with this repository's own inputs and assertions:

* one finite float32 log price per request, and each request's price
  depends on that request alone;
* comparables marked invalid never reach the prediction, whatever they hold,
  and the order of the comparables does not matter;
* the radius trim keeps each subject's valid comparables inside its radius,
  and a subject with none inside keeps its `min_keep` nearest valid ones
  (held against a per-row restatement of that rule, since the trim here is
  branch-free where the reference branches with torch.cond);
* Transformer blocks in bf16 or fp16 track the float32 model.
"""

import numpy as np
import pytest
import torch

from vectra_amd.price_transformer import model as model_lib

CONFIG = model_lib.ModelConfig(embedding_dim=24, attribute_dim=7, d_model=48, num_heads=4, num_layers=3,
                               ffn_dim=96, num_candidates=20, min_candidates=3)


@pytest.fixture(name='model')
def _model():
    torch.manual_seed(11)
    return model_lib.PriceTransformer(CONFIG).eval()


def _inputs(batch, seed=5):
    # Comparables spread over a 6 km box; radii of 2.5 km and 0.3 km in
    # turn, so some subjects have comparables inside and some fall back to
    # their nearest.
    inputs = model_lib.box_inputs(CONFIG, batch, seed=seed, box_km=6.0)
    return inputs._replace(radius_km=torch.tensor([2.5, 0.3]).repeat(batch)[:batch])


def test_one_finite_price_per_request_from_that_request_alone(model):
    inputs = _inputs(6)
    with torch.no_grad():
        prices = model(*inputs)
        alone = [model(*(t[i:i + 1] for t in inputs)) for i in range(6)]
    assert prices.shape == (6,) and prices.dtype == torch.float32
    assert torch.isfinite(prices).all()
    assert prices.unique().numel() == 6
    torch.testing.assert_close(torch.cat(alone), prices, rtol=1e-6, atol=1e-5)


def test_invalid_comparables_never_reach_the_prediction(model):
    inputs = _inputs(5, seed=8)
    gen = torch.Generator().manual_seed(2)
    valid = torch.rand(5, CONFIG.num_candidates, generator=gen) < 0.6
    valid[:, :CONFIG.min_candidates] = True
    inputs = inputs._replace(cand_valid=valid)
    junk = ~valid
    noisy = inputs._replace(
        cand_embedding=torch.where(junk[..., None], -inputs.cand_embedding, inputs.cand_embedding),
        cand_attributes=torch.where(junk[..., None], 1e3 * torch.randn(inputs.cand_attributes.shape, generator=gen),
                                    inputs.cand_attributes),
        cand_log_price=torch.where(junk, torch.full_like(inputs.cand_log_price, -250.0), inputs.cand_log_price),
        cand_sale_day=torch.where(junk, inputs.cand_sale_day - 1e5, inputs.cand_sale_day),
        cand_location=torch.where(junk[..., None], inputs.query_location[:, None, :] + 0.001,
                                  inputs.cand_location),
        cand_cell6=torch.where(junk, inputs.query_cell6[:, None], inputs.cand_cell6),
    )
    with torch.no_grad():
        torch.testing.assert_close(model(*noisy), model(*inputs), rtol=0, atol=0)


def test_the_order_of_the_comparables_does_not_matter(model):
    inputs = _inputs(4, seed=13)
    perm = torch.randperm(CONFIG.num_candidates, generator=torch.Generator().manual_seed(4))
    shuffled = inputs._replace(**{
        name: getattr(inputs, name)[:, perm]
        for name in model_lib.PricingInputs._fields if name.startswith('cand_')
    })
    with torch.no_grad():
        torch.testing.assert_close(model(*shuffled), model(*inputs), rtol=1e-6, atol=1e-5)


def _trim_per_row(distance, radius, valid, min_keep):
    """The trim's rule, row by row: the valid comparables inside the radius
    (distance <= radius); with none inside, the min_keep nearest valid ones
    (all of them if fewer)."""
    out = np.zeros(distance.shape, dtype=bool)
    for b in range(distance.shape[0]):
        live = [j for j in range(distance.shape[1]) if valid[b, j]]
        inside = [j for j in live if distance[b, j] <= radius[b]]
        keep = inside if inside else sorted(live, key=lambda j: distance[b, j])[:min_keep]
        out[b, keep] = True
    return out


def test_the_trim_follows_its_rule_on_random_rows():
    gen = torch.Generator().manual_seed(21)
    for trial in range(30):
        rows, cands, min_keep = 9, int(torch.randint(4, 17, (1,), generator=gen)), 1 + trial % 5
        distance = 12 * torch.rand(rows, cands, generator=gen)
        radius = 3 * torch.rand(rows, generator=gen)
        valid = torch.rand(rows, cands, generator=gen) < 0.7
        valid[0] = False                       # no valid comparable at all
        valid[1] = False
        valid[1, :2] = True                    # fewer valid than min_keep, none inside
        radius[1] = 0.0
        distance[2, 3] = radius[2]             # exactly on the radius: inside
        valid[2, 3] = True
        got = model_lib.trim_to_radius(distance, radius, valid, min_keep)
        want = _trim_per_row(distance.numpy(), radius.numpy(), valid.numpy(), min_keep)
        np.testing.assert_array_equal(got.numpy(), want, err_msg=f'trial {trial}')


def test_the_trim_on_named_rows():
    distance = torch.tensor([[3.0, 0.2, 4.5, 9.9, 1.1],
                             [8.0, 2.5, 7.0, 0.9, 6.0],
                             [0.4, 5.0, 0.3, 5.5, 0.2]])
    radius = torch.tensor([4.0, 0.5, 1.0])
    valid = torch.tensor([[True, True, True, True, False],
                          [True, True, True, True, True],
                          [True, True, True, True, False]])
    mask = model_lib.trim_to_radius(distance, radius, valid, min_keep=2).tolist()
    assert mask[0] == [True, True, False, False, False]   # inside 4 km; 1.1 km is invalid
    assert mask[1] == [False, True, False, True, False]   # nothing inside 0.5 km: the 2 nearest
    assert mask[2] == [True, False, True, False, False]   # inside 1 km; 0.2 km is invalid


@pytest.mark.parametrize('dtype,atol', [(torch.bfloat16, 2e-2), (torch.float16, 1e-2)])
def test_reduced_precision_blocks_track_float32(model, dtype, atol):
    inputs = _inputs(16, seed=30)
    with torch.no_grad():
        want = model(*inputs)
        assert model.set_block_dtype(dtype) is model
        got = model(*inputs)
        model.set_block_dtype(torch.float32)
    assert got.dtype == torch.float32
    assert all(p.dtype == dtype for p in model.set_block_dtype(dtype).blocks.parameters())
    assert all(p.dtype == torch.float32 for p in model.head.parameters())
    err = (got - want).abs().max().item()
    assert 0 < err <= atol, err
