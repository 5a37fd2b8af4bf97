"""Batched prediction (CPU): request assembly into a staging slot, padding,
and the per-request outputs, with an eager model behind a stand-in for the
GPU feeder (same host-side interface: next_slot / launch / finish)."""

import pytest
import torch

from vectra_amd.price_transformer import model as model_lib
from vectra_amd.serving import predict

CONFIG = model_lib.ModelConfig(d_model=32, num_heads=4, num_layers=1, attribute_dim=5, ffn_dim=64,
                               num_candidates=16)


class _HostFeeder:
    """The DeviceFeeder's host-side contract, running `model` eagerly."""

    def __init__(self, model, batch_size):
        self.batch_size = batch_size
        self.model = model
        example = model_lib.example_inputs(CONFIG, batch_size)
        self.host = model_lib.PricingInputs(*(torch.full_like(t, 7) for t in example))
        self.launched = []

    def next_slot(self):
        return 0, self.host

    def launch(self, slot, rows):
        for t in self.host:
            t[rows:].copy_(t[rows - 1:rows].expand(self.batch_size - rows, *t.shape[1:]))
        with torch.no_grad():
            out = self.model(*self.host).float()
        self.launched.append(model_lib.PricingInputs(*(t.clone() for t in self.host)))
        return out[:rows]

    def finish(self, handle):
        return handle


@pytest.fixture(scope='module')
def model():
    torch.manual_seed(0)
    return model_lib.PriceTransformer(CONFIG).eval()


@pytest.mark.parametrize('rows', [1, 5, 8])
def test_requests_are_assembled_and_padded(model, rows):
    batch = model_lib.example_inputs(CONFIG, rows, seed=3)
    feeder = _HostFeeder(model, 8)
    got = predict.Predictor(feeder, CONFIG.min_candidates)(predict.request_rows(batch))
    staged = feeder.launched[0]
    for field, want in zip(staged, batch):
        assert torch.equal(field[:rows], want)
        assert torch.equal(field[rows:], want[-1:].expand(8 - rows, *want.shape[1:]))
    padded = model_lib.PricingInputs(*(torch.cat([t, t[-1:].expand(8 - rows, *t.shape[1:])]) for t in batch))
    with torch.no_grad():
        want = model(*padded).float()[:rows]
    assert [p.log_price for p in got] == want.tolist()
    used = predict.comparables_used(batch, CONFIG.min_candidates)
    assert [p.candidates_used for p in got] == used.tolist()


def test_batch_size_limits(model):
    predictor = predict.Predictor(_HostFeeder(model, 4), CONFIG.min_candidates)
    with pytest.raises(ValueError):
        predictor([])
    with pytest.raises(ValueError):
        predictor(predict.request_rows(model_lib.example_inputs(CONFIG, 5)))


def test_comparables_used_counts_the_trimmed_set():
    batch = model_lib.example_inputs(CONFIG, 6, seed=4)
    valid = batch.cand_valid.clone()
    valid[0, 3:] = False
    radius = batch.radius_km.clone()
    radius[1] = 1e-6  # nothing inside: the nearest min_candidates are kept
    batch = batch._replace(cand_valid=valid, radius_km=radius)
    used = predict.comparables_used(batch, CONFIG.min_candidates)
    assert used[0] <= 3
    assert used[1] == CONFIG.min_candidates
    assert (used <= batch.cand_valid.sum(-1)).all()
