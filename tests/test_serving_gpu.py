"""The serving path on the GPU: pinned multi-slot staging, batched
prediction and the pipelined batcher, all feeding the price model compiled
with the `vectra` backend (every attention site on the HIP operator).

The staged path must give exactly the compiled model's outputs on the same
(padded) batch: it only moves the inputs, so the bar is bit equality.
"""

import asyncio

import pytest
import torch

from vectra_amd.export import compile_entry
from vectra_amd.kernels import _native
from vectra_amd.price_transformer import model as model_lib
from vectra_amd.serving import batcher as batcher_lib
from vectra_amd.serving import feeder as feeder_lib
from vectra_amd.serving import predict

pytestmark = pytest.mark.gpu

BATCH = 128


@pytest.fixture(scope='module')
def compiled():
    torch._dynamo.reset()  # pylint: disable=protected-access
    config = model_lib.ModelConfig(d_model=128, num_heads=8, num_layers=3, attribute_dim=16,
                                   ffn_dim=256, num_candidates=64)
    spec = compile_entry.ServingSpec('cuda', BATCH, 'float16')
    torch.manual_seed(0)
    model = compile_entry.prepare(model_lib.PriceTransformer(config), spec)
    fn, report, _ = compile_entry.compile_model(model, spec)
    assert report.sites == 3
    assert _native.HIP_LIBRARY in _native.loaded_libraries()
    yield fn, config
    torch._dynamo.reset()  # pylint: disable=protected-access


def _host_batch(config, n, seed):
    return model_lib.box_inputs(config, n, device='cpu', seed=seed)


def _padded(batch, size):
    n = batch[0].shape[0]
    return model_lib.PricingInputs(*(torch.cat([t, t[-1:].expand(size - n, *t.shape[1:])]) for t in batch))


def _direct(fn, batch):
    """The compiled model on the batch padded to BATCH, first n rows."""
    n = batch[0].shape[0]
    with torch.no_grad():
        out = fn(*_padded(batch, BATCH).to('cuda')).float().cpu()
    return out[:n]


@pytest.mark.timeout(900)
@pytest.mark.parametrize('graph', [False, True], ids=['launches', 'graph'])
@pytest.mark.parametrize('rows', [BATCH, 1, 77])
def test_staged_batches_match_the_compiled_model(compiled, rows, graph):
    fn, config = compiled
    feeder = feeder_lib.DeviceFeeder(fn, _host_batch(config, BATCH, 0), slots=2, graph=graph)
    batch = _host_batch(config, rows, seed=10 + rows)
    print(f'rows={rows} graph={graph}', flush=True)
    assert torch.equal(feeder.run(batch), _direct(fn, batch))


@pytest.mark.timeout(900)
@pytest.mark.parametrize('graph', [False, True], ids=['launches', 'graph'])
def test_batches_in_flight_together_match_one_at_a_time(compiled, graph):
    """Several rounds over both slots (each graph replayed several times),
    with the model also run eagerly on other inputs between launches."""
    fn, config = compiled
    feeder = feeder_lib.DeviceFeeder(fn, _host_batch(config, BATCH, 0), slots=2, graph=graph)
    sizes = [BATCH, 50, BATCH, 3, BATCH, 100, 7]
    batches = [_host_batch(config, n, seed=20 + i) for i, n in enumerate(sizes)]
    want = [_direct(fn, b) for b in batches]
    other = _host_batch(config, BATCH, seed=99).to('cuda')
    got, pending = [], []
    for batch in batches:
        if len(pending) == feeder.slots:
            got.append(feeder.finish(pending.pop(0)))
        pending.append(feeder.launch(*feeder.stage(batch)))
        with torch.no_grad():
            fn(*other)  # eager work between replays
    got += [feeder.finish(h) for h in pending]
    for i, (g, w) in enumerate(zip(got, want)):
        assert torch.equal(g, w), i


def test_a_slot_in_flight_is_not_reused(compiled):
    fn, config = compiled
    feeder = feeder_lib.DeviceFeeder(fn, _host_batch(config, BATCH, 0), slots=1)
    handle = feeder.launch(*feeder.stage(_host_batch(config, 4, 1)))
    with pytest.raises(RuntimeError):
        feeder.stage(_host_batch(config, 4, 2))
    feeder.finish(handle)
    with pytest.raises(ValueError):
        feeder.stage(_host_batch(config, BATCH + 1, 3))


@pytest.mark.timeout(900)
def test_pipelined_batcher_serves_every_request(compiled):
    fn, config = compiled
    feeder = feeder_lib.DeviceFeeder(fn, _host_batch(config, BATCH, 0), slots=2, graph=True)
    predictor = predict.Predictor(feeder, config.min_candidates)
    batch = _host_batch(config, 300, seed=30)
    requests = predict.request_rows(batch)
    used = predict.comparables_used(batch, config.min_candidates)

    async def scenario():
        b = batcher_lib.Batcher(max_batch_size=BATCH, window_s=0.005, launch=predictor.launch,
                                finish=predictor.finish, depth=feeder.slots)
        b.start()
        try:
            return await asyncio.gather(*(b.submit(r) for r in requests))
        finally:
            await b.close()

    results = asyncio.run(scenario())
    sizes = [r.batch_size for r in results]
    assert max(sizes) == BATCH and sum(1 for s in sizes if s == BATCH) >= 2 * BATCH
    # Each prediction is the compiled model's output for its request, whatever
    # batch it shared (the model is row-independent; padding repeats a row).
    start = 0
    for size in _batch_sizes(sizes):
        rows = model_lib.PricingInputs(*(t[start:start + size] for t in batch))
        want = _direct(fn, rows)
        for i in range(size):
            assert results[start + i].value.log_price == float(want[i])
            assert results[start + i].value.candidates_used == int(used[start + i])
        start += size


def _batch_sizes(sizes):
    """Consecutive batch sizes from per-request sizes (requests are served in order)."""
    out, i = [], 0
    while i < len(sizes):
        out.append(sizes[i])
        i += sizes[i]
    return out
