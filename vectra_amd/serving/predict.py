"""Batched prediction for the gateway: requests in, prices out.

Restates the model-facing half of the reference's serving/predict.py: one
request is one subject with its comparables, already featurised (the
reference's FeatureBuilder output for a single subject, predict.py:85-177);
a batch of requests is assembled straight into a DeviceFeeder slot's pinned
buffers, run through the compiled model, and every request gets its
predicted log price and the number of comparables the model attended to
after radius trimming (predict.py:180-196, 206-244).
"""

import dataclasses
from collections.abc import Sequence

import torch

from vectra_amd.price_transformer import microhood
from vectra_amd.price_transformer import model as model_lib
from vectra_amd.serving import feeder as feeder_lib


@dataclasses.dataclass
class Prediction:
    log_price: float
    candidates_used: int


def comparables_used(inputs: model_lib.PricingInputs, min_candidates: int) -> torch.Tensor:
    """[B] comparables the model attends to after radius trimming (the
    model's own trim_to_radius on the batch)."""
    distance = microhood.haversine_km(inputs.query_location, inputs.cand_location)
    mask = model_lib.trim_to_radius(distance, inputs.radius_km, inputs.cand_valid,
                                    min(min_candidates, inputs.cand_valid.shape[-1]))
    return mask.sum(-1)


def request_rows(batch: model_lib.PricingInputs) -> list[model_lib.PricingInputs]:
    """Splits a batch into single-subject requests (every field without the
    batch dimension)."""
    return [model_lib.PricingInputs(*(t[i] for t in batch)) for i in range(batch[0].shape[0])]


class Predictor:
    """Runs batches of requests through a compiled model on the GPU.

    `launch(requests)` assembles the requests into the feeder's next slot
    and enqueues the batch; `finish(handle)` waits for it and returns one
    Prediction per request.  They are the two stages a Batcher pipelines
    (Batcher(launch=p.launch, finish=p.finish, depth=feeder.slots)); calling
    them in turn is one synchronous batch.
    """

    def __init__(self, feeder: feeder_lib.DeviceFeeder, min_candidates: int):
        self._feeder = feeder
        self._min_candidates = min_candidates

    @property
    def batch_size(self) -> int:
        return self._feeder.batch_size

    def launch(self, requests: Sequence[model_lib.PricingInputs]):
        n = len(requests)
        if not 1 <= n <= self._feeder.batch_size:
            raise ValueError(f'a batch holds 1 .. {self._feeder.batch_size} requests, not {n}')
        slot, host = self._feeder.next_slot()
        for field, dst in enumerate(host):
            torch.stack([r[field] for r in requests], out=dst[:n])
        handle = self._feeder.launch(slot, n)
        # On the host while the GPU works (the copy only reads these rows).
        used = comparables_used(model_lib.PricingInputs(*(t[:n] for t in host)), self._min_candidates)
        return handle, used

    def finish(self, launched) -> list[Prediction]:
        handle, used = launched
        log_price = self._feeder.finish(handle)
        return [Prediction(float(p), int(u)) for p, u in zip(log_price.tolist(), used.tolist())]

    def __call__(self, requests: Sequence[model_lib.PricingInputs]) -> list[Prediction]:
        return self.finish(self.launch(requests))
