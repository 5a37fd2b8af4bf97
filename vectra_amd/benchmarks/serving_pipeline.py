"""End-to-end serving throughput: host batches in, predictions back on the host.

  python -m vectra_amd.benchmarks.serving_pipeline [--batch-size 1024] [--layers 3] \\
      [--batches 40] [--out serving_pipeline.json]

The price model at config 5 (d_model 128, 8 heads, 16 attributes, 64
comparables, 50 km box inputs) is compiled with the `vectra` backend, and
batches of the compiled size reach it from host memory the ways a gateway
can feed it:

  resident        inputs already on the GPU, the model launched kernel by
                  kernel (the model_throughput figure)
  resident_graph  inputs already on the GPU, the model replayed as a HIP graph
                  (the GPU-bound ceiling)
  reference_path  per batch: each input moved with .to('cuda') from pageable
                  memory, the model, the result back with .cpu() -- the
                  reference's ServingModel.predict + Predictor order
  serial          DeviceFeeder with one slot: one pinned copy per batch, the
                  graph, the result back, wait -- nothing overlaps
  pipelined       DeviceFeeder with two slots and graphs: the next batch's
                  copy overlaps the model on the current one (host batches
                  copied into the slot first)
  in_place        the same pipeline with the batch already assembled in the
                  slot's pinned buffer (a feature builder that writes there
                  directly), so only PCIe, the model and the result remain
  h2d             the host-to-device copy of one batch from pinned memory

Every staged result is checked bit for bit against the model on the same
batch resident on the GPU before anything is timed.  Rates are requests per
second (wall clock over --batches batches after --warmup).
"""

import argparse
import json
import statistics
import time

import torch

from vectra_amd.benchmarks import model_throughput
from vectra_amd.export import compile_entry
from vectra_amd.price_transformer import model as model_lib
from vectra_amd.serving import feeder as feeder_lib


def _wall(fn, batches: int, warmup: int, trials: int) -> float:
    """Median seconds per batch of `trials` runs of fn(i) for i < batches."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    out = []
    for _ in range(trials):
        start = time.perf_counter()
        for i in range(batches):
            fn(i)
        torch.cuda.synchronize()
        out.append((time.perf_counter() - start) / batches)
    return statistics.median(out)


def run(batch_size: int, layers: int, block_dtype: str, batches: int, warmup: int, trials: int,
        sets: int) -> dict:
    spec = compile_entry.ServingSpec('cuda', batch_size, block_dtype)
    torch.manual_seed(0)
    model = compile_entry.prepare(model_lib.PriceTransformer(model_throughput.config_5(layers)), spec)
    fn, report, _ = compile_entry.compile_model(model, spec)
    compile_entry.max_abs_error(fn, model, model.config, spec, batches=1)
    host = [model_lib.box_inputs(model.config, batch_size, device='cpu', seed=s) for s in range(sets)]
    device = [h.to('cuda') for h in host]
    input_bytes = sum(t.numel() * t.element_size() for t in host[0])

    with torch.no_grad():
        resident_out = [fn(*d).float().cpu() for d in device]
    feeder = feeder_lib.DeviceFeeder(fn, host[0], slots=2, graph=True)
    serial = feeder_lib.DeviceFeeder(fn, host[0], slots=1, graph=True)
    # Numerics: every staged path returns exactly the resident model's output
    # (graph replays included, with eager work between them).
    for h, want in zip(host, resident_out):
        assert torch.equal(feeder.run(h), want)
        assert torch.equal(serial.run(h), want)
        with torch.no_grad():
            assert torch.equal(fn(*[t.to('cuda') for t in h]).float().cpu(), want)

    graph_inputs = model_lib.PricingInputs(*(t.clone() for t in device[0]))
    graph = torch.cuda.CUDAGraph()
    with torch.no_grad():
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn(*graph_inputs)
        torch.cuda.current_stream().wait_stream(side)
        with torch.cuda.graph(graph):
            graph_out = fn(*graph_inputs).float()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(graph_out.cpu(), resident_out[0])

    def resident(i):
        with torch.no_grad():
            fn(*device[i % sets])

    def resident_graph(i):
        graph.replay()

    def reference_path(i):
        with torch.no_grad():
            fn(*[t.to('cuda') for t in host[i % sets]]).float().cpu()

    def serial_step(i):
        serial.run(host[i % sets])

    pending = []

    def pipelined_step(i):
        if len(pending) == feeder.slots:
            feeder.finish(pending.pop(0))
        pending.append(feeder.launch(*feeder.stage(host[i % sets])))

    def in_place_step(i):
        if len(pending) == feeder.slots:
            feeder.finish(pending.pop(0))
        slot, _ = feeder.next_slot()
        pending.append(feeder.launch(slot, batch_size))

    def drain():
        while pending:
            feeder.finish(pending.pop(0))

    # Fill both slots once so the in-place run reads real batches.
    for h in host[:feeder.slots]:
        feeder.run(h)
    results = {}
    results['resident'] = _wall(resident, batches, warmup, trials)
    results['resident_graph'] = _wall(resident_graph, batches, warmup, trials)
    results['reference_path'] = _wall(reference_path, batches, warmup, trials)
    results['serial'] = _wall(serial_step, batches, warmup, trials)
    results['pipelined'] = _wall(pipelined_step, batches, warmup, trials)
    drain()
    results['in_place'] = _wall(in_place_step, batches, warmup, trials)
    drain()

    pinned = torch.empty(feeder.bytes_per_batch, dtype=torch.uint8, pin_memory=True)
    dev = torch.empty(feeder.bytes_per_batch, dtype=torch.uint8, device='cuda')

    def h2d(i):
        dev.copy_(pinned, non_blocking=True)

    results['h2d'] = _wall(h2d, batches, warmup, trials)
    return {
        'config': {'batch_size': batch_size, 'layers': layers, 'block_dtype': block_dtype,
                   'num_candidates': model.config.num_candidates, 'sites': report.sites,
                   'input_bytes_per_batch': input_bytes},
        'device': torch.cuda.get_device_name(),
        'ms_per_batch': {k: v * 1e3 for k, v in results.items()},
        'requests_per_s': {k: batch_size / v for k, v in results.items() if k != 'h2d'},
        'h2d_GB_per_s': feeder.bytes_per_batch / results['h2d'] / 1e9,
        'pipelined_over_reference_path': results['reference_path'] / results['pipelined'],
        'in_place_over_reference_path': results['reference_path'] / results['in_place'],
        'numerics': 'staged outputs bit-identical to the resident model',
    }


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__.split('\n\n')[0])
    p.add_argument('--batch-size', type=int, default=1024)
    p.add_argument('--layers', type=int, default=3)
    p.add_argument('--block-dtype', default='float16', choices=['float16', 'bfloat16', 'float32'])
    p.add_argument('--batches', type=int, default=40)
    p.add_argument('--warmup', type=int, default=5)
    p.add_argument('--trials', type=int, default=5)
    p.add_argument('--sets', type=int, default=4, help='distinct host batches cycled through')
    p.add_argument('--out', default=None)
    args = p.parse_args(argv)
    result = run(args.batch_size, args.layers, args.block_dtype, args.batches, args.warmup, args.trials,
                 args.sets)
    line = json.dumps(result)
    print(line, flush=True)
    if args.out:
        with open(args.out, 'w', encoding='utf-8') as f:
            f.write(line + '\n')
    return 0


if __name__ == '__main__':
    raise SystemExit(main())
