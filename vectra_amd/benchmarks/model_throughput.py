"""Full-model serving throughput: eager vs Inductor vs the vectra compile.

  python -m vectra_amd.benchmarks.model_throughput --mode eager    --out eager.json
  python -m vectra_amd.benchmarks.model_throughput --mode inductor --out inductor.json
  python -m vectra_amd.benchmarks.model_throughput --mode vectra   --out vectra.json
  python -m vectra_amd.benchmarks.model_throughput --compare eager.json vectra.json [--min-ratio 3.0]

Restates the reference's benchmark/gpu_throughput/run_throughput.py:90-178
and compare_runs.py:46-63 on this build.  Throughput is measured on the
whole price model at the serving batch (config 5: d_model 128, 8 heads, 3 or
4 layers, 16 attributes, 64 comparables, batch 1024, 50 km box inputs).
Modes: `eager` (the baseline), `inductor` (torch.compile without the rewrite,
which separates Inductor's own fusion from the HIP operator) and `vectra`
(the deployment compile: every attention site on vectra::rbf_attention).
Each run first gates its numerics against the eager model (rtol 1e-3), then
times `--iters` forward passes after `--warmup` with events, as the median of
`--trials` trials.  `--compare` checks a candidate against a baseline: same
device, batch, precision and comparables, numerics within the gate, and a
throughput ratio of at least --min-ratio (the design's 3.0x).
"""

import argparse
import json
import os
import statistics
import sys

import torch

from vectra_amd.export import compile_entry
from vectra_amd.price_transformer import model as model_lib

MATCHED = ('device', 'batch_size', 'block_dtype', 'num_candidates', 'num_layers')


def config_5(layers: int) -> model_lib.ModelConfig:
    return model_lib.ModelConfig(d_model=128, num_heads=8, num_layers=layers, attribute_dim=16,
                                 ffn_dim=256, num_candidates=64)


def timed(fn, inputs, iters: int, warmup: int, trials: int) -> list[float]:
    """Seconds per forward pass of each trial."""
    out = []
    with torch.no_grad():
        for _ in range(warmup):
            fn(*inputs)
        torch.cuda.synchronize()
        for _ in range(trials):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            for _ in range(iters):
                fn(*inputs)
            end.record()
            end.synchronize()
            out.append(start.elapsed_time(end) / 1e3 / iters)
    return out


def run(mode: str, batch_size: int, layers: int, block_dtype: str, iters: int, warmup: int,
        trials: int) -> dict:
    device = 'cuda'
    spec = compile_entry.ServingSpec(device, batch_size, block_dtype)
    torch.manual_seed(0)
    eager = compile_entry.prepare(model_lib.PriceTransformer(config_5(layers)), spec)
    inputs = tuple(model_lib.box_inputs(eager.config, batch_size, device=device, seed=0))
    sites = 0
    if mode == 'eager':
        fn = eager
    elif mode == 'inductor':
        fn = torch.compile(eager, fullgraph=True, dynamic=False)
    else:
        fn, report, _ = compile_entry.compile_model(eager, spec)
        sites = report.sites
    worst, _ = compile_entry.max_abs_error(fn, eager, eager.config, spec, batches=2)
    seconds = timed(fn, inputs, iters, warmup, trials)
    per_batch = statistics.median(seconds)
    return {
        'mode': mode,
        'device': torch.cuda.get_device_name(device),
        'batch_size': batch_size,
        'block_dtype': block_dtype,
        'num_candidates': eager.config.num_candidates,
        'num_layers': layers,
        'rewritten_sites': sites,
        'ms_per_batch': per_batch * 1e3,
        'requests_per_s': batch_size / per_batch,
        'trials': trials,
        'iters_per_trial': iters,
        'max_abs_error_vs_eager': worst,
        'numerics_rtol': compile_entry.RTOL,
        'inputs': 'synthetic box_inputs (50 km box, sale ages 0-730 days), random-init weights',
        'versions': compile_entry.toolchain_versions(),
    }


def compare(baseline: dict, candidate: dict, min_ratio: float) -> tuple[bool, list[str], float]:
    """(passed, problems, throughput ratio)."""
    problems = [f'{key} differs: {baseline.get(key)} vs {candidate.get(key)}'
                for key in MATCHED if baseline.get(key) != candidate.get(key)]
    tolerance = candidate.get('numerics_rtol', 1e-3)
    # The output is a log price near 13, so rtol 1e-3 allows ~0.013.
    if candidate['max_abs_error_vs_eager'] > 13.0 * tolerance + 1e-3:
        problems.append(f"numerics: max |compiled - eager| = {candidate['max_abs_error_vs_eager']:.3g}")
    ratio = candidate['requests_per_s'] / baseline['requests_per_s']
    if ratio < min_ratio:
        problems.append(f'throughput ratio {ratio:.2f} < {min_ratio}')
    return not problems, problems, ratio


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__.split('\n\n')[0])
    p.add_argument('--mode', choices=['eager', 'inductor', 'vectra'])
    p.add_argument('--batch-size', type=int, default=1024)
    p.add_argument('--layers', type=int, default=3)
    p.add_argument('--block-dtype', choices=['float32', 'float16', 'bfloat16'], default='float16')
    p.add_argument('--iters', type=int, default=50)
    p.add_argument('--warmup', type=int, default=10)
    p.add_argument('--trials', type=int, default=5)
    p.add_argument('--out', default='')
    p.add_argument('--compare', nargs=2, metavar=('BASELINE', 'CANDIDATE'))
    p.add_argument('--min-ratio', type=float, default=3.0)
    args = p.parse_args(argv)
    if args.compare:
        with open(args.compare[0], encoding='utf-8') as f:
            baseline = json.load(f)
        with open(args.compare[1], encoding='utf-8') as f:
            candidate = json.load(f)
        passed, problems, ratio = compare(baseline, candidate, args.min_ratio)
        print(json.dumps({'passed': passed, 'ratio': ratio, 'problems': problems,
                          'baseline': baseline['mode'], 'candidate': candidate['mode']}))
        return 0 if passed else 1
    if args.mode is None:
        p.error('--mode or --compare is required')
    if not torch.cuda.is_available():
        print('model_throughput needs a GPU', file=sys.stderr)
        return 2
    result = run(args.mode, args.batch_size, args.layers, args.block_dtype, args.iters, args.warmup,
                 args.trials)
    text = json.dumps(result)
    if args.out:
        os.makedirs(os.path.dirname(args.out) or '.', exist_ok=True)
        with open(args.out, 'w', encoding='utf-8') as f:
            f.write(text + '\n')
    print(text, flush=True)
    return 0


if __name__ == '__main__':
    sys.exit(main())
