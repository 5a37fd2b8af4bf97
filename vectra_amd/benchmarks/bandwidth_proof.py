"""HBM bytes per query and achieved HBM bandwidth, eager versus fused, from
rocprofv3 counters.

  python -m vectra_amd.benchmarks.bandwidth_proof [--batches 64 1024] [--config serving] \\
      [--out bandwidth.json] [--work rocprof_bandwidth]

Restates the reference's benchmark/bandwidth/run_bandwidth_proof.py:16-120
with rocprofv3 in place of Nsight Compute.  For each batch and for both the
eager chain and the fused operator it profiles the attention region of
`vectra_amd.benchmarks.eager_gpu` three times: `--kernel-trace --stats` for
the kernels' time, then `--pmc FETCH_SIZE` and `--pmc WRITE_SIZE` for HBM
bytes (each counter scaled by what it reads for a device copy of known
size, `vectra_amd.benchmarks.copy_calibration`).  Per call of the region:

  dram_bytes            read + write bytes
  dram_bytes_per_query  dram_bytes / batch
  kernel_ns             time of the region's kernels
  dram_throughput_pct   dram_bytes / kernel_ns against the 8 TB/s peak

The default workload is the serving shape (B=1024, H=8, Lq=1, Lk=64, D=32,
bf16); `--config bandwidth` is the reference's own (H=4, Lq=Lk=65, fp16).
Each run makes 5 warm-up calls (one per rotating input set, 5 x the
working set: above the 256 MB Infinity Cache at B=1024) and `--reps` more.
The warm-up calls stay outside the measured region, as the reference's
harness keeps its warm-up outside the profiled NVTX range
(kernels/benchmarks/bandwidth.py:60-77): times (per dispatch, from the kernel
trace) and counters are summed over the dispatches of the `--reps` calls
after them and divided by `--reps`.  It then checks the gates the reference
reads from its serving SLO:

* fused / eager DRAM bytes <= 0.60 at every batch;
* fused DRAM throughput >= 65 % of peak at the batch whose working set
  exceeds the caches (1024), where it measures streaming, not launch latency.

The analytic budgets of `vectra_amd.benchmarks.roofline` are reported
beside the counters, and with `--read-ceiling` so is a plain read of the
fused bytes measured the same way (`eager_gpu --impl read`): what the
hardware itself reaches with one call at a time; where the output is at
least an eighth of the reads (the self-attention shapes), also a plain kernel
streaming the same reads and writes (`eager_gpu --impl readwrite`), and the
fused kernel's share of it.  Exits 1 when a gate fails.
"""

import argparse
import csv
import dataclasses
import json
import os
import subprocess
import sys

from vectra_amd.benchmarks import configs
from vectra_amd.benchmarks import roofline
from vectra_amd.benchmarks import rocprof_summary

# The GPU gates of the reference's serving SLO (serving/configs/slo.yaml:21-30).
SLO = {
    'gpu': {
        'dram_bytes_ratio_max': 0.60,
        'throughput_ratio_min': 3.0,
        'dram_throughput_pct_min': 65,
        'numerics_rtol': 1.0e-3,
    },
}

# The batch at which bandwidth utilisation is judged (working set > caches).
UTILIZATION_BATCH = 1024

# rocprofv3 names the runtime's copy kernels with this prefix; they move the
# host-built inputs, not the region's data.
RUNTIME_BLIT = rocprof_summary.RUNTIME_BLIT


def evaluate(measured: dict, slo: dict = SLO) -> list[str]:
    """Failures of a {batch: {impl: counters}} measurement against the SLO
    (run_bandwidth_proof.py:66-83)."""
    max_ratio = slo['gpu']['dram_bytes_ratio_max']
    min_pct = slo['gpu']['dram_throughput_pct_min']
    failures = []
    for batch, runs in measured.items():
        ratio = runs['fused']['dram_bytes'] / runs['eager']['dram_bytes']
        if ratio > max_ratio:
            failures.append(f'batch {batch}: fused/eager bytes {ratio:.3f} > {max_ratio}')
    utilization = measured.get(UTILIZATION_BATCH)
    if utilization is None:
        failures.append(f'batch {UTILIZATION_BATCH} was not profiled')
    elif utilization['fused']['dram_throughput_pct'] < min_pct:
        achieved = utilization['fused']['dram_throughput_pct']
        failures.append(f'fused DRAM throughput {achieved:.1f}% < {min_pct}%')
    return failures


def measured_dispatches(values: list[float], calls: int, warmup: int) -> list[float]:
    """The per-dispatch values of the calls after the first `warmup` (every
    call of the region launches the same number of kernels)."""
    if calls <= warmup or len(values) % calls:
        raise ValueError(f'{len(values)} dispatches do not divide into {calls} calls')
    return values[warmup * (len(values) // calls):]


def region_durations_ns(path: str) -> list[float]:
    """Each dispatch's duration from a `--kernel-trace` CSV, in launch order
    (runtime copy blits excluded)."""
    with open(path, encoding='utf-8') as f:
        rows = [r for r in csv.DictReader(f) if RUNTIME_BLIT not in r['Kernel_Name']]
    rows.sort(key=lambda r: int(r['Start_Timestamp']))
    return [float(int(r['End_Timestamp']) - int(r['Start_Timestamp'])) for r in rows]


def region_counter_values(path: str) -> list[float]:
    """A counter per dispatch, in dispatch order (runtime copy blits excluded;
    rows of one dispatch summed)."""
    per: dict[int, float] = {}
    with open(path, encoding='utf-8') as f:
        for r in csv.DictReader(f):
            if RUNTIME_BLIT not in r['Kernel_Name']:
                key = int(r['Dispatch_Id'])
                per[key] = per.get(key, 0.0) + float(r['Counter_Value'])
    return [per[k] for k in sorted(per)]


def region_counters(trace_csv: str, fetch_csv: str, write_csv: str, calls: int, warmup: int, batch: int,
                    scales: dict) -> dict:
    """Per-call bytes, time and throughput of a region from its three runs,
    over the calls after the first `warmup`."""
    measured = calls - warmup
    read = sum(measured_dispatches(region_counter_values(fetch_csv), calls, warmup)) * 1024.0 * scales[
        'fetch_scale'] / measured
    write = sum(measured_dispatches(region_counter_values(write_csv), calls, warmup)) * 1024.0 * scales[
        'write_scale'] / measured
    kernel_ns = sum(measured_dispatches(region_durations_ns(trace_csv), calls, warmup)) / measured
    dram_bytes = read + write
    return {
        'dram_bytes': dram_bytes,
        'dram_read_bytes': read,
        'dram_write_bytes': write,
        'dram_bytes_per_query': dram_bytes / batch,
        'kernel_ns': kernel_ns,
        'dram_throughput_pct': 100.0 * dram_bytes / (kernel_ns * 1e-9) / roofline.MI355X.hbm_bytes_per_s,
    }


def _rocprof(args: list[str], out_dir: str, name: str, program: list[str], timeout: int) -> str:
    """Runs `program` under rocprofv3 as a child process; returns its output directory."""
    target = os.path.join(out_dir, name)
    cmd = ['timeout', '-s', 'KILL', str(timeout), 'rocprofv3', *args, '--output-format', 'csv',
           '-d', target, '-o', name, '--', *program]
    print('+', ' '.join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    return target


def copy_scales(work: str) -> dict:
    """FETCH_SIZE / WRITE_SIZE bytes per counter byte, from a 512 MiB device copy."""
    program = [sys.executable, '-m', 'vectra_amd.benchmarks.copy_calibration']
    fetch = _rocprof(['--pmc', 'FETCH_SIZE'], work, 'copy_fetch', program, 90)
    write = _rocprof(['--pmc', 'WRITE_SIZE'], work, 'copy_write', program, 90)
    copy_bytes = 512 << 20
    cf = max(rocprof_summary.counter_per_dispatch(os.path.join(fetch, 'copy_fetch_counter_collection.csv'),
                                                  'copyBuffer'))
    cw = max(rocprof_summary.counter_per_dispatch(os.path.join(write, 'copy_write_counter_collection.csv'),
                                                  'copyBuffer'))
    return {'fetch_scale': copy_bytes / (cf * 1024.0), 'write_scale': copy_bytes / (cw * 1024.0)}


def measure(config_name: str, batch: int, impl: str, work: str, scales: dict, reps: int) -> dict:
    program = [sys.executable, '-m', 'vectra_amd.benchmarks.eager_gpu', '--impl', impl,
               '--config', config_name, '--batch', str(batch), '--reps', str(reps)]
    name = f'{impl}_{batch}'
    stats = _rocprof(['--kernel-trace', '--stats'], work, f'{name}_trace', program, 180)
    fetch = _rocprof(['--pmc', 'FETCH_SIZE'], work, f'{name}_fetch', program, 120)
    write = _rocprof(['--pmc', 'WRITE_SIZE'], work, f'{name}_write', program, 120)
    warmup = 5  # eager_gpu: one warm-up call per input set (5), then --reps
    return region_counters(os.path.join(stats, f'{name}_trace_kernel_trace.csv'),
                           os.path.join(fetch, f'{name}_fetch_counter_collection.csv'),
                           os.path.join(write, f'{name}_write_counter_collection.csv'),
                           warmup + reps, warmup, batch, scales)


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__.split('\n\n')[0])
    p.add_argument('--config', default='serving', choices=sorted(configs.CONFIGS))
    p.add_argument('--batches', type=int, nargs='+', default=[64, UTILIZATION_BATCH])
    p.add_argument('--reps', type=int, default=20)
    p.add_argument('--work', default='rocprof_bandwidth', help='rocprofv3 output directory')
    p.add_argument('--out', default=None)
    p.add_argument('--read-ceiling', action='store_true',
                   help='also profile a plain read of the fused bytes, reported beside the gates')
    args = p.parse_args(argv)
    os.makedirs(args.work, exist_ok=True)
    work = os.path.abspath(args.work)
    config = configs.CONFIGS[args.config]
    scales = copy_scales(work)
    measured, budgets = {}, {}
    ceilings = {}
    for batch in args.batches:
        measured[batch] = {impl: measure(args.config, batch, impl, work, scales, args.reps)
                           for impl in ('eager', 'fused')}
        if args.read_ceiling:
            ceilings[batch] = {'read': measure(args.config, batch, 'read', work, scales, args.reps)}
            shape = dataclasses.replace(config, batch=batch).shape()
            out_bytes = shape.planes * shape.n_q * shape.value_dim * shape.element_bytes
            if out_bytes * 8 >= roofline.fused_bytes(shape) - out_bytes:
                mixed = measure(args.config, batch, 'readwrite', work, scales, args.reps)
                # The fused kernel's rate as a share of the plain stream's.
                mixed['fused_share'] = mixed['kernel_ns'] / measured[batch]['fused']['kernel_ns']
                ceilings[batch]['read_write'] = mixed
        budgets[batch] = roofline.analyze(dataclasses.replace(config, batch=batch).shape())
    failures = evaluate(measured)
    report = {'config': args.config, 'copy_scales': scales, 'measured': measured,
              'analytic_budgets': budgets, 'failures': failures, 'passed': not failures}
    if ceilings:
        report['read_ceiling'] = ceilings
    text = json.dumps(report, indent=2)
    if args.out:
        with open(args.out, 'w', encoding='utf-8') as f:
            f.write(text + '\n')
    print(json.dumps({'failures': failures, 'passed': not failures}), flush=True)
    return 0 if not failures else 1


if __name__ == '__main__':
    sys.exit(main())
