"""Matrix-core utilisation of the long-key kernel, from rocprofv3 counters.

  python -m vectra_amd.benchmarks.mfma_utilization [--config long_key] [--steps 20] \\
      [--kernel rbf_tile_kernel] [--work rocprof_mfma] [--out mfma.json]

The reference measures its kernels by running a profiler over a command and
aggregating a fixed list of counters per kernel, then judging the result
(benchmark/bandwidth/collect_nsight_metrics.py:36-41,
run_bandwidth_proof.py:66-120).  This is that pattern for the compute-bound
config, on rocprofv3: two runs of `bench.py --config <config>` (the timed
long-key launches through the C ABI), each as a child process:

1. `--kernel-trace --stats`: every dispatch's duration, undisturbed;
2. `--pmc` with COUNTERS (one pass: 5 SQ counters and 1 GRBM counter):

     SQ_VALU_MFMA_BUSY_CYCLES  matrix-core busy cycles, summed over all SIMDs
     SQ_INSTS_MFMA             MFMA instructions issued
     SQ_INSTS_VALU             vector instructions issued (MFMAs included)
     SQ_WAVE_CYCLES            wave-resident cycles, summed over waves
     SQ_BUSY_CYCLES            cycles the shader engines were busy
     GRBM_GUI_ACTIVE           GPU-active cycles of the dispatch

For the named kernel (median over its dispatches) it reports:

  mfma_busy_pct      100 SQ_VALU_MFMA_BUSY_CYCLES / (SIMDs x active cycles):
                     the share of the matrix cores' cycles spent busy, at the
                     clock the dispatch actually ran (the counters' own
                     definition of utilisation);
  clock_ghz          active cycles / the dispatch's duration in the counter run;
  flops_pct          the algorithmic matrix FLOPs (2 B H Nq Nk (D + Dv), the
                     two products, roofline.matrix_flops) over the
                     undisturbed duration, against the 2.5 PFLOP/s dense bf16
                     peak (which assumes 2.4 GHz);
  issued_flops_pct   the same with every issued MFMA counted (16x16x32: 16384
                     FLOPs each; weight sums and their squares included);
  busy_cycles_per_mfma  SQ_VALU_MFMA_BUSY_CYCLES / SQ_INSTS_MFMA (16 for a
                     16x16x32 instruction at full rate).

The two utilisation figures differ by the clock (flops_pct assumes the peak's
2.4 GHz) and by the MFMAs that are not the reference's FLOPs.  If the
GRBM counter arrives summed over the XCDs (its per-dispatch rate would be
more than MAX_CLOCK_GHZ), it is divided by their number.
"""

import argparse
import csv
import json
import os
import statistics
import subprocess
import sys

from vectra_amd.benchmarks import configs
from vectra_amd.benchmarks import roofline
from vectra_amd.benchmarks import rocprof_summary

COUNTERS = ('SQ_VALU_MFMA_BUSY_CYCLES', 'SQ_INSTS_MFMA', 'SQ_INSTS_VALU', 'SQ_WAVE_CYCLES', 'SQ_BUSY_CYCLES',
            'GRBM_GUI_ACTIVE')
MFMA_16X16X32_FLOPS = 2 * 16 * 16 * 32
MAX_CLOCK_GHZ = 3.5  # above any shader clock: a larger rate means a sum over XCDs
SIMDS_PER_CU = 4

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))


def _rocprof(args: list[str], out_dir: str, name: str, program: list[str], timeout: int) -> str:
    target = os.path.join(out_dir, name)
    cmd = ['timeout', '-s', 'KILL', str(timeout), 'rocprofv3', *args, '--output-format', 'csv',
           '-d', target, '-o', name, '--', *program]
    print('+', ' '.join(cmd), flush=True)
    subprocess.run(cmd, check=True, cwd=ROOT)
    return target


def trace_durations_ns(path: str, kernel: str) -> list[float]:
    """Durations of the kernel's dispatches in a --kernel-trace CSV."""
    with open(path, encoding='utf-8') as f:
        return [float(int(r['End_Timestamp']) - int(r['Start_Timestamp']))
                for r in csv.DictReader(f) if kernel in r['Kernel_Name']]


def counter_rows(path: str, kernel: str) -> dict[int, dict]:
    """Per dispatch of the kernel: {counter: value} and the dispatch's duration
    in the counter run ('ns')."""
    per: dict[int, dict] = {}
    with open(path, encoding='utf-8') as f:
        for r in csv.DictReader(f):
            if kernel not in r['Kernel_Name']:
                continue
            d = per.setdefault(int(r['Dispatch_Id']), {})
            d[r['Counter_Name']] = d.get(r['Counter_Name'], 0.0) + float(r['Counter_Value'])
            d['ns'] = float(int(r['End_Timestamp']) - int(r['Start_Timestamp']))
    return per


def derive(dispatch: dict, spec: roofline.GpuSpec = roofline.MI355X) -> dict:
    """Utilisation figures of one dispatch's counters."""
    active = dispatch['GRBM_GUI_ACTIVE']
    summed_over_xcds = active / dispatch['ns'] > MAX_CLOCK_GHZ
    if summed_over_xcds:
        active /= spec.xcds
    simds = spec.compute_units * SIMDS_PER_CU
    mfma = dispatch['SQ_INSTS_MFMA']
    return {
        'active_cycles': active,
        'grbm_summed_over_xcds': summed_over_xcds,
        'clock_ghz': active / dispatch['ns'],
        'mfma_busy_pct': 100.0 * dispatch['SQ_VALU_MFMA_BUSY_CYCLES'] / (simds * active),
        'busy_cycles_per_mfma': dispatch['SQ_VALU_MFMA_BUSY_CYCLES'] / mfma if mfma else None,
        'valu_per_mfma': (dispatch['SQ_INSTS_VALU'] - mfma) / mfma if mfma else None,
    }


def summarize(trace_csv: str, counter_csv: str, kernel: str, flops: float,
              spec: roofline.GpuSpec = roofline.MI355X) -> dict:
    durations = trace_durations_ns(trace_csv, kernel)
    rows = counter_rows(counter_csv, kernel)
    if not durations or not rows:
        raise ValueError(f'no dispatch of {kernel} in the profiles')
    ns = statistics.median(durations)
    derived = [dict(derive(d, spec), **d) for d in rows.values()]
    med = {key: statistics.median(d[key] for d in derived)
           for key in ('mfma_busy_pct', 'clock_ghz', 'busy_cycles_per_mfma', 'valu_per_mfma', *COUNTERS)}
    issued = med['SQ_INSTS_MFMA'] * MFMA_16X16X32_FLOPS
    return {
        'kernel': kernel,
        'dispatches_traced': len(durations),
        'dispatches_counted': len(rows),
        'median_ns': ns,
        'counters_per_dispatch': {c: med[c] for c in COUNTERS},
        'grbm_summed_over_xcds': derived[0]['grbm_summed_over_xcds'],
        'clock_ghz': med['clock_ghz'],
        'mfma_busy_pct': med['mfma_busy_pct'],
        'busy_cycles_per_mfma': med['busy_cycles_per_mfma'],
        'valu_per_mfma': med['valu_per_mfma'],
        'algorithmic_flops': flops,
        'flops_pct': 100.0 * flops / (ns * 1e-9) / spec.bf16_mfma_flops,
        'issued_flops': issued,
        'issued_flops_pct': 100.0 * issued / (ns * 1e-9) / spec.bf16_mfma_flops,
        'achieved_tflops': flops / (ns * 1e-9) / 1e12,
    }


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__.split('\n\n')[0])
    p.add_argument('--config', default='long_key', choices=sorted(configs.CONFIGS))
    p.add_argument('--kernel', default='rbf_tile_kernel')
    p.add_argument('--steps', type=int, default=20)
    p.add_argument('--work', default='rocprof_mfma', help='rocprofv3 output directory')
    p.add_argument('--out', default=None)
    args = p.parse_args(argv)
    work = os.path.abspath(args.work)
    os.makedirs(work, exist_ok=True)
    program = [sys.executable, 'bench.py', '--config', args.config, '--steps', str(args.steps),
               '--warmup', '3', '--cpu-seconds', '0', '--no-read-ceiling']
    trace = _rocprof(['--kernel-trace', '--stats'], work, 'mfma_trace', program, 300)
    counters = _rocprof(['--pmc', *COUNTERS], work, 'mfma_pmc', program, 300)
    flops = roofline.matrix_flops(configs.CONFIGS[args.config].shape())
    report = summarize(os.path.join(trace, 'mfma_trace_kernel_trace.csv'),
                       os.path.join(counters, 'mfma_pmc_counter_collection.csv'), args.kernel, flops)
    report['config'] = args.config
    report['commands'] = {
        'trace': f'rocprofv3 --kernel-trace --stats -- {" ".join(program[1:])}',
        'counters': f'rocprofv3 --pmc {" ".join(COUNTERS)} -- {" ".join(program[1:])}',
    }
    report['stats'] = rocprof_summary.kernel_stats(os.path.join(trace, 'mfma_trace_kernel_stats.csv'), args.kernel)
    text = json.dumps(report, indent=2)
    if args.out:
        with open(args.out, 'w', encoding='utf-8') as f:
            f.write(text + '\n')
    print(text, flush=True)
    return 0


if __name__ == '__main__':
    sys.exit(main())
