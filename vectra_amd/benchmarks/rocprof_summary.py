"""Summaries of rocprofv3 output for the operator's kernels.

  python -m vectra_amd.benchmarks.rocprof_summary stats  <kernel_stats.csv> [--kernel NAME]
  python -m vectra_amd.benchmarks.rocprof_summary traffic \\
      --fetch <counter_collection.csv> --write <counter_collection.csv> \\
      --copy-fetch <counter_collection.csv> --copy-write <counter_collection.csv> \\
      --kernel rbf_stream_kernel --copy-bytes 536870912 --algorithmic-bytes 68288544 \\
      [--json out.json]
  python -m vectra_amd.benchmarks.rocprof_summary region \\
      --fetch <csv> --write <csv> --calls N --scales traffic.json [--json out.json]
  python -m vectra_amd.benchmarks.rocprof_summary ratio fused.json eager.json [--json out.json]

`stats` prints the per-kernel durations of a `rocprofv3 --kernel-trace
--stats` run.  `traffic` turns two `rocprofv3 --pmc FETCH_SIZE` /
`--pmc WRITE_SIZE` runs (KiB per dispatch) into HBM bytes per launch: each
counter is scaled by bytes / counter of a plain device copy of known size
measured the same way (vectra_amd.benchmarks.copy_calibration), and the
result is compared with the kernel's algorithmic bytes.  `region` sums the
counters over every dispatch of a run (runtime copy blits excluded) and
divides by the number of calls of the measured region, with the copy scale
factors of a `traffic` result; `ratio` divides one region's bytes by
another's (the fused operator's by the eager chain's).
"""

import argparse
import csv
import json
import statistics
import sys


def kernel_stats(path: str, kernel: str | None = None) -> list[dict]:
    rows = list(csv.DictReader(open(path, encoding='utf-8')))
    out = []
    for r in rows:
        if kernel and kernel not in r['Name']:
            continue
        out.append({
            'name': r['Name'],
            'calls': int(r['Calls']),
            'average_ns': float(r['AverageNs']),
            'min_ns': float(r['MinNs']),
            'max_ns': float(r['MaxNs']),
            'percent': float(r['Percentage']),
        })
    return out


def counter_per_dispatch(path: str, kernel: str) -> list[float]:
    """Counter values (summed over any per-dimension rows) of each dispatch."""
    per_dispatch: dict[str, float] = {}
    for r in csv.DictReader(open(path, encoding='utf-8')):
        if kernel in r['Kernel_Name']:
            key = r['Dispatch_Id']
            per_dispatch[key] = per_dispatch.get(key, 0.0) + float(r['Counter_Value'])
    return list(per_dispatch.values())


def traffic(args) -> dict:
    fetch = statistics.median(counter_per_dispatch(args.fetch, args.kernel))
    write = statistics.median(counter_per_dispatch(args.write, args.kernel))
    copy_fetch = max(counter_per_dispatch(args.copy_fetch, args.copy_kernel))
    copy_write = max(counter_per_dispatch(args.copy_write, args.copy_kernel))
    fetch_scale = args.copy_bytes / (copy_fetch * 1024.0)
    write_scale = args.copy_bytes / (copy_write * 1024.0)
    fetch_bytes = fetch * 1024.0 * fetch_scale
    write_bytes = write * 1024.0 * write_scale
    total = fetch_bytes + write_bytes
    return {
        'kernel': args.kernel,
        'fetch_size_kib_per_dispatch': fetch,
        'write_size_kib_per_dispatch': write,
        'copy_fetch_size_kib': copy_fetch,
        'copy_write_size_kib': copy_write,
        'fetch_scale': fetch_scale,
        'write_scale': write_scale,
        'hbm_read_bytes': fetch_bytes,
        'hbm_write_bytes': write_bytes,
        'traffic_bytes': total,
        'algorithmic_bytes': args.algorithmic_bytes,
        'traffic_over_algorithmic': total / args.algorithmic_bytes if args.algorithmic_bytes else None,
    }


RUNTIME_BLIT = '__amd_rocclr_'


def region(args) -> dict:
    """HBM bytes per call of a region: every dispatch of the run, summed."""
    with open(args.scales, encoding='utf-8') as f:
        scales = json.load(f)
    totals, kernels = {}, {}
    for name, path in (('fetch', args.fetch), ('write', args.write)):
        total = 0.0
        for r in csv.DictReader(open(path, encoding='utf-8')):
            if RUNTIME_BLIT in r['Kernel_Name']:
                continue
            total += float(r['Counter_Value'])
            if name == 'fetch':
                short = r['Kernel_Name'].split('(')[0][:80]
                kernels[short] = kernels.get(short, 0.0) + float(r['Counter_Value'])
        totals[name] = total
    read = totals['fetch'] * 1024.0 * scales['fetch_scale'] / args.calls
    write = totals['write'] * 1024.0 * scales['write_scale'] / args.calls
    return {
        'region': args.name,
        'calls': args.calls,
        'hbm_read_bytes_per_call': read,
        'hbm_write_bytes_per_call': write,
        'traffic_bytes_per_call': read + write,
        'fetch_scale': scales['fetch_scale'],
        'write_scale': scales['write_scale'],
        'read_bytes_by_kernel_per_call': {
            k: v * 1024.0 * scales['fetch_scale'] / args.calls
            for k, v in sorted(kernels.items(), key=lambda kv: -kv[1])
        },
    }


def ratio(args) -> dict:
    with open(args.fused, encoding='utf-8') as f:
        fused = json.load(f)
    with open(args.eager, encoding='utf-8') as f:
        eager = json.load(f)
    return {
        'fused_bytes_per_call': fused['traffic_bytes_per_call'],
        'eager_bytes_per_call': eager['traffic_bytes_per_call'],
        'bytes_ratio': fused['traffic_bytes_per_call'] / eager['traffic_bytes_per_call'],
        'gate': 0.60,
    }


def main(argv=None):
    p = argparse.ArgumentParser()
    sub = p.add_subparsers(dest='cmd', required=True)
    s = sub.add_parser('stats')
    s.add_argument('csv')
    s.add_argument('--kernel', default=None)
    t = sub.add_parser('traffic')
    t.add_argument('--fetch', required=True)
    t.add_argument('--write', required=True)
    t.add_argument('--copy-fetch', required=True)
    t.add_argument('--copy-write', required=True)
    t.add_argument('--kernel', required=True)
    t.add_argument('--copy-kernel', default='copyBuffer')
    t.add_argument('--copy-bytes', type=int, default=512 << 20)
    t.add_argument('--algorithmic-bytes', type=int, default=0)
    t.add_argument('--json', default=None)
    g = sub.add_parser('region')
    g.add_argument('--fetch', required=True)
    g.add_argument('--write', required=True)
    g.add_argument('--calls', type=int, required=True)
    g.add_argument('--scales', required=True, help='a traffic result (its fetch/write scales)')
    g.add_argument('--name', default='region')
    g.add_argument('--json', default=None)
    r = sub.add_parser('ratio')
    r.add_argument('fused')
    r.add_argument('eager')
    r.add_argument('--json', default=None)
    args = p.parse_args(argv)
    if args.cmd == 'stats':
        for row in kernel_stats(args.csv, args.kernel):
            print(json.dumps(row))
        return
    result = {'traffic': traffic, 'region': region, 'ratio': ratio}[args.cmd](args)
    text = json.dumps(result, indent=2)
    if args.json:
        with open(args.json, 'w', encoding='utf-8') as f:
            f.write(text + '\n')
    print(text)


if __name__ == '__main__':
    sys.exit(main())
