"""A plain device copy of known size, for scaling HBM byte counters.

  rocprofv3 --pmc FETCH_SIZE -- python3 -m vectra_amd.benchmarks.copy_calibration
  rocprofv3 --pmc WRITE_SIZE -- python3 -m vectra_amd.benchmarks.copy_calibration

Copies --mib MiB (default 512, twice the Infinity Cache) from one buffer to
another --reps times.  Each copy reads and writes exactly that many bytes, so
(bytes) / (counter KiB per dispatch * 1024) is the factor that turns the
counter into bytes for the operator's kernel measured the same way.
"""

import argparse
import json

import torch


def main():
    p = argparse.ArgumentParser()
    p.add_argument('--mib', type=int, default=512)
    p.add_argument('--reps', type=int, default=3)
    args = p.parse_args()
    n = args.mib << 20
    src = torch.randint(0, 255, (n,), dtype=torch.uint8, device='cuda')
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(args.reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    assert torch.equal(dst[:4096], src[:4096])
    print(json.dumps({'copy_bytes_per_dispatch': n, 'reps': args.reps}))


if __name__ == '__main__':
    main()
