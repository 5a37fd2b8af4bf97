"""The eager operator chain on the GPU, beside the fused operator.

  python -m vectra_amd.benchmarks.eager_gpu --impl eager|fused|read [--config serving] [--batch B] [--reps 20]

`eager_rbf_attention` restates the reference's eager chain
(kernels/vectra_kernels/reference.py:46-58): the [B, H, Lq, Lk, D]
difference, its square and sum, `-d * scale (+ bias)`, softmax and the
product with v, each a separate kernel.  For 16-bit inputs the coefficient
is cast to the input dtype first, as the reference's benchmarks do
(kernels/benchmarks/throughput.py:129-131), so the chain stays in that dtype.

`--impl read` is a plain HBM read of the fused operator's algorithmic
bytes instead: the ceiling the hardware reaches under the same timing;
`--impl readwrite` streams the operator's reads in and its output's bytes
out in one launch (at most 8 bytes read per byte written, so not the serving
shape's 1 in 133): the ceiling of a kernel with the operator's mix.

The script runs the chosen implementation `--reps` times over rotating input
sets (after one warm-up call per set) and prints one JSON line with the
median time per call and the number of calls made.  Under
`rocprofv3 --pmc FETCH_SIZE` and `--pmc WRITE_SIZE` the counters summed
over every dispatch of the run, divided by that number of calls, are the
measured HBM bytes of one call of the region; `rocprof_summary region`
does the arithmetic.  Inputs are built on the host and copied, so the run's
only kernels are the region's own (and the runtime's copy blits, which the
summary excludes).
"""

import argparse
import json
import statistics

import torch

from vectra_amd.benchmarks import configs
import vectra_amd.kernels  # noqa: F401  (registers torch.ops.vectra.rbf_attention)


def eager_rbf_attention(q, k, v, scale, key_bias=None):
    """The unfused chain, in the inputs' dtype (reference.py:54-58)."""
    if q.dtype != torch.float32:
        scale = scale.to(q.dtype)
    sq_dist = (q.unsqueeze(-2) - k.unsqueeze(-3)).pow(2).sum(-1)
    logits = -sq_dist * scale
    if key_bias is not None:
        logits = logits + key_bias
    return torch.softmax(logits, dim=-1) @ v


def fused(q, k, v, scale, key_bias=None):
    return torch.ops.vectra.rbf_attention(q, k, v, scale, key_bias)


IMPLS = {'eager': eager_rbf_attention, 'fused': fused}


def read_region(config, batch, n_sets):
    """A plain HBM read of the fused operator's algorithmic bytes (the
    hardware's ceiling under the same one-call-at-a-time timing), one buffer
    per input set.  Buffers and the sink are built on the host and copied, so
    the only kernel of a call is the read."""
    from vectra_amd.benchmarks import read_ceiling  # pylint: disable=import-outside-toplevel
    from vectra_amd.benchmarks import roofline  # pylint: disable=import-outside-toplevel
    import dataclasses  # pylint: disable=import-outside-toplevel

    nbytes = roofline.fused_bytes(dataclasses.replace(config, batch=batch or config.batch).shape())
    nbytes = (nbytes + 15) // 16 * 16
    gen = torch.Generator().manual_seed(0)
    bufs = [torch.randint(0, 256, (nbytes,), dtype=torch.uint8, generator=gen).to('cuda') for _ in range(n_sets)]
    blocks = torch.cuda.get_device_properties(0).multi_processor_count * 8
    sink = torch.zeros(blocks * read_ceiling.THREADS, dtype=torch.int32).to('cuda')
    stream = torch.cuda.current_stream()
    return [lambda b=b: read_ceiling.read_once(b, sink, blocks, stream) for b in bufs]


def read_write_region(config, batch, n_sets):
    """One launch per call streaming the fused operator's reads in and its
    output's bytes out, one pair of buffers per input set (built on the host
    and copied, so the only kernel of a call is the stream)."""
    from vectra_amd.benchmarks import read_ceiling  # pylint: disable=import-outside-toplevel
    from vectra_amd.benchmarks import roofline  # pylint: disable=import-outside-toplevel
    import dataclasses  # pylint: disable=import-outside-toplevel

    shape = dataclasses.replace(config, batch=batch or config.batch).shape()
    out_bytes = shape.planes * shape.n_q * shape.value_dim * shape.element_bytes
    read_bytes = (roofline.fused_bytes(shape) - out_bytes + 15) // 16 * 16
    write_bytes = (out_bytes + 15) // 16 * 16
    gen = torch.Generator().manual_seed(0)
    srcs = [torch.randint(0, 256, (read_bytes,), dtype=torch.uint8, generator=gen).to('cuda') for _ in range(n_sets)]
    dsts = [torch.zeros(write_bytes, dtype=torch.uint8).to('cuda') for _ in range(n_sets)]
    blocks = torch.cuda.get_device_properties(0).multi_processor_count * 8
    sink = torch.zeros(blocks * read_ceiling.THREADS, dtype=torch.int32).to('cuda')
    stream = torch.cuda.current_stream()
    return [lambda s=s, d=d: read_ceiling.read_write_once(s, d, sink, blocks, stream) for s, d in zip(srcs, dsts)]


def main():
    p = argparse.ArgumentParser()
    p.add_argument('--impl', choices=sorted(IMPLS) + ['read', 'readwrite'], required=True)
    p.add_argument('--config', default='serving', choices=sorted(configs.CONFIGS))
    p.add_argument('--sets', type=int, default=5)
    p.add_argument('--reps', type=int, default=20)
    p.add_argument('--batch', type=int, default=None, help='first B batch entries of the config (default: all)')
    args = p.parse_args()
    config = configs.CONFIGS[args.config]
    if args.impl == 'read':
        calls_of_set = read_region(config, args.batch, args.sets)
    elif args.impl == 'readwrite':
        calls_of_set = read_write_region(config, args.batch, args.sets)
    else:
        fn = IMPLS[args.impl]
        sets = [configs.make_inputs(config, seed=s, batch=args.batch).to('cuda') for s in range(args.sets)]
        calls_of_set = [lambda s=s: fn(*s.args()) for s in sets]
    calls = 0
    for call in calls_of_set:
        call()
        calls += 1
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    times = []
    for i in range(args.reps):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        calls_of_set[i % args.sets]()
        end.record(stream)
        end.synchronize()
        calls += 1
        times.append(start.elapsed_time(end))
    print(json.dumps({
        'impl': args.impl,
        'config': config.name,
        'batch': args.batch or config.batch,
        'calls': calls,
        'median_ms': statistics.median(times),
        'dtype': str(config.dtype).replace('torch.', ''),
    }), flush=True)


if __name__ == '__main__':
    main()
