"""The practical HBM read ceiling at a workload's size (benchmark only).

Times vectra_bench_read_stream (read_ceiling.hip, in libvectra_bench.so):
a plain read of the same number of bytes as the operator's algorithmic
traffic, rotating over buffers whose total exceeds the 256 MB Infinity
Cache, with the median of trials of HIP-graph replays -- the same timing
as bench.py uses for the operator.

  python -m vectra_amd.benchmarks.read_ceiling [--bytes 68288544] [--write-bytes N]

With --write-bytes, the launch also writes N bytes, interleaved with the
reads as a kernel producing one output word from every few input words
does: the ceiling for kernels with a large write share.
"""

import argparse
import ctypes
import functools
import json
import os
import statistics

import torch

from vectra_amd.kernels import _native

BENCH_LIBRARY = os.path.join(_native.LIB_DIR, 'libvectra_bench.so')
ROTATION_BYTES = 320 << 20
THREADS = 256


@functools.cache
def _lib() -> ctypes.CDLL:
    if not os.path.exists(BENCH_LIBRARY):
        raise _native.NativeLibraryMissing(f'{BENCH_LIBRARY} is missing; build with `make -C vectra_amd/csrc`')
    lib = ctypes.CDLL(BENCH_LIBRARY)
    lib.vectra_bench_read_stream.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                            ctypes.c_int32, ctypes.c_void_p]
    lib.vectra_bench_read_stream.restype = ctypes.c_int
    lib.vectra_bench_read_write_stream.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
                                                  ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p]
    lib.vectra_bench_read_write_stream.restype = ctypes.c_int
    return lib


def read_once(buf: torch.Tensor, sink: torch.Tensor, blocks: int, stream: torch.cuda.Stream) -> None:
    nbytes = buf.numel() * buf.element_size()
    if sink.numel() < blocks * THREADS:
        raise ValueError('sink holds fewer than blocks * 256 words')
    status = _lib().vectra_bench_read_stream(buf.data_ptr(), nbytes, sink.data_ptr(), blocks,
                                             ctypes.c_void_p(stream.cuda_stream))
    if status != 0:
        raise RuntimeError(f'vectra_bench_read_stream failed with status {status}')


def read_write_once(src: torch.Tensor, dst: torch.Tensor, sink: torch.Tensor, blocks: int,
                    stream: torch.cuda.Stream) -> None:
    """One launch streaming all of `src` in and all of `dst` out."""
    read_bytes, write_bytes = src.numel() * src.element_size(), dst.numel() * dst.element_size()
    if sink.numel() < blocks * THREADS:
        raise ValueError('sink holds fewer than blocks * 256 words')
    if not 16 <= write_bytes <= read_bytes or read_bytes // write_bytes > 8 or (read_bytes | write_bytes) % 16:
        raise ValueError('needs 16-byte multiples with 16 <= write_bytes <= read_bytes <= 8 * write_bytes')
    status = _lib().vectra_bench_read_write_stream(src.data_ptr(), read_bytes, dst.data_ptr(), write_bytes,
                                                   sink.data_ptr(), blocks, ctypes.c_void_p(stream.cuda_stream))
    if status != 0:
        raise RuntimeError(f'vectra_bench_read_write_stream failed with status {status}')


def measure(nbytes: int, trials: int = 20, per_trial: int = 100, blocks: int | None = None) -> dict:
    """Median time of one read of `nbytes` from HBM, in a HIP graph."""
    nbytes = (nbytes + 15) // 16 * 16
    n_bufs = max(5, -(-ROTATION_BYTES // nbytes))
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device='cuda').random_() for _ in range(n_bufs)]
    if blocks is None:
        blocks = torch.cuda.get_device_properties(0).multi_processor_count * 8
    sink = torch.zeros(blocks * THREADS, dtype=torch.int32, device='cuda')
    stream = torch.cuda.current_stream()
    for i in range(n_bufs):
        read_once(bufs[i], sink, blocks, stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):  # captures on torch's own side stream
        capture = torch.cuda.current_stream()
        for i in range(per_trial):
            read_once(bufs[i % n_bufs], sink, blocks, capture)
    graph.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(trials):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        graph.replay()
        end.record(stream)
        end.synchronize()
        times.append(start.elapsed_time(end) / per_trial)
    ms = statistics.median(times)
    return {
        'bytes': nbytes,
        'us': ms * 1e3,
        'GB/s': nbytes / (ms / 1e3) / 1e9,
        'blocks': blocks,
        'buffers': n_bufs,
        'trials': trials,
        'launches_per_trial': per_trial,
    }


def measure_read_write(read_bytes: int, write_bytes: int, trials: int = 20, per_trial: int = 100,
                       blocks: int | None = None) -> dict:
    """Median time of one launch that streams `read_bytes` in and
    `write_bytes` out (vectra_bench_read_write_stream), in a HIP graph over
    rotating buffers: the practical ceiling of a kernel with that mix."""
    read_bytes = (read_bytes + 15) // 16 * 16
    write_bytes = (write_bytes + 15) // 16 * 16
    if not 16 <= write_bytes <= read_bytes or read_bytes // write_bytes > 8:
        raise ValueError('needs 16 <= write_bytes <= read_bytes <= 8 * write_bytes')
    n_sets = max(5, -(-ROTATION_BYTES // (read_bytes + write_bytes)))
    srcs = [torch.empty(read_bytes, dtype=torch.uint8, device='cuda').random_() for _ in range(n_sets)]
    dsts = [torch.empty(write_bytes, dtype=torch.uint8, device='cuda') for _ in range(n_sets)]
    if blocks is None:
        blocks = torch.cuda.get_device_properties(0).multi_processor_count * 8
    sink = torch.zeros(blocks * THREADS, dtype=torch.int32, device='cuda')

    def launch(i, stream):
        read_write_once(srcs[i], dsts[i], sink, blocks, stream)

    stream = torch.cuda.current_stream()
    for i in range(n_sets):
        launch(i, stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        capture = torch.cuda.current_stream()
        for i in range(per_trial):
            launch(i % n_sets, capture)
    graph.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(trials):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        graph.replay()
        end.record(stream)
        end.synchronize()
        times.append(start.elapsed_time(end) / per_trial)
    ms = statistics.median(times)
    total = read_bytes + write_bytes
    return {'read_bytes': read_bytes, 'write_bytes': write_bytes, 'us': ms * 1e3, 'GB/s': total / (ms / 1e3) / 1e9,
            'blocks': blocks, 'buffers': n_sets, 'trials': trials, 'launches_per_trial': per_trial}


def main():
    p = argparse.ArgumentParser()
    p.add_argument('--bytes', type=int, default=68288544)
    p.add_argument('--write-bytes', type=int, default=0,
                   help='also write this many bytes in the same launch (read + write ceiling)')
    p.add_argument('--blocks', type=int, default=None)
    args = p.parse_args()
    if args.write_bytes:
        print(json.dumps(measure_read_write(args.bytes, args.write_bytes, blocks=args.blocks)))
    else:
        print(json.dumps(measure(args.bytes, blocks=args.blocks)))


if __name__ == '__main__':
    main()
