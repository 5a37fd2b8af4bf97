"""The benchmark library's streaming ceilings (vectra_amd/benchmarks/read_ceiling.hip).

They are not part of the operator, but bench.py divides by their times, so
the read + write kernel is checked to move exactly the bytes it is asked to:
each output word is the XOR of the matching words of the input regions, and
nothing past the output is written.
"""

import ctypes
import os

import numpy as np
import pytest
import torch

from vectra_amd.benchmarks import read_ceiling


def _library_or_skip():
    if not os.path.exists(read_ceiling.BENCH_LIBRARY):
        pytest.skip('libvectra_bench.so is not built')
    return read_ceiling._lib()


def test_exports_both_ceilings():
    lib = _library_or_skip()
    for name in ('vectra_bench_read_stream', 'vectra_bench_read_write_stream'):
        assert hasattr(lib, name)


def test_read_write_rejects_bad_sizes():
    lib = _library_or_skip()
    buf = ctypes.create_string_buffer(256)
    ptr = (ctypes.addressof(buf) + 15) // 16 * 16
    sink = ctypes.create_string_buffer(1024 * 4)
    for read_bytes, write_bytes in ((64, 0), (32, 48), (16 * 9, 16), (40, 16)):
        # Rejected before any launch: no device memory is touched.
        assert lib.vectra_bench_read_write_stream(ptr, read_bytes, ptr, write_bytes, ctypes.addressof(sink), 1,
                                                  None) == 1


@pytest.mark.gpu
@pytest.mark.parametrize('read_words,write_words', [(3 * 1000, 1000), (3 * 1000 + 7, 1000), (4096, 4096)])
def test_read_write_writes_the_xor_of_its_regions(read_words, write_words):
    lib = _library_or_skip()
    gen = torch.Generator().manual_seed(read_words + write_words)
    src = torch.randint(0, 2 ** 31 - 1, (read_words * 4,), generator=gen, dtype=torch.int32)
    dst = torch.full((write_words * 4 + 64,), 7, dtype=torch.int32)  # a guard past the output
    src_d, dst_d = src.cuda(), dst.cuda()
    blocks = 4
    sink = torch.zeros(blocks * 256, dtype=torch.int32, device='cuda')
    print(f'read_write_stream: read {read_words} words, write {write_words}', flush=True)
    status = lib.vectra_bench_read_write_stream(src_d.data_ptr(), read_words * 16, dst_d.data_ptr(), write_words * 16,
                                                sink.data_ptr(), blocks,
                                                ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert status == 0
    torch.cuda.synchronize()
    words = src.numpy().reshape(read_words, 4)
    ratio = read_words // write_words
    want = np.zeros((write_words, 4), np.int32)
    for u in range(ratio):
        want ^= words[u * write_words:(u + 1) * write_words]
    got = dst_d.cpu().numpy()
    np.testing.assert_array_equal(got[:write_words * 4].reshape(write_words, 4), want)
    assert (got[write_words * 4:] == 7).all()
