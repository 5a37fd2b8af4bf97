"""Writes tests/golden/scan_golden.npz: inputs and the reference engine's own
outputs for its distance functions and for the selection of
ShardIndex::ExhaustiveSearch (the k nearest under CloserFirst).

The outputs come from the reference sources themselves (engine/src/index/
simd_distance.cc and pq_codec.cc under /root/reference), compiled by
oracle/Makefile into oracle/_ref/libref_scan.so and called through its C shim
(oracle/ref_scan_shim.cc).  The fixture lets the oracle and the HIP kernels be
checked against the reference where /root/reference is absent (the GPU box).

    make -C oracle && python tests/golden/make_scan_golden.py
"""

import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
REF = os.path.join(ROOT, 'oracle', '_ref', 'libref_scan.so')
OUT = os.path.join(ROOT, 'tests', 'golden', 'scan_golden.npz')

ROW_DIMS = (0, 1, 2, 7, 15, 16, 17, 31, 32, 33, 63, 64, 100, 127, 128, 129, 255, 300)
ADC_SUBSPACES = (1, 2, 3, 4, 5, 8, 16, 17, 32, 64)
TABLE_SHAPES = ((128, 16), (96, 32), (40, 8), (18, 1), (64, 2))
ROWS = 24
# (rows, dimension, k, with candidate ids)
NEAREST_CASES = ((200, 32, 50, False), (300, 17, 30, True), (40, 128, 100, False), (25, 0, 10, False),
                 (120, 64, 120, True))


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def main():
    lib = ctypes.CDLL(REF)
    rng = np.random.default_rng(20251202)
    arrays = {}
    for dim in ROW_DIMS:
        # Values over several binades, some rows far from the query.
        scale = np.exp2(rng.integers(-6, 7, size=(ROWS, 1))).astype(np.float32)
        rows = (rng.standard_normal((ROWS, dim)) * scale).astype(np.float32)
        query = rng.standard_normal(dim).astype(np.float32)
        arrays[f'rows_{dim}'] = rows
        arrays[f'query_{dim}'] = query
        for metric, name in ((0, 'l2'), (1, 'ip'), (2, 'norm')):
            out = np.zeros(ROWS, np.float32)
            lib.ref_scan_rows(metric, _p(query), _p(rows), ctypes.c_int64(ROWS), ctypes.c_int64(max(dim, 1)), dim,
                              _p(out))
            arrays[f'{name}_{dim}'] = out
    for m in ADC_SUBSPACES:
        table = (rng.standard_normal(m * 256) * 10).astype(np.float32)
        codes = rng.integers(0, 256, (ROWS, m), dtype=np.uint8)
        out = np.zeros(ROWS, np.float32)
        lib.ref_pq_adc_rows(_p(table), _p(codes), ctypes.c_int64(ROWS), ctypes.c_int64(m), m, _p(out))
        arrays[f'adc_table_{m}'] = table
        arrays[f'adc_codes_{m}'] = codes
        arrays[f'adc_{m}'] = out
    for dim, m in TABLE_SHAPES:
        books = rng.standard_normal(dim * 256).astype(np.float32)
        query = rng.standard_normal(dim).astype(np.float32)
        table = np.zeros(m * 256, np.float32)
        assert lib.ref_pq_distance_table(dim, m, _p(books), _p(query), _p(table)) == 0
        arrays[f'books_{dim}_{m}'] = books
        arrays[f'tquery_{dim}_{m}'] = query
        arrays[f'table_{dim}_{m}'] = table
    # The k nearest (CloserFirst, search_scratch.h) among candidates: ids with
    # duplicates and ids past the row count (ExhaustiveSearch skips those,
    # shard_index.cc:245), rows repeated so that distances tie, and k above
    # the candidate count.  Drawn after everything above, so those arrays
    # are unchanged.
    for case, (n, dim, k, with_ids) in enumerate(NEAREST_CASES):
        rows = rng.standard_normal((n, dim)).astype(np.float32)
        rows[n // 2:n // 2 + n // 10] = rows[:n // 10]  # exact copies: equal distances
        query = rng.standard_normal(dim).astype(np.float32)
        if with_ids:
            ids = rng.integers(0, n + n // 4, size=n, dtype=np.uint32)  # some past the row count
            ids[: n // 8] = ids[n // 8: 2 * (n // 8)]  # duplicated candidates
        else:
            ids = np.arange(n, dtype=np.uint32)
        cand = ids[ids < n]
        dist = np.zeros(n, np.float32)
        lib.ref_scan_rows(0, _p(query), _p(rows), ctypes.c_int64(n), ctypes.c_int64(max(dim, 1)), dim, _p(dist))
        cand_dist = np.ascontiguousarray(dist[cand.astype(np.int64)])
        out_d = np.zeros(k, np.float32)
        out_n = np.zeros(k, np.uint32)
        lib.ref_nearest.restype = ctypes.c_int64
        m = lib.ref_nearest(_p(cand_dist), _p(cand), ctypes.c_int64(cand.shape[0]), ctypes.c_int64(k), _p(out_d),
                            _p(out_n))
        arrays[f'near_rows_{case}'] = rows
        arrays[f'near_query_{case}'] = query
        arrays[f'near_ids_{case}'] = ids if with_ids else np.zeros(0, np.uint32)
        arrays[f'near_k_{case}'] = np.array(k)
        arrays[f'near_dist_{case}'] = out_d[:m]
        arrays[f'near_node_{case}'] = out_n[:m]
    np.savez_compressed(OUT, **arrays)
    print('wrote', OUT, os.path.getsize(OUT), 'bytes')


if __name__ == '__main__':
    main()
