"""The HIP distance scans (libvectra_scan.so) against the reference's own
outputs and the CPU restatement, bit for bit (GPU).

Every comparison is on the float32 bit patterns: the kernels keep the
reference's order of operations (engine/src/index/simd_distance.cc), so any
difference is a bug, not rounding.  NaN outputs (invalid candidate ids, NaN
inputs) are compared as NaN.
"""

import os

import numpy as np
import pytest
import torch

from oracle import scan as oracle
from vectra_amd.index import scan
from vectra_amd.kernels import _native

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden', 'scan_golden.npz')


def _same(got, want, msg=''):
    got = np.asarray(got.cpu() if isinstance(got, torch.Tensor) else got, dtype=np.float32)
    want = np.asarray(want, dtype=np.float32)
    assert got.shape == want.shape, (got.shape, want.shape, msg)
    both_nan = np.isnan(got) & np.isnan(want)
    g = np.where(both_nan, 0, got.view(np.uint32))
    w = np.where(both_nan, 0, want.view(np.uint32))
    bad = np.flatnonzero(g != w)
    assert bad.size == 0, f'{msg}: {bad.size} differ, first at {bad[:5]}: {got.ravel()[bad[:5]]} vs {want.ravel()[bad[:5]]}'


def _gpu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.fixture(scope='module')
def golden():
    with np.load(GOLDEN) as data:
        return dict(data)


def test_the_scan_library_is_the_one_loaded():
    _native.scan_library()
    assert _native.SCAN_LIBRARY in _native.loaded_libraries()


def test_row_distances_equal_the_reference_outputs(golden):
    for key in [k for k in golden if k.startswith('rows_')]:
        dim = key.split('_')[1]
        rows, query = _gpu(golden[key]), _gpu(golden[f'query_{dim}'][None])
        print(f'rows dim {dim}', flush=True)
        _same(scan.l2_squared_distances(query, rows)[0], golden[f'l2_{dim}'], f'l2 dim {dim}')
        _same(scan.inner_products(query, rows)[0], golden[f'ip_{dim}'], f'ip dim {dim}')
        _same(scan.squared_norms(rows), golden[f'norm_{dim}'], f'norm dim {dim}')


def test_adc_and_tables_equal_the_reference_outputs(golden):
    for key in [k for k in golden if k.startswith('adc_codes_')]:
        m = key.rsplit('_', 1)[1]
        got = scan.pq_adc_distances(_gpu(golden[f'adc_table_{m}'][None]), _gpu(golden[key]))
        _same(got[0], golden[f'adc_{m}'], f'adc m {m}')
    for key in [k for k in golden if k.startswith('books_')]:
        _, dim, m = key.split('_')
        got = scan.pq_distance_tables(_gpu(golden[f'tquery_{dim}_{m}'][None]), _gpu(golden[key]), int(m))
        _same(got[0], golden[f'table_{dim}_{m}'], key)


@pytest.mark.parametrize('dim', [1, 5, 16, 17, 64, 100, 128, 129, 257, 1000])
@pytest.mark.parametrize('queries', [1, 3, 4, 9])
def test_row_scans_against_the_oracle(dim, queries):
    rng = np.random.default_rng(dim * 31 + queries)
    n = 3001
    rows = (rng.standard_normal((n, dim)) * np.exp2(rng.integers(-8, 9, size=(n, 1)))).astype(np.float32)
    q = rng.standard_normal((queries, dim)).astype(np.float32)
    print(f'dim {dim} queries {queries}', flush=True)
    _same(scan.l2_squared_distances(_gpu(q), _gpu(rows)), oracle.distances(q, rows, 'l2'), 'l2')
    _same(scan.inner_products(_gpu(q), _gpu(rows)), oracle.distances(q, rows, 'ip'), 'ip')
    _same(scan.squared_norms(_gpu(rows)), oracle.squared_norms(rows), 'norm')


# Several queries over 128-dimensional rows take the capped-grid kernel with
# the queries in registers.
@pytest.mark.parametrize('dim', [77, 128])
def test_strided_rows_and_queries_and_candidate_ids(dim):
    rng = np.random.default_rng(5)
    n = 2000
    wide = torch.from_numpy(rng.standard_normal((n, dim + 19)).astype(np.float32)).cuda()
    rows = wide[:, 3:3 + dim]                  # row stride dim + 19, offset 3 elements
    qwide = torch.from_numpy(rng.standard_normal((6, dim + 53)).astype(np.float32)).cuda()
    queries = qwide[:, 10:10 + dim]
    ids_np = rng.integers(0, n, 700).astype(np.int32)
    ids_np[[0, 5, 9]] = [n, n + 1000, 2**31 - 1]  # past the rows: NaN, and nothing read
    ids_np[10:20] = ids_np[20]                  # repeats
    ids = torch.from_numpy(ids_np).cuda()
    want_ids = ids_np.astype(np.int64)
    valid = want_ids < n
    rows_np, q_np = rows.cpu().numpy(), queries.cpu().numpy()
    want = np.full((6, 700), np.nan, np.float32)
    want[:, valid] = oracle.distances(q_np, rows_np, 'l2', want_ids[valid])
    got = scan.l2_squared_distances(queries, rows, ids=ids)
    _same(got, want, 'strided l2 with ids')
    assert torch.isnan(got[:, [0, 5, 9]]).all()
    # uint32 ids and a caller-provided output
    out = torch.full((6, 700), 7.0, device='cuda')
    scan.inner_products(queries, rows, ids=ids.view(torch.uint32), out=out)
    want_ip = np.full((6, 700), np.nan, np.float32)
    want_ip[:, valid] = oracle.distances(q_np, rows_np, 'ip', want_ids[valid])
    _same(out, want_ip, 'strided ip with uint32 ids')


@pytest.mark.parametrize('dim,n_q', [(40, 1), (128, 5)])
def test_special_values_propagate_like_the_reference(dim, n_q):
    rows = np.ones((6, dim), np.float32)
    rows[1, 3] = np.inf
    rows[2, 20] = np.nan
    rows[3, 39] = -np.inf                       # in the tail at 40 dimensions
    rows[4, :] = 3e19                           # squares overflow to inf
    rows[5, :] = 1e-23                          # products underflow to subnormals and zero
    q = np.zeros((n_q, dim), np.float32)
    q[:, 3] = np.inf                            # inf - inf = NaN in row 1
    q[1:, 7] = -2.5
    for fn, metric in ((scan.l2_squared_distances, 'l2'), (scan.inner_products, 'ip')):
        _same(fn(_gpu(q), _gpu(rows)), oracle.distances(q, rows, metric), metric)
    _same(scan.squared_norms(_gpu(rows)), oracle.squared_norms(rows), 'norm')


def test_a_full_shard_scan_equals_the_oracle():
    # One query against 2^20 rows of 128 floats (a quarter of a shard at the
    # reference's max_elements; configs/hnsw_params.textproto).
    rng = np.random.default_rng(11)
    n, dim = 1 << 20, 128
    rows = rng.standard_normal((n, dim), dtype=np.float32)
    q = rng.standard_normal((1, dim), dtype=np.float32)
    got = scan.l2_squared_distances(_gpu(q), _gpu(rows))
    _same(got[0], oracle.l2_squared(q[0], rows), 'shard scan')


@pytest.mark.parametrize('m', [1, 2, 3, 4, 5, 7, 8, 16, 17, 31, 32, 64, 65, 100, 256])
def test_adc_scans_against_the_oracle(m):
    rng = np.random.default_rng(m)
    n, queries = 4099, 3
    tables = (rng.standard_normal((queries, m * 256)) * 20).astype(np.float32)
    codes = rng.integers(0, 256, (n, m), dtype=np.uint8)
    got = scan.pq_adc_distances(_gpu(tables), _gpu(codes))
    want = np.stack([oracle.pq_adc(tables[i], codes) for i in range(queries)])
    print(f'adc m {m}', flush=True)
    _same(got, want, f'adc m {m}')


@pytest.mark.parametrize('m', [1, 3, 4, 5, 8, 13, 16, 17, 20, 29, 32])
def test_adc_short_codes_on_16_byte_boundaries(m):
    # Codes of <= 32 bytes with a 16-byte-aligned base and stride take the
    # kernel's 16-byte-load path (the next codes requested before the
    # current ones are summed).
    rng = np.random.default_rng(100 + m)
    n = 5003
    wide = torch.from_numpy(rng.integers(0, 256, (n, 48), dtype=np.uint8)).cuda()
    codes = wide[:, :m]                        # stride 48 bytes
    tables = (rng.standard_normal((2, m * 256)) * 3).astype(np.float32)
    ids_np = rng.integers(0, n, 1501).astype(np.int32)
    ids_np[3] = n + 7
    codes_np = codes.cpu().numpy()
    got = scan.pq_adc_distances(_gpu(tables), codes)
    want = np.stack([oracle.pq_adc(tables[i], codes_np) for i in range(2)])
    _same(got, want, f'aligned adc m {m}')
    got_ids = scan.pq_adc_distances(_gpu(tables), codes, ids=torch.from_numpy(ids_np).cuda())
    want_ids = np.full((2, 1501), np.nan, np.float32)
    ok = ids_np < n
    for i in range(2):
        want_ids[i, ok] = oracle.pq_adc(tables[i], codes_np[ids_np[ok]])
    _same(got_ids, want_ids, f'aligned adc m {m} with ids')


def test_adc_with_unaligned_codes_and_ids():
    rng = np.random.default_rng(2)
    n, m = 3000, 16
    wide = torch.from_numpy(rng.integers(0, 256, (n, 19), dtype=np.uint8)).cuda()
    codes = wide[:, 1:1 + m]                   # stride 19 bytes, base offset 1: byte loads
    tables = (rng.standard_normal((2, m * 256)) * 5).astype(np.float32)
    ids_np = rng.integers(0, n, 500).astype(np.int32)
    ids_np[7] = n                               # past the codes: NaN
    got = scan.pq_adc_distances(_gpu(tables), codes, ids=torch.from_numpy(ids_np).cuda())
    codes_np = codes.cpu().numpy()
    want = np.full((2, 500), np.nan, np.float32)
    ok = ids_np < n
    for i in range(2):
        want[i, ok] = oracle.pq_adc(tables[i], codes_np[ids_np[ok]])
    _same(got, want, 'unaligned adc with ids')


def test_adc_stream_over_several_grid_strides():
    # The 16-byte ADC kernel (the engine's 16 sub-spaces) over more codes
    # than one pass of its grid covers, ending mid-stride; a table whose rows
    # start 4 bytes past a 16-byte boundary (staged word by word); ids past
    # the codes; and ids into an empty code set (every distance NaN).
    rng = np.random.default_rng(31)
    m, n = 16, (1 << 20) + 12345
    codes = rng.integers(0, 256, (n, m), dtype=np.uint8)
    wide = (rng.standard_normal((2, m * 256 + 3)) * 7).astype(np.float32)
    tables_np = np.ascontiguousarray(wide[:, 1:1 + m * 256])
    tables = _gpu(wide)[:, 1:1 + m * 256]
    assert tables.data_ptr() % 16 == 4
    codes_gpu = _gpu(codes)
    print(f'adc stream n {n}', flush=True)
    got = scan.pq_adc_distances(tables, codes_gpu)
    _same(got, np.stack([oracle.pq_adc(tables_np[i], codes) for i in range(2)]), 'adc stream')
    ids_np = rng.integers(0, n + n // 50, 700_001).astype(np.int32)
    got = scan.pq_adc_distances(tables, codes_gpu, ids=torch.from_numpy(ids_np).cuda())
    want = np.full((2, ids_np.shape[0]), np.nan, np.float32)
    ok = ids_np < n
    assert 0 < (~ok).sum() < ok.sum()
    for i in range(2):
        want[i, ok] = oracle.pq_adc(tables_np[i], codes[ids_np[ok]])
    _same(got, want, 'adc stream with ids')
    empty = torch.zeros(0, m, dtype=torch.uint8, device='cuda')
    got = scan.pq_adc_distances(tables, empty, ids=torch.arange(5, dtype=torch.int32, device='cuda'))
    assert got.shape == (2, 5) and torch.isnan(got).all()


@pytest.mark.parametrize('dim,m', [(128, 16), (128, 8), (96, 32), (256, 8), (48, 3), (512, 16), (17, 17), (272, 8)])
def test_tables_against_the_oracle(dim, m):
    rng = np.random.default_rng(dim + m)
    books = rng.standard_normal((m, 256, dim // m)).astype(np.float32)
    queries = rng.standard_normal((5, dim)).astype(np.float32)
    got = scan.pq_distance_tables(_gpu(queries), _gpu(books), m)
    want = np.stack([oracle.pq_distance_table(queries[i], books, m) for i in range(5)])
    _same(got, want, f'tables dim {dim} m {m}')


@pytest.mark.parametrize('dim,m', [(128, 16), (64, 16), (256, 16), (512, 16), (96, 32)])
def test_tables_for_many_queries_with_strides(dim, m):
    # Blocks of 16 queries per workgroup (sub-vectors of 4, 8, 16 or 32
    # floats), a last block of 5, queries and tables with row padding.
    rng = np.random.default_rng(dim + 7 * m)
    n_q = 37
    books = rng.standard_normal((m, 256, dim // m)).astype(np.float32)
    wide_q = _gpu(rng.standard_normal((n_q, dim + 3)).astype(np.float32))
    queries = wide_q[:, 2:2 + dim]
    out = torch.full((n_q, m * 256 + 9), 7.0, device='cuda')
    got = scan.pq_distance_tables(queries, _gpu(books), m, out=out[:, :m * 256])
    q_np = queries.cpu().numpy()
    want = np.stack([oracle.pq_distance_table(q_np[i], books, m) for i in range(n_q)])
    print(f'tables dim {dim} m {m} queries {n_q}', flush=True)
    _same(got, want, f'tables dim {dim} m {m}')
    assert (out[:, m * 256:] == 7.0).all()


def test_tables_then_adc_rank_like_the_reference_search():
    # ComputeDistanceTable then PqAdcDistance over every code, as
    # engine/tests/tools/index_study.cc:79-83 does per query.
    rng = np.random.default_rng(9)
    dim, m, n = 128, 16, 20000
    books = rng.standard_normal((m, 256, dim // m)).astype(np.float32)
    queries = rng.standard_normal((4, dim)).astype(np.float32)
    codes = rng.integers(0, 256, (n, m), dtype=np.uint8)
    tables = scan.pq_distance_tables(_gpu(queries), _gpu(books), m)
    got = scan.pq_adc_distances(tables, _gpu(codes))
    want = np.stack([oracle.pq_adc(oracle.pq_distance_table(queries[i], books, m), codes) for i in range(4)])
    _same(got, want, 'tables + adc')


def test_empty_inputs():
    rows = torch.zeros(0, 16, device='cuda')
    assert scan.l2_squared_distances(torch.zeros(2, 16, device='cuda'), rows).shape == (2, 0)
    assert scan.squared_norms(rows).shape == (0,)
    assert scan.pq_adc_distances(torch.zeros(1, 256, device='cuda'),
                                 torch.zeros(0, 1, dtype=torch.uint8, device='cuda')).shape == (1, 0)
    zero_dim = scan.l2_squared_distances(torch.zeros(1, 0, device='cuda'), torch.zeros(5, 0, device='cuda'))
    assert zero_dim.tolist() == [[0.0] * 5]


# Exhaustive k-nearest search (vectra_scan_top_k).

def _check_nearest(query, rows, k, ids=None, msg=''):
    """Every entry point's (distances, nodes) against the oracle: nodes
    exactly, distances bit for bit (NaN as NaN).  Below 64 queries the split
    form spreads a query over several workgroups; the others keep one."""
    want_d, want_n = oracle.nearest(query, rows, k, ids)
    for form in scan.TOP_K_FORMS:
        print(f'  form={form}', flush=True)
        got_d, got_n = scan.nearest(_gpu(query), _gpu(rows), k, None if ids is None else _gpu(ids), form=form)
        np.testing.assert_array_equal(got_n.cpu().numpy(), want_n, err_msg=f'{msg} {form}')
        _same(got_d, want_d, f'{msg} {form}')


def test_nearest_equals_the_reference_outputs(golden):
    for case in sorted(int(k.split('_')[2]) for k in golden if k.startswith('near_k_')):
        ids = golden[f'near_ids_{case}']
        query, rows, k = golden[f'near_query_{case}'][None], golden[f'near_rows_{case}'], int(golden[f'near_k_{case}'])
        print(f'nearest fixture case {case}', flush=True)
        got_d, got_n = scan.nearest(_gpu(query), _gpu(rows), k, _gpu(ids) if ids.size else None)
        want_d, want_n = golden[f'near_dist_{case}'], golden[f'near_node_{case}']
        m = want_n.shape[0]
        np.testing.assert_array_equal(got_n.cpu().numpy()[0, :m], want_n, err_msg=f'case {case}')
        _same(got_d[0, :m], want_d, f'case {case}')
        assert (got_n.cpu().numpy()[0, m:] == scan.NO_NODE).all() and torch.isinf(got_d[0, m:]).all()


# Up to 1023 queries take 16-wave workgroups, from 1024 on 4-wave ones; k up
# to 64 / waves takes the wave-sort first selection (4 and 16 here), 17 the
# LDS sort.
@pytest.mark.parametrize('n,dim,k,queries', [(2048, 128, 10, 4), (2048, 128, 100, 2), (700, 17, 1, 3),
                                             (5000, 32, 1024, 2), (300, 300, 64, 2), (100, 0, 20, 2),
                                             (1, 8, 5, 1), (30, 16, 1024, 1), (300, 24, 16, 1100),
                                             (2048, 128, 10, 1024), (5000, 128, 1024, 2), (2999, 128, 7, 1030),
                                             (3001, 128, 64, 3), (3001, 128, 4, 5), (2048, 128, 16, 1024),
                                             (2048, 128, 17, 1024), (2050, 128, 33, 1031), (3000, 128, 1024, 1025)])
def test_nearest_against_the_oracle(n, dim, k, queries):
    rng = np.random.default_rng(n + dim + k)
    rows = rng.standard_normal((n, dim)).astype(np.float32)
    rows[n // 2: n // 2 + n // 10] = rows[: n // 10]  # equal distances, ranked by node
    q = rng.standard_normal((queries, dim)).astype(np.float32)
    print(f'nearest n={n} dim={dim} k={k} queries={queries}', flush=True)
    _check_nearest(q, rows, k, msg=f'n={n} dim={dim} k={k}')


def test_nearest_for_many_queries_with_candidate_ids():
    """From 1024 queries up (4-wave workgroups, 128-dimensional rows in the
    pipelined kernel): an odd query count, two equal queries, candidate ids
    with duplicates, ids past the row count and NaN and infinite distances,
    k from 1 to 1024 (overflow merges)."""
    rng = np.random.default_rng(41)
    n = 1500
    rows = rng.standard_normal((n, 128)).astype(np.float32)
    rows[5, 3] = np.nan
    rows[6, 0] = np.inf
    q = rng.standard_normal((1027, 128)).astype(np.float32)
    q[1] = q[0]  # equal keys for two queries
    ids = rng.integers(0, n + 300, 2400).astype(np.uint32)
    ids[:100] = ids[100:200]
    ids[200:202] = [5, 6]
    for k in (1, 10, 1000, 1024):
        print(f'nearest ids queries=1027 k={k}', flush=True)
        _check_nearest(q, rows, k, ids=ids, msg=f'k={k}')


# 128-dimensional rows take the pipelined kernels (two register sets of rows).
@pytest.mark.parametrize('dim', [40, 128])
def test_nearest_with_candidate_ids_and_special_values(dim):
    rng = np.random.default_rng(3)
    n = 900
    rows = rng.standard_normal((n, dim)).astype(np.float32)
    rows[5, 3] = np.nan     # a NaN distance: after every number
    rows[6, 0] = np.inf     # an infinite distance
    rows[7] = 0.0
    q = rng.standard_normal((3, dim)).astype(np.float32)
    ids = rng.integers(0, n + 200, 1500).astype(np.uint32)  # some past the row count: skipped
    ids[:100] = ids[100:200]                                # duplicates: kept
    ids[200:203] = [5, 6, 7]
    for k in (1, 16, 257, 1024):
        print(f'nearest ids dim={dim} k={k}', flush=True)
        _check_nearest(q, rows, k, ids, msg=f'ids dim={dim} k={k}')
    # A query equal to a row: distance exactly 0 first.
    q2 = rows[[11]].copy()
    d, nodes = scan.nearest(_gpu(q2), _gpu(rows), 3)
    assert d[0, 0].item() == 0.0 and nodes[0, 0].item() == 11


@pytest.mark.parametrize('dim', [16, 128])
def test_nearest_keeps_up_when_every_candidate_is_better(dim):
    """Distances falling with the row index: every candidate beats the k-th
    best so far, so the kernel merges its buffer again and again."""
    n, k = 6000, 1024
    rng = np.random.default_rng(9)
    q = rng.standard_normal((1, dim)).astype(np.float32)
    u = np.zeros(dim, np.float32)
    u[0] = 1.0
    rows = (q + np.outer((n - np.arange(n)) * 0.01, u)).astype(np.float32)
    _check_nearest(q, rows, k, msg='descending')


def test_nearest_over_a_large_shard():
    rng = np.random.default_rng(21)
    rows = rng.standard_normal((200_000, 128)).astype(np.float32)
    q = rng.standard_normal((2, 128)).astype(np.float32)
    print('nearest over 200k rows', flush=True)
    _check_nearest(q, rows, 10, msg='200k rows')


@pytest.mark.parametrize('dim', [24, 128])
@pytest.mark.parametrize('valid', [0, 7, 90])
def test_split_ranges_with_few_or_no_valid_candidates(valid, dim):
    """Ranges whose candidates are mostly (or all) ids past the row count:
    their lists end in empty slots, and the merge must still return exactly
    the valid candidates, then +inf and NO_NODE."""
    rng = np.random.default_rng(50 + valid)
    rows = rng.standard_normal((100, dim)).astype(np.float32)
    q = rng.standard_normal((2, dim)).astype(np.float32)
    ids = rng.integers(100, 1000, 300).astype(np.uint32)  # past the rows: skipped
    ids[rng.choice(300, valid, replace=False)] = rng.integers(0, 100, valid)
    for k in (10, 64, 100):
        print(f'split with {valid} valid candidates, k={k}', flush=True)
        assert scan.workspace_bytes(_gpu(q), _gpu(rows), k, _gpu(ids)) > 0
        _check_nearest(q, rows, k, ids, msg=f'valid={valid} k={k}')


@pytest.mark.parametrize('dim', [32, 128])
@pytest.mark.parametrize('k,length,skipped', [(1000, 1030, 30), (993, 1031, 32), (1024, 1060, 20)])
def test_split_range_merged_on_overflow_below_k(k, length, skipped, dim):
    """A range whose buffer overflows while it holds fewer than k keys (ids
    past the row count skipped among its first 1024 candidates), then a short
    last round: the range's earlier keys must survive the last selection
    (tests/topk_model.py names the case).  Two ranges of `length` ids; every
    form, no_alloc included, against the oracle."""
    rng = np.random.default_rng(k + skipped)
    n_rows = 3000
    rows = rng.standard_normal((n_rows, dim)).astype(np.float32)
    q = rng.standard_normal((1, dim)).astype(np.float32)
    ids = rng.integers(0, n_rows, 2 * length).astype(np.uint32)
    ids[rng.choice(1024, size=skipped, replace=False)] = n_rows + rng.integers(0, 500, skipped)
    assert scan.workspace_bytes(_gpu(q), _gpu(rows), k, _gpu(ids)) > 0  # the split form is taken
    print(f'split overflow below k: dim={dim} k={k} ids={2 * length} skipped={skipped}', flush=True)
    _check_nearest(q, rows, k, ids, msg=f'overflow k={k}')


def test_split_workspace_is_reused_across_calls():
    """One workspace over calls of different sizes: each call leaves its
    arrival counters at zero, so the next one's merges start clean."""
    rng = np.random.default_rng(17)
    rows = rng.standard_normal((6000, 64)).astype(np.float32)
    cases = [(5, 6000, 100), (1, 300, 10), (63, 2048, 7), (2, 6000, 1024), (1, 65, 1), (4, 4000, 33)]
    args = [(rng.standard_normal((n_q, 64)).astype(np.float32), n, k) for n_q, n, k in cases]
    need = max(scan.workspace_bytes(_gpu(q), _gpu(rows[:n]), k) for q, n, k in args)
    assert need > 0
    workspace = torch.zeros(need, dtype=torch.uint8, device='cuda')
    for q, n, k in args:
        print(f'workspace reuse: queries={q.shape[0]} rows={n} k={k}', flush=True)
        got_d, got_n = scan.nearest(_gpu(q), _gpu(rows[:n]), k, workspace=workspace)
        want_d, want_n = oracle.nearest(q, rows[:n], k)
        np.testing.assert_array_equal(got_n.cpu().numpy(), want_n)
        _same(got_d, want_d, f'rows={n} k={k}')
        torch.cuda.synchronize()
        assert not workspace[:256].any(), 'arrival counters left non-zero'


def test_nearest_matches_the_row_scan_and_a_sort():
    """The distances are the row scan's, bit for bit, and the nodes a stable
    sort of them."""
    rng = np.random.default_rng(4)
    rows = _gpu(rng.standard_normal((3000, 96)).astype(np.float32))
    q = _gpu(rng.standard_normal((5, 96)).astype(np.float32))
    d, nodes = scan.nearest(q, rows, 50)
    full = scan.l2_squared_distances(q, rows)
    order = torch.from_numpy(np.argsort(full.cpu().numpy(), axis=1, kind='stable')[:, :50])
    assert torch.equal(nodes.cpu().to(torch.int64), order)
    _same(d, torch.gather(full.cpu(), 1, order))


@pytest.mark.parametrize('form', scan.TOP_K_FORMS)
def test_an_empty_candidate_list_selects_nothing(form):
    """An empty ids tensor (whose data pointer is NULL) means no candidates, not
    every row: the NULL `ids` of the C ABI is reserved for "every row"."""
    g = torch.Generator().manual_seed(7)
    rows = torch.randn(300, 32, generator=g).cuda()
    queries = torch.randn(3, 32, generator=g).cuda()
    empty = torch.zeros(0, dtype=torch.int32, device='cuda')
    d, n = scan.nearest(queries, rows, 10, empty, form=form)
    torch.cuda.synchronize()
    assert torch.isinf(d).all() and bool((d > 0).all())
    assert bool((n.cpu().to(torch.int64) == scan.NO_NODE).all())
    want_d, want_n = oracle.nearest(queries.cpu().numpy(), rows.cpu().numpy(), 10, np.zeros(0, dtype=np.int64))
    assert np.array_equal(d.cpu().numpy(), want_d) and np.array_equal(n.cpu().numpy(), want_n)


def test_an_empty_candidate_list_scans_nothing():
    g = torch.Generator().manual_seed(8)
    rows = torch.randn(50, 16, generator=g).cuda()
    queries = torch.randn(2, 16, generator=g).cuda()
    empty = torch.zeros(0, dtype=torch.int32, device='cuda')
    for fn in (scan.l2_squared_distances, scan.inner_products):
        out = fn(queries, rows, empty)
        torch.cuda.synchronize()
        assert tuple(out.shape) == (2, 0)
    codes = torch.randint(0, 256, (40, 4), dtype=torch.uint8, generator=g).cuda()
    tables = torch.randn(2, 4 * 256, generator=g).cuda()
    out = scan.pq_adc_distances(tables, codes, empty)
    torch.cuda.synchronize()
    assert tuple(out.shape) == (2, 0)
