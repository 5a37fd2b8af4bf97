"""Pins oracle/scan.py, the CPU restatement of the engine's distance kernels.

* Bit for bit against the reference engine's own outputs: the committed
  fixture tests/golden/scan_golden.npz (made by tests/golden/
  make_scan_golden.py from the reference sources compiled into oracle/_ref),
  and, where /root/reference has been built into oracle/_ref here, against
  that library on fresh random inputs.
* The reference's own known-answer tests, restated
  (engine/tests/unit/simd_parity_test.cc:29-66): every dimension 1..300
  against a float64 sum within 1e-5 (1 + dim) (1 + |sum|), and the ADC sums of
  table[i] = (i % 97) / 4 with codes (37 s + 11) % 256.
* Planted mistakes in the restatement (a sequential instead of a pairwise
  fold, a fused multiply-add, another ADC chain order, an off-by-one tail)
  each fail the bit-level pin.
"""

import ctypes
import os

import numpy as np
import pytest

from oracle import scan

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, 'tests', 'golden', 'scan_golden.npz')
REF = os.path.join(ROOT, 'oracle', '_ref', 'libref_scan.so')


def _bits(x):
    return np.asarray(x, dtype=np.float32).view(np.uint32)


@pytest.fixture(scope='module')
def golden():
    with np.load(GOLDEN) as data:
        return dict(data)


@pytest.fixture(scope='module')
def ref():
    if not os.path.exists(REF):
        pytest.skip('oracle/_ref/libref_scan.so not built (make -C oracle, needs /root/reference)')
    return ctypes.CDLL(REF)


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _ref_rows(ref, metric, query, rows):
    out = np.zeros(rows.shape[0], np.float32)
    ref.ref_scan_rows(metric, _p(query), _p(rows), ctypes.c_int64(rows.shape[0]),
                      ctypes.c_int64(max(rows.shape[1], 1)), rows.shape[1], _p(out))
    return out


def test_row_distances_match_the_reference_fixture(golden):
    dims = sorted(int(k.split('_')[1]) for k in golden if k.startswith('rows_'))
    assert len(dims) >= 15
    for dim in dims:
        rows, query = golden[f'rows_{dim}'], golden[f'query_{dim}']
        np.testing.assert_array_equal(_bits(scan.l2_squared(query, rows)), _bits(golden[f'l2_{dim}']), err_msg=dim)
        np.testing.assert_array_equal(_bits(scan.inner_product(query, rows)), _bits(golden[f'ip_{dim}']), err_msg=dim)
        np.testing.assert_array_equal(_bits(scan.squared_norms(rows)), _bits(golden[f'norm_{dim}']), err_msg=dim)


def test_adc_and_tables_match_the_reference_fixture(golden):
    for key in [k for k in golden if k.startswith('adc_codes_')]:
        m = int(key.rsplit('_', 1)[1])
        got = scan.pq_adc(golden[f'adc_table_{m}'], golden[key])
        np.testing.assert_array_equal(_bits(got), _bits(golden[f'adc_{m}']), err_msg=m)
    for key in [k for k in golden if k.startswith('books_')]:
        _, dim, m = key.split('_')
        got = scan.pq_distance_table(golden[f'tquery_{dim}_{m}'], golden[key], int(m))
        np.testing.assert_array_equal(_bits(got), _bits(golden[f'table_{dim}_{m}']), err_msg=key)


def test_random_inputs_match_the_reference_build(ref):
    rng = np.random.default_rng(7)
    for dim in list(range(0, 70)) + [127, 128, 129, 200, 513]:
        rows = (rng.standard_normal((31, dim)) * rng.uniform(1e-3, 1e3)).astype(np.float32)
        query = rng.standard_normal(dim).astype(np.float32)
        for metric, fn in ((0, lambda: scan.l2_squared(query, rows)), (1, lambda: scan.inner_product(query, rows)),
                           (2, lambda: scan.squared_norms(rows))):
            np.testing.assert_array_equal(_bits(fn()), _bits(_ref_rows(ref, metric, query, rows)),
                                          err_msg=f'dim {dim} metric {metric}')
    for m in (1, 2, 3, 4, 6, 7, 9, 16, 31, 64, 200, 256):
        table = rng.standard_normal(m * 256).astype(np.float32) * 50
        codes = rng.integers(0, 256, (40, m), dtype=np.uint8)
        want = np.zeros(40, np.float32)
        ref.ref_pq_adc_rows(_p(table), _p(codes), ctypes.c_int64(40), ctypes.c_int64(m), m, _p(want))
        np.testing.assert_array_equal(_bits(scan.pq_adc(table, codes)), _bits(want), err_msg=m)
    for dim, m in ((128, 16), (128, 4), (48, 3), (16, 16), (272, 8), (33, 1)):
        books = rng.standard_normal(dim * 256).astype(np.float32)
        query = rng.standard_normal(dim).astype(np.float32)
        want = np.zeros(m * 256, np.float32)
        assert ref.ref_pq_distance_table(dim, m, _p(books), _p(query), _p(want)) == 0
        np.testing.assert_array_equal(_bits(scan.pq_distance_table(query, books, m)), _bits(want), err_msg=(dim, m))


def test_every_dimension_against_float64_like_the_reference_parity_test():
    # simd_parity_test.cc:29-49, with seeded normal data in place of the
    # test library's clustered vectors.
    rng = np.random.default_rng(1)
    for dim in range(1, 301):
        a, b = rng.standard_normal((2, dim)).astype(np.float32)
        l2 = float(np.sum((a.astype(np.float64) - b.astype(np.float64)) ** 2))
        dot = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
        norm = float(np.dot(a.astype(np.float64), a.astype(np.float64)))
        tol = 1e-5 * (1.0 + dim)
        assert abs(float(scan.l2_squared(a, b[None])[0]) - l2) <= tol * (1.0 + l2), dim
        assert abs(float(scan.inner_product(a, b[None])[0]) - dot) <= tol * (1.0 + abs(dot)), dim
        assert abs(float(scan.squared_norms(a[None])[0]) - norm) <= tol * (1.0 + norm), dim


@pytest.mark.parametrize('subspaces', [1, 3, 4, 8, 16, 17, 32])
def test_adc_sums_table_entries_like_the_reference_parity_test(subspaces):
    # simd_parity_test.cc:51-66.
    table = (np.arange(subspaces * 256) % 97).astype(np.float32) * np.float32(0.25)
    code = np.array([(s * 37 + 11) % 256 for s in range(subspaces)], dtype=np.uint8)
    expected = sum(float(table[s * 256 + int(code[s])]) for s in range(subspaces))
    got = float(scan.pq_adc(table, code[None])[0])
    assert abs(got - expected) <= 1e-4 * (1.0 + expected)
    # Multiples of 1/4 below 2^22: every partial sum is exact.
    assert got == expected


def test_closed_forms():
    rows = np.array([[3.0, 4.0], [0.0, 0.0]], np.float32)
    assert scan.l2_squared(np.zeros(2, np.float32), rows).tolist() == [25.0, 0.0]
    assert scan.squared_norms(rows).tolist() == [25.0, 0.0]
    assert scan.inner_product(np.array([1.0, 2.0], np.float32), rows).tolist() == [11.0, 0.0]
    # Zero dimensions: every distance is 0 (the reference adds nothing).
    assert scan.l2_squared(np.zeros(0, np.float32), np.zeros((3, 0), np.float32)).tolist() == [0.0] * 3
    # A row equal to the query.
    v = np.random.default_rng(3).standard_normal(77).astype(np.float32)
    assert scan.l2_squared(v, v[None]).tolist() == [0.0]


class _Planted:
    """The restatement with one plausible mistake, for the pins to catch."""

    @staticmethod
    def sequential_fold(query, rows):
        lanes = np.zeros((rows.shape[0], 16), np.float32)
        full = rows.shape[1] - rows.shape[1] % 16
        for i in range(0, full, 16):
            d = (query[None, i:i + 16] - rows[:, i:i + 16]).astype(np.float32)
            lanes = lanes + (d * d).astype(np.float32)
        total = np.zeros(rows.shape[0], np.float32)
        for j in range(16):
            total = total + lanes[:, j]
        for i in range(full, rows.shape[1]):
            d = (query[i] - rows[:, i]).astype(np.float32)
            total = total + (d * d).astype(np.float32)
        return total

    @staticmethod
    def fused_terms(query, rows):
        # acc + d * d rounded once (a fused multiply-add), evaluated in float64.
        lanes = np.zeros((rows.shape[0], 16), np.float32)
        full = rows.shape[1] - rows.shape[1] % 16
        for i in range(0, full, 16):
            d = (query[None, i:i + 16] - rows[:, i:i + 16]).astype(np.float32)
            lanes = (lanes.astype(np.float64) + d.astype(np.float64) ** 2).astype(np.float32)
        width, lanes = 8, lanes.copy()
        while width:
            lanes[:, :width] = lanes[:, :width] + lanes[:, width:2 * width]
            width //= 2
        total = lanes[:, 0]
        for i in range(full, rows.shape[1]):
            d = (query[i] - rows[:, i]).astype(np.float32)
            total = (total.astype(np.float64) + d.astype(np.float64) ** 2).astype(np.float32)
        return total

    @staticmethod
    def chained_adc(table, codes):
        total = np.zeros(codes.shape[0], np.float32)
        for s in range(codes.shape[1]):
            total = total + table[s * 256 + codes[:, s].astype(np.int64)]
        return total

    @staticmethod
    def tail_from_wrong_start(query, rows):
        # The tail starts one step early: the last full step is added twice.
        dim = rows.shape[1]
        out = scan.l2_squared(query, rows)
        if dim >= 16:
            extra = scan.l2_squared(query[dim - dim % 16 - 1:dim - dim % 16], rows[:, dim - dim % 16 - 1:dim - dim % 16])
            out = (out + extra).astype(np.float32)
        return out


def test_planted_mistakes_fail_the_bit_level_pin(golden):
    def mismatches(fn, key_rows, key_out):
        bad = 0
        for k in [k for k in golden if k.startswith(key_rows)]:
            dim = k.split('_')[1]
            rows, query = golden[k], golden[f'query_{dim}']
            if rows.shape[1] < 16:
                continue
            bad += not np.array_equal(_bits(fn(query, rows)), _bits(golden[f'{key_out}_{dim}']))
        return bad

    assert mismatches(_Planted.sequential_fold, 'rows_', 'l2') > 0
    assert mismatches(_Planted.fused_terms, 'rows_', 'l2') > 0
    assert mismatches(_Planted.tail_from_wrong_start, 'rows_', 'l2') > 0
    adc_bad = sum(not np.array_equal(_bits(_Planted.chained_adc(golden[f'adc_table_{m}'], golden[f'adc_codes_{m}'])),
                                     _bits(golden[f'adc_{m}']))
                  for m in (8, 16, 17, 32, 64))
    assert adc_bad > 0
    # The correct restatement matches on the same cases.
    assert mismatches(scan.l2_squared, 'rows_', 'l2') == 0


# ExhaustiveSearch's selection: the k nearest under CloserFirst.

def _nearest_case(golden, case):
    ids = golden[f'near_ids_{case}']
    return (golden[f'near_query_{case}'][None], golden[f'near_rows_{case}'], int(golden[f'near_k_{case}']),
            ids if ids.size else None, golden[f'near_dist_{case}'], golden[f'near_node_{case}'])


def test_nearest_matches_the_reference_fixture(golden):
    cases = sorted(int(k.split('_')[2]) for k in golden if k.startswith('near_k_'))
    assert len(cases) >= 5
    for case in cases:
        query, rows, k, ids, want_d, want_n = _nearest_case(golden, case)
        got_d, got_n = scan.nearest(query, rows, k, ids)
        m = want_n.shape[0]
        np.testing.assert_array_equal(_bits(got_d[0, :m]), _bits(want_d), err_msg=f'case {case}')
        np.testing.assert_array_equal(got_n[0, :m], want_n, err_msg=f'case {case}')
        # Past the candidates: empty slots.
        assert np.isposinf(got_d[0, m:]).all() and (got_n[0, m:] == scan.NO_NODE).all()


def test_nearest_matches_the_reference_build(ref):
    ref.ref_nearest.restype = ctypes.c_int64
    rng = np.random.default_rng(77)
    for n, dim, k in ((500, 24, 1), (500, 24, 37), (64, 3, 64), (1000, 130, 200)):
        rows = rng.standard_normal((n, dim)).astype(np.float32)
        rows[n // 3: n // 3 + 20] = rows[:20]  # ties
        query = rng.standard_normal(dim).astype(np.float32)
        dist = _ref_rows(ref, 0, query, rows)
        nodes = np.arange(n, dtype=np.uint32)
        want_d, want_n = np.zeros(k, np.float32), np.zeros(k, np.uint32)
        m = ref.ref_nearest(_p(dist), _p(nodes), ctypes.c_int64(n), ctypes.c_int64(k), _p(want_d), _p(want_n))
        got_d, got_n = scan.nearest(query[None], rows, k)
        np.testing.assert_array_equal(_bits(got_d[0, :m]), _bits(want_d[:m]))
        np.testing.assert_array_equal(got_n[0, :m], want_n[:m])


def test_nearest_by_brute_force():
    """Tiny cases against Python's sort of (distance, node) pairs, with the
    candidate rules written out: ids past the row count skipped, duplicates
    kept, NaN after every number."""
    rng = np.random.default_rng(5)
    for trial in range(40):
        n, dim = int(rng.integers(1, 12)), int(rng.integers(0, 6))
        rows = rng.integers(-2, 3, (n, dim)).astype(np.float32)  # small integers: many equal distances
        if trial % 5 == 0 and dim:
            rows[rng.integers(n), 0] = np.nan
        query = rng.integers(-2, 3, dim).astype(np.float32)
        ids = rng.integers(0, n + 3, int(rng.integers(0, 15))).astype(np.uint32) if trial % 2 else None
        k = int(rng.integers(1, 16))
        cand = list(range(n)) if ids is None else [int(i) for i in ids if i < n]
        pairs = []
        for node in cand:
            d = float(np.float32(sum(float(np.float32(q - r)) ** 2 for q, r in zip(query, rows[node]))))
            pairs.append((np.isnan(d), 0.0 if np.isnan(d) else d, node))
        pairs.sort()
        got_d, got_n = scan.nearest(query[None], rows, k, ids)
        for r in range(k):
            if r < len(pairs):
                nan, d, node = pairs[r]
                assert got_n[0, r] == node, (trial, r)
                assert np.isnan(got_d[0, r]) if nan else got_d[0, r] == d, (trial, r)
            else:
                assert got_n[0, r] == scan.NO_NODE and np.isposinf(got_d[0, r])


def test_a_planted_tie_mistake_fails_the_fixture(golden, monkeypatch):
    """Ties broken by descending node id (or left in scan order) fail the pin."""
    query, rows, k, ids, want_d, want_n = _nearest_case(golden, 4)
    real_lexsort = np.lexsort

    def descending_ties(keys):
        nodes, d, nan = keys
        return real_lexsort((-nodes, d, nan))
    monkeypatch.setattr(scan.np, 'lexsort', descending_ties)
    _, got_n = scan.nearest(query, rows, k, ids)
    assert not np.array_equal(got_n[0, :want_n.shape[0]], want_n)
