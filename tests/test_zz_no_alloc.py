"""vectra_scan_top_k_no_alloc (the split top-k on the library's static
scratch) against vectra_scan_top_k_ws (the same kernels on a caller's
workspace): the same bits, on two calls in a row, the second smaller.  It
runs last (test_zz_*): a failure here must not hide the other tests."""

import numpy as np
import pytest
import torch

from oracle import scan as oracle
from vectra_amd.index import scan

pytestmark = pytest.mark.gpu


def _gpu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _bits(t):
    return t.cpu().contiguous().view(torch.int32).numpy()


@pytest.mark.parametrize('ids', [False, True])
def test_no_alloc_top_k_equals_the_workspace_form_twice(ids):
    rng = np.random.default_rng(29 + int(ids))
    rows = rng.standard_normal((5000, 96)).astype(np.float32)
    rows[2500:2600] = rows[:100]  # equal distances, ranked by node
    # The first call spreads 6 queries over 16 ranges each; the second is a
    # single query over fewer candidates and a smaller k.
    for n_q, n, k in ((6, 5000, 100), (1, 700, 10)):
        q = rng.standard_normal((n_q, 96)).astype(np.float32)
        cand = rng.integers(0, n + 50, 3 * n).astype(np.uint32) if ids else None  # some past the rows
        print(f'no-alloc top-k: queries={n_q} rows={n} k={k} ids={ids}', flush=True)
        args = (_gpu(q), _gpu(rows[:n]), k, None if cand is None else _gpu(cand))
        assert scan.workspace_bytes(*args) > 0  # the split form is taken
        want_d, want_n = scan.nearest(*args, form='split')
        got_d, got_n = scan.nearest(*args, form='no_alloc')
        torch.cuda.synchronize()
        assert torch.equal(got_n, want_n)
        np.testing.assert_array_equal(_bits(got_d), _bits(want_d))
        # And both against the oracle.
        o_d, o_n = oracle.nearest(q, rows[:n], k, cand)
        np.testing.assert_array_equal(got_n.cpu().numpy(), o_n)
        np.testing.assert_array_equal(_bits(got_d), np.ascontiguousarray(o_d).view(np.int32))


def test_no_alloc_top_k_with_ranges_merged_below_k():
    """Large k over two ranges whose first 1024 ids hold some past the row
    count: range 0's buffer overflows with fewer than k keys, then takes a
    short last round.  Two calls in a row, the second smaller."""
    rng = np.random.default_rng(41)
    n_rows, dim = 3000, 32
    rows = rng.standard_normal((n_rows, dim)).astype(np.float32)
    for k, length, skipped in ((1024, 1060, 20), (1000, 1030, 30)):
        q = rng.standard_normal((1, dim)).astype(np.float32)
        ids = rng.integers(0, n_rows, 2 * length).astype(np.uint32)
        ids[rng.choice(1024, size=skipped, replace=False)] = n_rows + 7
        print(f'no-alloc top-k below k: k={k} ids={2 * length} skipped={skipped}', flush=True)
        args = (_gpu(q), _gpu(rows), k, _gpu(ids))
        assert scan.workspace_bytes(*args) > 0
        want_d, want_n = scan.nearest(*args, form='split')
        got_d, got_n = scan.nearest(*args, form='no_alloc')
        torch.cuda.synchronize()
        assert torch.equal(got_n, want_n)
        np.testing.assert_array_equal(_bits(got_d), _bits(want_d))
        o_d, o_n = oracle.nearest(q, rows, k, ids)
        np.testing.assert_array_equal(got_n.cpu().numpy(), o_n)
        np.testing.assert_array_equal(_bits(got_d), np.ascontiguousarray(o_d).view(np.int32))
