"""The top-k kernel's selection loop, modelled on the CPU (tests/topk_model.py),
against a plain sort of the same keys: every form (rounds of 64, 256 and 384
candidates), k across the range where an overflow merge can keep fewer than k
keys (993 ... 1024 for the split form), candidates skipped as ids past the row
count (shard_index.cc:245), and the split form's range merge.  The rule that
tells an empty buffer (nothing selected yet) from a full one is planted wrong
once (the k-th key still empty), and the case that breaks it is named."""

import numpy as np
import pytest

from tests import topk_model as model


def _case(rng, n, k, skip_frac, descending=False, dup_frac=0.0):
    d = rng.random(n).astype(np.float32)
    if descending:
        d = np.sort(d)[::-1].copy()  # every candidate beats the k-th so far
    nodes = rng.permutation(n).astype(np.uint32)
    if dup_frac:
        dup = rng.random(n) < dup_frac
        nodes[dup] = nodes[0]
        d[dup] = d[0]  # the same row visited twice: the same key, kept twice
    valid = rng.random(n) >= skip_frac
    return model.candidate_keys(d, nodes, valid)


@pytest.mark.parametrize('form', ['split', 'narrow', 'wide', 'wide128'])
@pytest.mark.parametrize('k', [1, 4, 5, 10, 16, 17, 54, 64, 65, 500, 993, 1000, 1024])
def test_the_selection_keeps_the_k_smallest(form, k):
    rng = np.random.default_rng(k * 7 + len(form))
    for n, skip, desc in ((k // 2 + 1, 0.0, False), (k + 37, 0.03, False), (2 * k + 130, 0.02, False),
                          (3000, 0.3, False), (2100, 0.0, True), (4099, 0.01, True)):
        keys = _case(rng, n, k, skip, descending=desc, dup_frac=0.01)
        got = model.top_k(keys, k, form)
        np.testing.assert_array_equal(got, model.sorted_k(keys, k), err_msg=f'{form} k={k} n={n}')


def _overflow_case(k, length, skipped):
    """One query's list over two ranges of `length` candidates each, with
    `skipped` ids past the rows among range 0's first 1024, so that range 0's
    fill after 16 rounds of 64 lands above KEYS - k - 64 but below k."""
    rng = np.random.default_rng(k + skipped)
    n = 2 * length
    d = rng.random(n).astype(np.float32)
    valid = np.ones(n, dtype=bool)
    valid[rng.choice(1024, size=skipped, replace=False)] = False
    return model.candidate_keys(d, np.arange(n, dtype=np.uint32), valid)


@pytest.mark.parametrize('k,length,skipped', [(1000, 1030, 30), (993, 1031, 32), (1024, 1060, 20), (1010, 1040, 30)])
def test_an_overflow_merge_below_k_then_a_short_last_round(k, length, skipped):
    keys = _overflow_case(k, length, skipped)
    assert model.split_ranges(len(keys), k) == (2, length)
    # Range 0 merges once on overflow with fewer than k keys in hand.
    fill = 1024 - skipped
    assert model.KEYS - k - 64 < fill < k
    want = model.sorted_k(keys, k)
    np.testing.assert_array_equal(model.top_k(keys, k, 'split'), want)
    # The same model with the emptiness test the kernel once used (the k-th
    # key still empty) drops the range's best keys: the planted rule fails.
    bad = model.top_k(keys, k, 'split', empty_test='worst')
    assert not np.array_equal(bad, want)
    lost = np.setdiff1d(want, bad)
    merged_first = np.array([c for c in keys[:1024] if c is not None], dtype=np.uint64)
    assert lost.size >= 1 and np.all(np.isin(lost, merged_first))


def test_only_the_split_form_takes_the_one_wave_first_selection():
    # Rounds of 256 and 384 always merge (keys[0 .. k) in the sort), so the
    # emptiness rule cannot matter there.
    keys = _overflow_case(1000, 1030, 30)
    for form in ('narrow', 'wide', 'wide128'):
        want = model.sorted_k(keys, 1000)
        np.testing.assert_array_equal(model.top_k(keys, 1000, form, empty_test='worst'), want)


def test_the_k_way_merge_of_ranges():
    rng = np.random.default_rng(5)
    for k, splits in ((10, 32), (64, 32), (1, 64), (33, 2)):
        parts = [np.sort(rng.integers(0, 1 << 40, k).astype(np.uint64)) for _ in range(splits)]
        parts[1][:] = parts[0]  # ties across ranges
        got = model.merge_ranges(parts, k)
        np.testing.assert_array_equal(got, np.sort(np.concatenate(parts))[:k])


def test_split_geometry_matches_the_host_rule():
    # scan.hip top_k_splits: splits * next_pow2(k) <= 2048, at most 64 ranges
    # of at least 64 candidates, none below 64 queries' worth of workgroups.
    assert model.split_ranges(2048, 10) == (32, 64)
    assert model.split_ranges(2060, 1000) == (2, 1030)
    assert model.split_ranges(100, 10) == (2, 50)
    assert model.split_ranges(64, 10) == (1, 64)
    assert model.split_ranges(5000, 1024, queries=64) == (1, 5000)
