"""A CPU model of scan_top_k_kernel's selection (vectra_amd/csrc/scan/scan.hip).

The kernel keeps the k best 64-bit keys of a candidate list in an LDS buffer
of KEYS slots: the k best so far in keys[0 .. k), the candidates that beat
the k-th since the last merge appended at keys[k ..].  After every round of
`round_len` candidates it decides whether to select (sort and keep the first
k), and it selects once more at the end; the split form runs this per range
and then merges the ranges' lists.  This module restates that control flow
in numpy, step for step, so that its branch logic (when a merge happens, which
selection runs, what an overflow merge leaves behind) can be checked on the
CPU against a plain sort of the candidates:

    round loop      scan.hip scan_top_k_kernel, the `for (base ...)` loop
    merge trigger   `(worst == kNoKey && n >= k) || n > kTopKKeys - k - round`
    first_select    one wave sorts the <= 64 new keys into keys[0 .. 64)
    wave_select     one wave sorts keys[0 .. k + n) (k + n <= 64), or each
                    wave the k best of its 64 candidates, then one wave those
    merge           bitonic sort of keys[0 .. k + n), padded to a power of 2
    split merge     k-way merge of the ranges' sorted lists (k, splits <= 64)
                    or a full sort of them

Which selection runs first is the point of the model.  `first_select` is only
right while keys[0 .. k) is still empty; `empty_test='merged'` (the kernel's
rule: nothing selected yet in this range) keeps that so, `empty_test='worst'`
(the k-th key still empty) does not after an overflow merge that kept fewer
than k keys.  The reference semantics being modelled: ShardIndex's bounded
heap (engine/src/index/shard_index.cc:111-120, PushBounded) over the
candidates ExhaustiveSearch visits (:236-264), which skips nodes past the
published count (:245); a multiset of the k smallest (distance, node) keys is
exactly what that heap keeps.
"""

import numpy as np

KEYS = 2048                      # kTopKKeys
NO_KEY = np.uint64(0xFFFFFFFFFFFFFFFF)  # kNoKey: an empty slot
WAVE = 64                        # kWaveLanes

# (threads, candidates per group, steps) of each kernel instance and the
# round length it gives: groups = threads / 16, round = groups * cands * steps.
FORMS = {
    'split': (256, 4, 1),      # the split form (vectra_scan_top_k_ws / no_alloc)
    'narrow': (256, 4, 4),     # 1024 queries or more
    'wide': (1024, 6, 1),      # fewer queries, one workgroup each (any dimension)
    'wide128': (1024, 4, 1),   # the same for 128-dimensional rows (the pipelined kernel)
}


def round_len(form):
    threads, cands, steps = FORMS[form]
    return threads // 16 * cands * steps


def _select(keys, k, n, first, rnd, threads):
    """select(first, n): first_select when a round fits one wave; else, in
    kernels whose rounds exceed a wave, the wave sorts (wave_select: k + n <=
    64 in one wave, or a first selection of at most one candidate per thread
    with k <= 64 / waves, each wave keeping the k best of its 64 and one wave
    sorting those lists); else merge."""
    if rnd <= WAVE and first and n <= WAVE:
        lanes = np.full(WAVE, NO_KEY, dtype=np.uint64)
        lanes[:n] = keys[k:k + n]
        lanes.sort()
        m = min(k, WAVE)
        keys[:m] = lanes[:m]
        return
    waves = threads // WAVE
    if rnd <= WAVE:
        pass  # the split form's kernel has no wave_select
    elif k + n <= WAVE:
        lanes = np.full(WAVE, NO_KEY, dtype=np.uint64)
        lanes[:k + n] = keys[:k + n]
        lanes.sort()
        keys[:k] = lanes[:k]
        return
    elif first and n <= threads and waves * k <= WAVE:
        lanes = np.full(threads, NO_KEY, dtype=np.uint64)
        lanes[:n] = keys[k:k + n]
        per_wave = np.sort(lanes.reshape(waves, WAVE), axis=1)[:, :k]
        keys[:waves * k] = per_wave.reshape(-1)
        best = np.full(WAVE, NO_KEY, dtype=np.uint64)
        best[:waves * k] = keys[:waves * k]
        best.sort()
        keys[:k] = best[:k]
        return
    size = 2
    while size < k + n:
        size <<= 1
    assert size <= KEYS, (size, k, n)
    keys[k + n:size] = NO_KEY
    keys[:size] = np.sort(keys[:size])


def range_k_best(cand_keys, k, form, empty_test='merged'):
    """The k best keys one workgroup keeps from `cand_keys` (its range, in
    candidate order; None marks a candidate it skips, an id past the rows).

    Returns the workgroup's keys[0 .. k) after its last selection."""
    rnd = round_len(form)
    assert KEYS - 1024 >= rnd
    keys = np.full(KEYS, NO_KEY, dtype=np.uint64)
    fill = 0
    worst = NO_KEY
    merged = False
    for base in range(0, len(cand_keys), rnd):
        for key in cand_keys[base:base + rnd]:
            if key is not None and np.uint64(key) < worst:
                keys[k + fill] = key
                fill += 1
        n = fill
        if (worst == NO_KEY and n >= k) or n > KEYS - k - rnd:
            first = (not merged) if empty_test == 'merged' else (worst == NO_KEY)
            _select(keys, k, n, first, rnd, FORMS[form][0])
            merged = True
            fill = 0
            worst = keys[k - 1]
    if fill > 0:
        first = (not merged) if empty_test == 'merged' else (worst == NO_KEY)
        _select(keys, k, fill, first, rnd, FORMS[form][0])
    return keys[:k].copy()


def merge_ranges(parts, k):
    """The last workgroup's merge of `parts` (one sorted k-key list per
    range): k-way over one wave's lanes when k and the range count are at
    most 64 (the smallest head k times, the lowest range on a tie), else a
    sort of every key."""
    splits = len(parts)
    if k <= WAVE and splits <= WAVE:
        pos = [0] * splits
        out = np.full(k, NO_KEY, dtype=np.uint64)
        for r in range(k):
            heads = [parts[i][pos[i]] if pos[i] < k else NO_KEY for i in range(splits)]
            win = int(np.argmin(np.array(heads, dtype=np.uint64)))  # lowest index on a tie
            out[r] = heads[win]
            pos[win] += 1
        return out
    return np.sort(np.concatenate(parts))[:k]


def split_ranges(num_cand, k, queries=1):
    """(splits, split_len) of the split form (scan.hip top_k_splits and
    use_workspace): ranges of at least 64 candidates, at most 64 of them,
    splits * next_pow2(k) <= KEYS."""
    if queries < 1 or queries >= 64:
        return 1, num_cand
    kp = 1
    while kp < k:
        kp <<= 1
    s = min(KEYS // kp, 64, (num_cand + 63) // 64)
    if s < 2:
        return 1, num_cand
    return s, (num_cand + s - 1) // s


def top_k(cand_keys, k, form='split', empty_test='merged'):
    """The kernel's result for one query: its k best keys in order."""
    if form == 'split':
        splits, length = split_ranges(len(cand_keys), k)
        if splits > 1:
            parts = [range_k_best(cand_keys[s * length:(s + 1) * length], k, form, empty_test)
                     for s in range(splits)]
            return merge_ranges(parts, k)
    return range_k_best(list(cand_keys), k, form, empty_test)


def sorted_k(cand_keys, k):
    """What the bounded heap keeps: the k smallest keys, padded with empty slots."""
    live = np.array([c for c in cand_keys if c is not None], dtype=np.uint64)
    out = np.full(k, NO_KEY, dtype=np.uint64)
    live.sort()
    m = min(k, live.size)
    out[:m] = live[:m]
    return out


def candidate_keys(distances, nodes, valid):
    """Keys as nearest_key builds them (distance order above the node id) for
    finite non-negative distances; None where the candidate is skipped."""
    d = np.asarray(distances, dtype=np.float32)
    assert np.all(d >= 0) and np.all(np.isfinite(d))
    ordered = d.view(np.uint32).astype(np.uint64) | np.uint64(0x80000000)
    keys = (ordered << np.uint64(32)) | np.asarray(nodes, dtype=np.uint64)
    return [int(key) if ok else None for key, ok in zip(keys, valid)]
