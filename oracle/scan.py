"""CPU restatement of the engine's distance kernels (test infrastructure only).

Only tests/, __graft_entry__.smoke() and the CPU leg of the scan benchmark
import this module: it is the checker the HIP scan kernels are compared with,
never part of the product path.

The reference kernels (engine/src/index/simd_distance.cc) fix the order of
every floating-point operation, and the HIP kernels follow that order, so
the comparison is bit for bit:

* L2SquaredDistance (simd_distance.cc:36-51): sixteen float accumulators;
  element i + j of every full 16-element step goes to accumulator j as
  `acc_j = acc_j + d * d` (the product rounded to float, then the sum); the
  accumulators are folded by ReduceLanes (simd_distance.cc:27-32): widths 8,
  4, 2, 1, `lane_i = lane_i + lane_(i + width)`; the elements past the last
  full step are then added one at a time to that sum.
* InnerProduct (:53-62) and SquaredNorm (:64-66): the same with `a * b`.
* PqAdcDistance (:68-81): four chains over sub-spaces s, s+1, s+2, s+3 in
  steps of four, combined as (l0 + l1) + (l2 + l3), then the remaining
  sub-spaces one at a time.
* ProductQuantizer::ComputeDistanceTable (pq_codec.cc:208-217):
  table[s * 256 + c] = L2SquaredDistance(query sub-vector s, centroid (s, c)).

Each function here works on many rows at once with numpy float32 arrays;
numpy rounds every float32 operation to nearest-even and never fuses a
multiply into an add, which is what the reference's ISO C++ build does
(-std=c++20: GCC contracts no expressions in ISO mode).

* ShardIndex::ExhaustiveSearch's selection (shard_index.cc:236-264): the k
  nearest candidates by L2SquaredDistance, kept by PushBounded (:111-120) in
  a bounded heap ordered by CloserFirst (search_scratch.h: distance
  ascending, ties by node id), then sorted by it; candidate ids not below
  the row count are skipped (:245).  `nearest` restates it as a stable sort
  on (distance, node); NaN distances, which CloserFirst cannot order, are
  ranked after every number here, ties by node.

Pins (tests/test_scan_oracle.py): bit-for-bit against the reference sources
compiled by oracle/Makefile into oracle/_ref (where /root/reference exists),
the reference's own known-answer tests (simd_parity_test.cc:29-66), a float64
sum, and brute-force scalar loops written independently in the test.
"""

import numpy as np

LANES = 16        # accumulators of L2SquaredDistance / InnerProduct (simd_distance.cc:24)
PQ_CENTROIDS = 256  # kPqCentroids (include/vectra/index/simd_distance.h)


def _reduce_lanes(lanes):
    """ReduceLanes (simd_distance.cc:27-32) over the last axis of `lanes` [..., 16]."""
    lanes = lanes.copy()
    width = LANES // 2
    while width > 0:
        lanes[..., :width] = lanes[..., :width] + lanes[..., width:2 * width]
        width //= 2
    return lanes[..., 0]


def _lane_sum(terms, dim, n):
    """The 16-accumulator reduction of simd_distance.cc:36-62: `terms(lo, hi)`
    returns the float32 terms of elements lo .. hi - 1 of every row, [n, hi - lo]."""
    lanes = np.zeros((n, LANES), dtype=np.float32)
    full = dim - dim % LANES
    for i in range(0, full, LANES):
        lanes = lanes + terms(i, i + LANES)
    total = _reduce_lanes(lanes)
    for i in range(full, dim):
        total = total + terms(i, i + 1)[:, 0]
    return total.astype(np.float32)


def _rows_2d(query, rows):
    a = np.asarray(query, dtype=np.float32)
    b = np.asarray(rows, dtype=np.float32)
    if b.ndim == 1:
        b = b[None, :]
    assert a.shape == (b.shape[1],), (a.shape, b.shape)
    return a, b


def l2_squared(query, rows):
    """L2SquaredDistance(query, row, dim) for every row of `rows` [n, dim] -> [n] float32."""
    a, b = _rows_2d(query, rows)

    def terms(lo, hi):
        d = (a[None, lo:hi] - b[:, lo:hi]).astype(np.float32)
        return (d * d).astype(np.float32)
    return _lane_sum(terms, b.shape[1], b.shape[0])


def inner_product(query, rows):
    """InnerProduct(query, row, dim) for every row -> [n] float32."""
    a, b = _rows_2d(query, rows)
    return _lane_sum(lambda lo, hi: (a[None, lo:hi] * b[:, lo:hi]).astype(np.float32), b.shape[1], b.shape[0])


def squared_norms(rows):
    """SquaredNorm(row, dim) = InnerProduct(row, row, dim) for every row -> [n] float32."""
    b = np.asarray(rows, dtype=np.float32)
    return _lane_sum(lambda lo, hi: (b[:, lo:hi] * b[:, lo:hi]).astype(np.float32), b.shape[1], b.shape[0])


def distances(queries, rows, metric='l2', ids=None):
    """[q, n] float32: the metric from each query to each row (or to rows[ids])."""
    queries = np.asarray(queries, dtype=np.float32)
    rows = np.asarray(rows, dtype=np.float32)
    picked = rows if ids is None else rows[np.asarray(ids, dtype=np.int64)]
    fn = l2_squared if metric == 'l2' else inner_product
    out = np.zeros((queries.shape[0], picked.shape[0]), dtype=np.float32)
    for q in range(queries.shape[0]):
        if picked.shape[0]:
            out[q] = fn(queries[q], picked)
    return out


def pq_adc(table, codes):
    """PqAdcDistance(table, code, m) for every code of `codes` [n, m] uint8 -> [n] float32.

    `table` is [m * 256] float32 (sub-space major)."""
    table = np.asarray(table, dtype=np.float32).reshape(-1)
    codes = np.asarray(codes, dtype=np.uint8)
    n, m = codes.shape
    assert table.shape[0] == m * PQ_CENTROIDS, (table.shape, codes.shape)
    entry = lambda s: table[s * PQ_CENTROIDS + codes[:, s].astype(np.int64)]  # noqa: E731
    chains = [np.zeros(n, dtype=np.float32) for _ in range(4)]
    s = 0
    while s + 4 <= m:
        for c in range(4):
            chains[c] = (chains[c] + entry(s + c)).astype(np.float32)
        s += 4
    total = ((chains[0] + chains[1]).astype(np.float32) + (chains[2] + chains[3]).astype(np.float32))
    total = total.astype(np.float32)
    for r in range(s, m):
        total = (total + entry(r)).astype(np.float32)
    return total


def pq_distance_table(query, codebooks, subspaces):
    """ComputeDistanceTable (pq_codec.cc:208-217) -> [subspaces * 256] float32.

    `codebooks` is [subspaces, 256, dim / subspaces] float32 (the layout of
    ProductQuantizer::codebooks(), pq_codec.h: [subspace][centroid][dim])."""
    query = np.asarray(query, dtype=np.float32)
    dim = query.shape[0]
    dsub = dim // subspaces
    books = np.asarray(codebooks, dtype=np.float32).reshape(subspaces, PQ_CENTROIDS, dsub)
    table = np.zeros(subspaces * PQ_CENTROIDS, dtype=np.float32)
    for s in range(subspaces):
        table[s * PQ_CENTROIDS:(s + 1) * PQ_CENTROIDS] = l2_squared(query[s * dsub:(s + 1) * dsub], books[s])
    return table


NO_NODE = 0xFFFFFFFF  # node of a result slot past the candidates' count


def nearest(queries, rows, k, ids=None):
    """ExhaustiveSearch's results for each query: (distances [q, k] float32,
    nodes [q, k] uint32), nearest first by (distance, node); slots past the
    number of candidates hold +inf and NO_NODE.  Candidate ids >= len(rows)
    are skipped; duplicate ids are kept, as the reference keeps them."""
    queries = np.asarray(queries, dtype=np.float32)
    rows = np.asarray(rows, dtype=np.float32)
    nodes = np.arange(rows.shape[0], dtype=np.int64) if ids is None else np.asarray(ids, dtype=np.int64)
    nodes = nodes[nodes < rows.shape[0]]
    dist = distances(queries, rows, 'l2', nodes)
    out_d = np.full((queries.shape[0], k), np.inf, dtype=np.float32)
    out_n = np.full((queries.shape[0], k), NO_NODE, dtype=np.uint32)
    m = min(k, nodes.shape[0])
    for q in range(queries.shape[0]):
        d = dist[q]
        nan = np.isnan(d)
        # Keys (nan, distance, node): numbers before NaN, then by node.
        order = np.lexsort((nodes, np.where(nan, 0, d), nan))[:m]
        out_d[q, :m] = d[order]
        out_n[q, :m] = nodes[order]
    return out_d, out_n
