"""Workloads of the distance-scan benchmark (`python bench.py --scan NAME`).

Sizes follow the reference engine's index configuration
(engine/configs/hnsw_params.textproto: 128-dimensional float vectors,
16-byte PQ codes, up to 4,000,000 vectors per shard, exhaustive scans up to
2,048 rows, re-rank depth 128):

============  ===============================================================
flat_shard    ShardIndex::ExhaustiveSearch (shard_index.cc:236-264) over a
              whole shard: L2SquaredDistance of one query to 4,000,000 rows
flat_shard_q4 the same for four queries at once (each row read once)
exhaustive    the exhaustive scan the reference actually runs: one query,
              2,048 rows (exhaustive_scan_threshold)
pq_shard      PqAdcDistance of one query table over 4,000,000 16-byte codes
              (the ADC pass of a search over a whole shard)
pq_candidates the same over 500,000 candidate ids drawn at random from the
              shard's 4,000,000 codes (a candidate list's ADC pass: random
              16-byte reads)
pq_tables     ComputeDistanceTable for 1,024 queries (dimension 128,
              16 sub-spaces)
exhaustive_   ShardIndex::ExhaustiveSearch for 1,024 queries at once, each
topk          over the same 2,048 rows (exhaustive_scan_threshold), k = 10:
              the k nearest in CloserFirst order
single_topk   the same for one query (the engine's per-request case)
============  ===============================================================

The top-k workloads read the same rows for every query (the L2 caches
serve them after the first), so their bound is the vector ALU rather than
HBM: three fp32 operations (subtract, multiply, add) per dimension of each
distance, against the 39.3 T lane operations per second of MI355X's vector
units (256 CUs x 4 SIMDs x 16 lanes x 2.4 GHz, unpacked fp32).

Algorithmic bytes per launch count every input byte once and every output
byte once: rows (or codes, or codebooks), queries (or tables) and the
distances written.  Inputs rotate over more than the 256 MB Infinity Cache
where one set is smaller than that.
"""

import dataclasses

import torch

from vectra_amd.index import scan

ROTATION_BYTES = 320 << 20
PQ_CENTROIDS = 256


@dataclasses.dataclass(frozen=True)
class Workload:
    name: str
    kind: str            # 'rows', 'adc' or 'tables'
    queries: int
    count: int           # rows, codes, or (for tables) unused
    dim: int = 128
    subspaces: int = 16
    unit: str = 'distances/s'
    k: int = 0           # nearest rows kept per query ('topk')
    ids: int = 0         # candidate ids drawn from the codes ('adc'; 0: every code)

    def algorithmic_bytes(self) -> int:
        if self.kind == 'rows':
            return self.count * self.dim * 4 + self.queries * self.dim * 4 + self.queries * self.count * 4
        if self.kind == 'adc':
            n = self.ids or self.count  # candidates: one code, (an id) and a distance each
            return (n * self.subspaces + (4 * n if self.ids else 0)
                    + self.queries * self.subspaces * PQ_CENTROIDS * 4 + self.queries * n * 4)
        if self.kind == 'topk':  # rows and queries in, k (distance, node) pairs out
            return self.count * self.dim * 4 + self.queries * self.dim * 4 + self.queries * self.k * 8
        # tables: queries + codebooks in, tables out
        return (self.queries * self.dim * 4 + PQ_CENTROIDS * self.dim * 4
                + self.queries * self.subspaces * PQ_CENTROIDS * 4)

    def outputs_per_launch(self) -> int:
        if self.kind == 'tables':
            return self.queries * self.subspaces * PQ_CENTROIDS
        if self.kind == 'adc' and self.ids:
            return self.queries * self.ids
        return self.queries * self.count

    def set_bytes(self) -> int:
        if self.kind in ('rows', 'topk'):
            return self.count * self.dim * 4
        if self.kind == 'adc':
            return self.count * self.subspaces
        return PQ_CENTROIDS * self.dim * 4 + self.queries * self.dim * 4


WORKLOADS = {w.name: w for w in (
    Workload('flat_shard', 'rows', 1, 4_000_000),
    Workload('flat_shard_q4', 'rows', 4, 4_000_000),
    Workload('exhaustive', 'rows', 1, 2048),
    Workload('pq_shard', 'adc', 1, 4_000_000),
    Workload('pq_candidates', 'adc', 1, 4_000_000, ids=500_000),
    Workload('pq_tables', 'tables', 1024, 0, unit='table entries/s'),
    Workload('exhaustive_topk', 'topk', 1024, 2048, k=10),
    Workload('single_topk', 'topk', 1, 2048, k=10),
)}

# The kernel each workload runs (pq_shard's 16-byte codes take the 16-byte-load ADC kernel).
KERNEL_NAMES = {'rows': 'scan_rows_kernel', 'adc': 'pq_adc_vec_kernel', 'tables': 'pq_table_sub_kernel',
                'topk': 'scan_top_k_kernel'}
VALU_LANE_OPS_PER_S = 256 * 4 * 16 * 2.4e9  # MI355X vector units, unpacked fp32


def sets_needed(w: Workload) -> int:
    return max(1, min(512, -(-ROTATION_BYTES // max(w.set_bytes(), 1))))


def make_sets(w: Workload, seed: int = 0, device='cuda') -> list[dict]:
    """Input sets on the GPU (float32 normal vectors, uniform codes)."""
    gen = torch.Generator(device='cpu').manual_seed(seed)
    n_sets = sets_needed(w)
    sets = []
    if w.kind in ('rows', 'topk'):
        # One host draw, varied per set on the device (scaled), to keep set-up fast.
        base = torch.randn(w.count, w.dim, generator=gen).to(device)
        for i in range(n_sets):
            sets.append({'queries': torch.randn(w.queries, w.dim, generator=gen).to(device),
                         'rows': base if i == 0 else base * (1.0 + i / 64)})
        if w.kind == 'topk':
            # The split form's workspace (zeroed once; each call leaves its
            # counters zero), made before the timed region.
            need = scan.workspace_bytes(sets[0]['queries'], sets[0]['rows'], w.k)
            workspace = torch.zeros(max(need, 1), dtype=torch.uint8, device=device)
            for s in sets:
                s['workspace'] = workspace
    elif w.kind == 'adc':
        base = torch.randint(0, 256, (w.count, w.subspaces), generator=gen, dtype=torch.uint8).to(device)
        for i in range(n_sets):
            sets.append({'tables': (torch.rand(w.queries, w.subspaces * PQ_CENTROIDS, generator=gen) * 8).to(device),
                         'codes': base if i == 0 else base ^ i})
            if w.ids:
                sets[-1]['ids'] = torch.randint(0, w.count, (w.ids,), generator=gen, dtype=torch.int32).to(device)
    else:
        for _ in range(n_sets):
            sets.append({'queries': torch.randn(w.queries, w.dim, generator=gen).to(device),
                         'codebooks': torch.randn(w.subspaces, PQ_CENTROIDS, w.dim // w.subspaces,
                                                  generator=gen).to(device)})
    return sets


def make_output(w: Workload, device='cuda'):
    if w.kind == 'topk':
        return (torch.empty(w.queries, w.k, device=device), torch.empty(w.queries, w.k, dtype=torch.uint32,
                                                                        device=device))
    if w.kind == 'tables':
        return torch.empty(w.queries, w.subspaces * PQ_CENTROIDS, device=device)
    return torch.empty(w.queries, w.ids or w.count, device=device)


def launch(w: Workload, inputs: dict, out: torch.Tensor) -> torch.Tensor:
    """One launch of the workload's kernel on the current stream."""
    if w.kind == 'rows':
        return scan.l2_squared_distances(inputs['queries'], inputs['rows'], out=out)
    if w.kind == 'topk':
        return scan.nearest(inputs['queries'], inputs['rows'], w.k, out=out, workspace=inputs.get('workspace'))
    if w.kind == 'adc':
        return scan.pq_adc_distances(inputs['tables'], inputs['codes'], ids=inputs.get('ids'), out=out)
    return scan.pq_distance_tables(inputs['queries'], inputs['codebooks'], w.subspaces, out=out)
