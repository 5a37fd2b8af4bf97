"""Benchmark of torch.ops.vectra.rbf_attention on one MI355X.

  python bench.py [--steps K] [--warmup W] [--config serving]

A step is one call of the operator over one batch of the configuration
(default: the serving shape B=1024, H=8, Lq=1, Lk=64, D=32, bf16, per-head
gamma, ragged key-padding masks).  Inputs are resident in HBM before timing.
Each step reads a different one of R input sets whose total exceeds the
256 MB Infinity Cache, so every launch streams its K and V from HBM.

Numerics are gated before anything is timed: the fp32 output of the same
kernel must match the eager chain (the CPU baseline below) within rtol 1e-3 /
atol 1e-4 (bf16/fp16 inputs) or 1e-5 / 1e-6 (fp32), and the operator's
v.dtype output must be exactly that fp32 result rounded once.

A timed step is one launch of the operator's kernel through the C ABI
(vectra_rbf_attention_fwd, the boundary the operator's GPU implementation
calls) with the arguments the operator passes for that input set: output in
v.dtype, automatic kernel selection.  The argument structs are built once,
so the host enqueues a launch in a few microseconds, well inside a launch's
GPU time.  The K timed steps run as trials of up to 100 launches, bracketed
by torch.cuda.synchronize() and by events on the stream the kernels run on;
the first trial is queued behind an untimed lead-in (one HIP-graph replay
of launches), so no trial starts on an idle GPU and the host stays ahead of
the device (see time_trials).  `--launch graph` times HIP-graph replays of
operator calls instead (each replay adds ~13 us of graph start-up on the GPU
before its first kernel).

The CPU baseline is timed after the GPU: the GPU then never idles through
the CPU leg right before its timed region (an idle GPU lowers its clocks).

Prints one JSON line:  queries/s (value), ms_per_step, the roofline of the
kernel (algorithmic bytes / average launch time vs 8 TB/s) and the CPU
baseline (the eager chain, torch fp32, on the host cores).
"""

import argparse
import ctypes
import json
import math
import os
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from vectra_amd.benchmarks import configs  # noqa: E402
from vectra_amd.benchmarks import roofline  # noqa: E402
from vectra_amd.kernels import _native  # noqa: E402
from vectra_amd.kernels import capi  # noqa: E402
import vectra_amd.kernels  # noqa: E402,F401  (registers the operator)

# Input sets rotate over at least this many bytes (> the 256 MB MALL).
ROTATION_BYTES = 320 << 20
MIN_SETS = 5

KERNEL_NAMES = {
    'stream': 'rbf_stream_kernel',
    'generic': 'rbf_generic_kernel',
    'mfma': 'rbf_mfma_kernel',
    'plane': 'rbf_plane_kernel',
    'tile': 'rbf_tile_kernel',
}


def log(*args):
    print(*args, file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split('\n\n')[0])
    p.add_argument('--gpus', type=int, default=1)
    p.add_argument('--steps', type=int, default=2000)
    p.add_argument('--warmup', type=int, default=20)
    p.add_argument('--config', default='serving', choices=sorted(configs.CONFIGS))
    p.add_argument('--dtype', default=None, choices=['bf16', 'fp16', 'fp32'])
    p.add_argument('--launch', default='capi', choices=['capi', 'graph', 'op'],
                   help='timed launches: C-ABI calls (default), HIP-graph replays of operator calls, '
                   'or a host loop of operator calls')
    p.add_argument('--no-graph', action='store_true', help='same as --launch op')
    p.add_argument('--cpu-seconds', type=float, default=12.0,
                   help='CPU-baseline budget (0 skips the CPU leg; numerics then use the '
                   'bit-exact rounding check only)')
    p.add_argument('--sets', type=int, default=0, help='input sets to rotate (0: auto)')
    p.add_argument('--no-read-ceiling', action='store_true',
                   help='skip the plain-read ceiling measurement')
    p.add_argument('--scan', default=None,
                   help='benchmark a distance scan of the engine (vectra_amd/benchmarks/scan_workloads.py: '
                   'flat_shard, flat_shard_q4, exhaustive, pq_shard, pq_candidates, pq_tables, exhaustive_topk, '
                   'single_topk) instead of the operator')
    return p.parse_args()


# The eager chain materialises [.., Nq, Nk, D] in fp32; the CPU sample is
# bounded to this many elements of that tensor (a slice of planes and query
# rows), and its rate converted to subjects per second.
CPU_SAMPLE_ELEMENTS = 1 << 26


def cpu_sample(config, inputs):
    """(sliced inputs, batches, heads, query rows) the CPU leg runs on."""
    per_row = config.n_k * config.head_dim
    rows_cap = max(1, CPU_SAMPLE_ELEMENTS // per_row)
    batches, heads, n_q = config.batch, config.heads, config.n_q
    if batches * heads * n_q > rows_cap:
        batches = max(1, rows_cap // (heads * n_q))
    if batches * heads * n_q > rows_cap:
        heads = max(1, rows_cap // n_q)
    if batches * heads * n_q > rows_cap:
        n_q = rows_cap
    bias = inputs.key_bias[:batches, :heads] if inputs.key_bias is not None else None
    scale = inputs.scale
    if scale.dim() == 4 and scale.shape[1] > 1:
        scale = scale[:, :heads]
    sliced = configs.Inputs(inputs.q[:batches, :heads, :n_q], inputs.k[:batches, :heads],
                            inputs.v[:batches, :heads], scale, bias, None)
    return sliced, batches, heads, n_q


def cpu_reference(config, host_inputs):
    """The eager chain (the oracle's restatement of the reference's
    reference.py:54-58) in torch fp32 on the CPU sample: the numerics gate's
    comparator.  Returns (output, (batches, heads, query rows) of the sample)."""
    from oracle import rbf as oracle  # noqa: E402  (cpu_baseline leg only)

    sample, batches, heads, n_q = cpu_sample(config, host_inputs)
    chunk = 64 if n_q > 1 else None
    return oracle.eager_fp32(*sample.args(), batch_chunk=chunk), (batches, heads, n_q)


def cpu_baseline(config, host_inputs, seconds):
    """Times the eager chain (the oracle's restatement of the reference's
    reference.py:54-58) in torch fp32 on the host cores; returns the record."""
    from oracle import rbf as oracle  # noqa: E402  (cpu_baseline leg only)

    threads = torch.get_num_threads()
    sample, batches, heads, n_q = cpu_sample(config, host_inputs)
    chunk = 64 if n_q > 1 else None
    oracle.eager_fp32(*sample.args(), batch_chunk=chunk)  # warm-up
    reps, start = 0, time.perf_counter()
    while True:
        oracle.eager_fp32(*sample.args(), batch_chunk=chunk)
        reps += 1
        elapsed = time.perf_counter() - start
        if elapsed >= seconds:
            break
    rows_per_s = batches * heads * n_q * reps / elapsed
    qps = rows_per_s / (config.heads * config.n_q)  # subjects per second
    cpu_model = 'unknown'
    try:
        with open('/proc/cpuinfo', encoding='utf-8') as f:
            for line in f:
                if line.startswith('model name'):
                    cpu_model = line.split(':', 1)[1].strip()
                    break
    except OSError:
        pass
    whole = (batches, heads, n_q) == (config.batch, config.heads, config.n_q)
    # The operator's own CPU path (the C++ kernel behind the CPU dispatch key)
    # on the same sample, in the input dtype.
    torch.ops.vectra.rbf_attention(*sample.args())
    op_reps, op_start = 0, time.perf_counter()
    while True:
        torch.ops.vectra.rbf_attention(*sample.args())
        op_reps += 1
        op_elapsed = time.perf_counter() - op_start
        if op_elapsed >= seconds / 2:
            break
    op_qps = batches * heads * n_q * op_reps / op_elapsed / (config.heads * config.n_q)
    record = {
        'value': qps,
        'unit': 'queries/s',
        'cores': threads,
        'kind': 'port',
        'sample': (
            f'eager chain (sub, pow, sum, scale, bias, softmax, matmul) in torch fp32 on '
            + (f'all {config.batch} subjects' if whole else
               f'{batches} subject(s) x {heads} head(s) x {n_q} query row(s), scaled to subjects')
            + f' of input set 0 ({"bf16" if config.dtype == torch.bfloat16 else "input"} values upcast), '
            f'{reps} reps in {elapsed:.1f}s on {threads} threads of {cpu_model}'
        ),
        'op_cpu_path': {'value': op_qps, 'unit': 'queries/s', 'reps': op_reps,
                        'note': 'torch.ops.vectra.rbf_attention on CPU tensors (fused C++ loop), same sample'},
    }
    return record


# The K timed steps run as trials of this many launches (the last trial takes
# any remainder); the reported time per step is the median over trials.
TRIAL_STEPS = 100


# The untimed lead-in queued right before the first timed trial (about
# LEAD_MS of GPU work) and before each later one (about TRIAL_LEAD_MS), each
# one HIP-graph replay of at most LEAD_MAX_STEPS launches.  The later ones
# keep the GPU a few milliseconds behind the host even where the host is slow
# to enqueue (under a profiler's per-launch interception), so the timed
# launches always run back to back.
LEAD_MS = 25.0
TRIAL_LEAD_MS = 12.0
LEAD_MAX_STEPS = 4096


def time_trials(step, steps, warmup, stream, mode='capi'):
    """Milliseconds per step of each trial of the K = `steps` timed launches.

    `step(i)` enqueues launch i on the current stream.  With mode 'capi' or
    'op' a trial is a host loop of launches; with 'graph' it is one HIP-graph
    replay of them (each replay spends ~13 us on the GPU before its first
    kernel, inside the trial).  Each trial is bracketed by events on
    `stream`, the stream the kernels run on, and the K launches by
    synchronisations on both sides.

    The W warm-up launches run first and the device is synchronised.  Then a
    lead-in of about LEAD_MS of untimed launches (at least W) is queued as one
    graph replay and the first trial's start event is recorded straight behind it,
    with no synchronisation between: the host enqueues the timed launches
    while the lead-in runs, so the start event does not fire on an idle GPU,
    the GPU clocks have ramped up, and the host's launch latency stays
    outside the timed region.  Each later trial is queued behind a shorter
    lead-in of the same kind (TRIAL_LEAD_MS).
    """
    sizes = [TRIAL_STEPS] * (steps // TRIAL_STEPS) + ([steps % TRIAL_STEPS] if steps % TRIAL_STEPS else [])
    for i in range(3):  # first launches of each instantiation, outside any capture
        step(i)
    torch.cuda.synchronize()
    probe_start, probe_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    probe_start.record(stream)
    step(0)
    probe_end.record(stream)
    torch.cuda.synchronize()
    per_launch_ms = max(probe_start.elapsed_time(probe_end), 1e-3)
    lead_steps = max(warmup, min(LEAD_MAX_STEPS, math.ceil(LEAD_MS / per_launch_ms)))
    trial_lead_steps = max(1, min(LEAD_MAX_STEPS, math.ceil(TRIAL_LEAD_MS / per_launch_ms)))
    graphs = {}
    for size in (set(sizes) if mode == 'graph' else set()) | {lead_steps, trial_lead_steps}:
        graphs[size] = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graphs[size]):
            for i in range(size):
                step(i)
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    graphs[lead_steps].replay()  # no synchronisation: the trials queue behind it
    events = []
    for trial, size in enumerate(sizes):
        if trial:
            graphs[trial_lead_steps].replay()  # untimed, unsynchronised
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        if mode == 'graph':
            graphs[size].replay()
        else:
            for i in range(size):
                step(i)
        end.record(stream)
        events.append((size, start, end))
    torch.cuda.synchronize()
    return [start.elapsed_time(end) / size for size, start, end in events], lead_steps


def load_profile(name):
    """A committed JSON summary under profiles/, or None."""
    path = os.path.join(ROOT, 'profiles', name)
    if not os.path.exists(path):
        return None
    with open(path, encoding='utf-8') as f:
        return json.load(f)


# ---------------------------------------------------------------- scans

REF_SCAN = os.path.join(ROOT, 'oracle', '_ref', 'libref_scan.so')
SCAN_CPU_ROWS = 65536  # rows (codes, tables) per CPU call and in the numerics sample
SCAN_CPU_TOPK_QUERIES = 16  # queries per CPU call of a top-k workload, and in its numerics sample


def _scan_cpu(w, inputs):
    """(callable computing the workload's outputs for a bounded sample of set
    0 on the CPU, the sample's output count, kind).  The reference engine's own
    code (oracle/_ref, built from its sources) where that library is present,
    else the numpy restatement (oracle/scan.py)."""
    import numpy as np  # noqa: E402

    from oracle import scan as oracle  # noqa: E402  (cpu_baseline leg only)

    lib = ctypes.CDLL(REF_SCAN) if os.path.exists(REF_SCAN) else None
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    if w.kind == 'rows':
        rows = inputs['rows'][:SCAN_CPU_ROWS].cpu().numpy()
        queries = inputs['queries'].cpu().numpy()
        n = rows.shape[0]

        def run():
            out = np.empty((queries.shape[0], n), np.float32)
            for q in range(queries.shape[0]):
                if lib is not None:
                    lib.ref_scan_rows(0, ptr(queries[q]), ptr(rows), ctypes.c_int64(n), ctypes.c_int64(w.dim),
                                      w.dim, ptr(out[q]))
                else:
                    out[q] = oracle.l2_squared(queries[q], rows)
            return out
        return run, queries.shape[0] * n, ('reference' if lib is not None else 'port')
    if w.kind == 'topk':
        # ExhaustiveSearch per query: the distance to every row, then the k
        # nearest under the reference's CloserFirst (oracle/_ref's shim over
        # its header), or the numpy restatement.
        rows = np.ascontiguousarray(inputs['rows'].cpu().numpy())
        queries = np.ascontiguousarray(inputs['queries'][:SCAN_CPU_TOPK_QUERIES].cpu().numpy())
        n = rows.shape[0]
        nodes = np.arange(n, dtype=np.uint32)
        if lib is not None:
            lib.ref_nearest.restype = ctypes.c_int64

        def run():
            if lib is None:
                return oracle.nearest(queries, rows, w.k)
            out_d = np.full((queries.shape[0], w.k), np.inf, np.float32)
            out_n = np.full((queries.shape[0], w.k), oracle.NO_NODE, np.uint32)
            dist = np.empty(n, np.float32)
            for q in range(queries.shape[0]):
                lib.ref_scan_rows(0, ptr(queries[q]), ptr(rows), ctypes.c_int64(n), ctypes.c_int64(w.dim), w.dim,
                                  ptr(dist))
                lib.ref_nearest(ptr(dist), ptr(nodes), ctypes.c_int64(n), ctypes.c_int64(w.k), ptr(out_d[q]),
                                ptr(out_n[q]))
            return out_d, out_n
        return run, queries.shape[0] * n, ('reference' if lib is not None else 'port')
    if w.kind == 'adc':
        if 'ids' in inputs:  # the codes the first candidates name, in candidate order
            codes = np.ascontiguousarray(inputs['codes'][inputs['ids'][:SCAN_CPU_ROWS].long()].cpu().numpy())
        else:
            codes = np.ascontiguousarray(inputs['codes'][:SCAN_CPU_ROWS].cpu().numpy())
        tables = inputs['tables'].cpu().numpy()
        n = codes.shape[0]

        def run():
            out = np.empty((tables.shape[0], n), np.float32)
            for q in range(tables.shape[0]):
                if lib is not None:
                    lib.ref_pq_adc_rows(ptr(tables[q]), ptr(codes), ctypes.c_int64(n), ctypes.c_int64(w.subspaces),
                                        w.subspaces, ptr(out[q]))
                else:
                    out[q] = oracle.pq_adc(tables[q], codes)
            return out
        return run, tables.shape[0] * n, ('reference' if lib is not None else 'port')
    queries = inputs['queries'][:64].cpu().numpy()
    books = np.ascontiguousarray(inputs['codebooks'].cpu().numpy())

    def run():
        out = np.empty((queries.shape[0], w.subspaces * 256), np.float32)
        for q in range(queries.shape[0]):
            if lib is not None:
                assert lib.ref_pq_distance_table(w.dim, w.subspaces, ptr(books), ptr(queries[q]), ptr(out[q])) == 0
            else:
                out[q] = oracle.pq_distance_table(queries[q], books, w.subspaces)
        return out
    return run, queries.shape[0] * w.subspaces * 256, ('reference' if lib is not None else 'port')


def scan_main(args):
    """`--scan NAME`: one JSON line for a distance scan of the engine."""
    from vectra_amd.benchmarks import scan_workloads  # noqa: E402

    if args.scan not in scan_workloads.WORKLOADS:
        raise SystemExit(f'unknown scan workload {args.scan!r}; one of {sorted(scan_workloads.WORKLOADS)}')
    w = scan_workloads.WORKLOADS[args.scan]
    sets = scan_workloads.make_sets(w)
    out = scan_workloads.make_output(w)
    n_sets = len(sets)
    log(f'scan {w.name}: {w.set_bytes() / 1e6:.1f} MB per input set, rotating {n_sets} sets')
    torch.cuda.synchronize()

    # ---- Numerics gate: bit for bit against the CPU on a sample of set 0. ----
    cpu_run, cpu_outputs, cpu_kind = (None, 0, None)
    if args.cpu_seconds > 0:
        import numpy as np  # noqa: E402

        cpu_run, cpu_outputs, cpu_kind = _scan_cpu(w, sets[0])
        got = scan_workloads.launch(w, sets[0], out)
        torch.cuda.synchronize()
        want = cpu_run()
        if w.kind == 'topk':  # (distances, nodes) of the sampled queries
            got = tuple(t[:want[0].shape[0]].cpu().numpy() for t in got)
            same = (np.array_equal(got[0].view(np.uint32), want[0].view(np.uint32))
                    and np.array_equal(got[1], want[1]))
            size = want[0].size
        else:
            got = got[:want.shape[0], :want.shape[1]].cpu().numpy()
            same = np.array_equal(got.view(np.uint32), want.view(np.uint32))
            size = want.size
        if not same:
            raise SystemExit('numerics gate: the scan differs from the CPU reference')
        log(f'numerics gate passed: {size} outputs bit-identical to the {cpu_kind} CPU code')

    stream = torch.cuda.current_stream()

    def step(i):
        scan_workloads.launch(w, sets[i % n_sets], out)

    trial_ms, lead_steps = time_trials(step, args.steps, args.warmup, stream, mode='capi')
    ms = statistics.median(trial_ms)
    seconds = ms / 1e3

    cpu = None
    if cpu_run is not None:
        cpu_run()
        reps, start = 0, time.perf_counter()
        while True:
            cpu_run()
            reps += 1
            elapsed = time.perf_counter() - start
            if elapsed >= args.cpu_seconds:
                break
        what = ("the reference engine's own functions, compiled from its sources" if cpu_kind == 'reference'
                else 'the numpy restatement of them')
        cpu = {'value': cpu_outputs * reps / elapsed, 'unit': w.unit, 'cores': 1, 'kind': cpu_kind,
               'sample': f'{cpu_outputs} outputs of set 0 per call ({what}), one thread, '
                         f'{reps} calls in {elapsed:.1f}s'}
        log(f'cpu baseline: {cpu["value"]:.4g} {w.unit} ({cpu_kind})')

    nbytes = w.algorithmic_bytes()
    achieved = nbytes / seconds / 1e9
    if w.kind == 'topk':
        # Rows re-read by every query from the L2 caches: bound by the vector
        # ALU (three fp32 operations per dimension of each distance).
        terms = w.queries * w.count * w.dim
        line_roof = {'bound': 'valu', 'achieved': 3 * terms / seconds / 1e12,
                     'peak': scan_workloads.VALU_LANE_OPS_PER_S / 1e12, 'unit': 'T lane-ops/s',
                     'kernel': scan_workloads.KERNEL_NAMES[w.kind], 'traffic': None, 'algorithmic_bytes': nbytes,
                     'hbm_GB/s': achieved}
    else:
        line_roof = {'bound': 'hbm', 'achieved': achieved, 'peak': roofline.MI355X.hbm_bytes_per_s / 1e9,
                     'unit': 'GB/s', 'kernel': scan_workloads.KERNEL_NAMES[w.kind], 'traffic': None,
                     'algorithmic_bytes': nbytes}
    line_roof['frac'] = line_roof['achieved'] / line_roof['peak']
    measured = load_profile(f'traffic_scan_{w.name}.json')
    if measured is not None and measured.get('kernel') == line_roof['kernel']:
        line_roof['traffic'] = measured['traffic_bytes']
        line_roof['traffic_source'] = f'profiles/traffic_scan_{w.name}.json'
    if not args.no_read_ceiling and nbytes >= (1 << 20) and w.kind != 'topk':
        from vectra_amd.benchmarks import read_ceiling  # noqa: E402

        ceiling = read_ceiling.measure(nbytes)
        line_roof['read_ceiling'] = {'us': ceiling['us'], 'GB/s': ceiling['GB/s'],
                                     'frac_of_peak': ceiling['GB/s'] / line_roof['peak'],
                                     'kernel_over_ceiling': achieved / ceiling['GB/s']}
        log(f'read ceiling: {ceiling["us"]:.2f} us, {ceiling["GB/s"]:.0f} GB/s')
    result = {
        'metric': f'engine distance scan {w.name}: {w.unit} + % of HBM peak',
        'value': w.outputs_per_launch() / seconds,
        'unit': w.unit,
        'n_gpus': 1, 'steps': args.steps, 'warmup': args.warmup, 'ms_per_step': ms,
        'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None, 'dtype': 'f32', 'data': 'synthetic',
        'config': {'workload': f'{w.name}: {w.kind}, queries={w.queries} count={w.count} dim={w.dim} '
                               f'subspaces={w.subspaces}' + (f' k={w.k}' if w.k else ''),
                   'input_sets': n_sets, 'trials': len(trial_ms), 'lead_in_launches': lead_steps},
        'roofline': line_roof,
        'cpu_baseline': cpu,
        'native_libraries': [os.path.relpath(p, ROOT) for p in _native.loaded_libraries()],
    }
    print(json.dumps(result), flush=True)


def main():
    args = parse_args()
    if args.gpus != 1:
        print(
            f'bench.py measures one GPU; --gpus {args.gpus} is not supported '
            '(the operator shards over batches with no exchange between GPUs).',
            file=sys.stderr,
        )
        sys.exit(2)
    if not torch.cuda.is_available():
        print('bench.py needs a GPU', file=sys.stderr)
        sys.exit(1)
    if args.scan:
        scan_main(args)
        return

    config = configs.CONFIGS[args.config]
    if args.dtype:
        config = config.with_dtype({'bf16': torch.bfloat16, 'fp16': torch.float16,
                                    'fp32': torch.float32}[args.dtype])
    shape = config.shape()
    host0 = configs.make_inputs(config, seed=0)
    per_set = host0.nbytes()
    n_sets = args.sets or max(MIN_SETS, math.ceil(ROTATION_BYTES / per_set))
    log(f'config {config.name}: {per_set / 1e6:.1f} MB per input set, rotating {n_sets} sets')
    sets = [host0.to('cuda')] + [
        configs.make_inputs(config, seed=s).to('cuda') for s in range(1, n_sets)
    ]
    torch.cuda.synchronize()

    # ---- Numerics gate (before any timing). ----
    fp32 = capi.forward(*sets[0].args(), out_dtype=torch.float32)
    out = torch.ops.vectra.rbf_attention(*sets[0].args())
    torch.cuda.synchronize()
    if not torch.equal(out, fp32.to(out.dtype)):
        raise SystemExit('numerics gate: operator output is not the rounded fp32 result')
    if args.cpu_seconds > 0:
        want, (nb, nh, nr) = cpu_reference(config, host0)
        tol = (1e-5, 1e-6) if config.dtype == torch.float32 else (1e-3, 1e-4)
        torch.testing.assert_close(fp32[:nb, :nh, :nr].cpu(), want, rtol=tol[0], atol=tol[1],
                                   equal_nan=True)
        log('numerics gate passed against the eager chain')

    # The operator's own launch arguments for each input set: output in
    # v.dtype (a buffer per set, as the operator allocates one per call),
    # automatic kernel selection.
    launches = []
    for inputs in sets:
        dst = torch.empty((*inputs.q.shape[:-1], inputs.v.shape[-1]), dtype=inputs.v.dtype, device='cuda')
        scale4, bias4 = capi.broadcast_operands(inputs.q, inputs.k, inputs.scale, inputs.key_bias)
        launches.append((capi.make_args(inputs.q, inputs.k, inputs.v, dst, scale4, bias4), dst, scale4, bias4))
    variant = capi.VARIANT_NAMES[capi.select_variant(launches[0][0])]
    stream = torch.cuda.current_stream()
    mode = 'op' if args.no_graph else args.launch
    if mode == 'capi':
        fwd = _native.hip_library().vectra_rbf_attention_fwd
        arg_refs = [ctypes.byref(entry[0]) for entry in launches]

        def step(i):
            # The current stream: `stream`, or a capture stream inside a graph capture.
            status = fwd(arg_refs[i % n_sets], ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            if status:
                raise SystemExit(f'launch failed: {capi.status_string(status)}')
    else:
        def step(i):
            return torch.ops.vectra.rbf_attention(*sets[i % n_sets].args())

    trial_ms, lead_steps = time_trials(step, args.steps, args.warmup, stream, mode=mode)
    # The timed launches wrote what the operator returns for their sets.
    for inputs, (_, dst, _, _) in zip(sets, launches):
        if mode == 'capi' and not torch.equal(dst, torch.ops.vectra.rbf_attention(*inputs.args())):
            raise SystemExit('the timed launches wrote other values than the operator returns')
    ms = statistics.median(trial_ms)

    # ---- CPU baseline leg, after the GPU timing. ----
    cpu = None
    if args.cpu_seconds > 0:
        cpu = cpu_baseline(config, host0, args.cpu_seconds)
        log(f'cpu baseline: {cpu["value"]:.4g} queries/s on {cpu["cores"]} threads')
    seconds = ms / 1e3
    fused = roofline.fused_bytes(shape)
    # Bound of the workload: HBM unless its intensity is above the ridge.
    mfma_bound = roofline.analyze(shape)['fused_is_memory_bound'] is False
    if mfma_bound:
        achieved = roofline.matrix_flops(shape) / seconds / 1e12
        line_roof = {'bound': 'mfma', 'achieved': achieved,
                     'peak': roofline.MI355X.bf16_mfma_flops / 1e12, 'unit': 'TFLOP/s'}
    else:
        achieved = fused / seconds / 1e9
        line_roof = {'bound': 'hbm', 'achieved': achieved,
                     'peak': roofline.MI355X.hbm_bytes_per_s / 1e9, 'unit': 'GB/s'}
    line_roof['frac'] = line_roof['achieved'] / line_roof['peak']
    line_roof['kernel'] = KERNEL_NAMES.get(variant, variant)
    if variant == 'plane' and config.dtype == torch.float32:
        line_roof['kernel'] = 'rbf_plane32_kernel'  # the fp32 instantiation
    line_roof['traffic'] = None
    # HBM bytes per launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    # runs of this workload (profiles/traffic_<config>.json, made by
    # vectra_amd.benchmarks.rocprof_summary), if they measured this kernel.
    measured = load_profile(f'traffic_{config.name}.json')
    if measured is not None and measured.get('kernel') == line_roof['kernel']:
        line_roof['traffic'] = measured['traffic_bytes']
        line_roof['traffic_source'] = f'profiles/traffic_{config.name}.json'
    # Measured bytes of the operator over those of the eager chain at the same
    # shape (profiles/bytes_ratio_<config>.json, rocprof_summary ratio).
    ratio = load_profile(f'bytes_ratio_{config.name}.json')
    if ratio is not None:
        line_roof['bytes_ratio_vs_eager'] = ratio['bytes_ratio']
        line_roof['bytes_ratio_source'] = f'profiles/bytes_ratio_{config.name}.json'
    # A plain streaming read of the same number of bytes, timed the same way:
    # the practical ceiling for an HBM-bound kernel.
    if not mfma_bound and not args.no_read_ceiling:
        from vectra_amd.benchmarks import read_ceiling  # noqa: E402

        ceiling = read_ceiling.measure(fused)
        line_roof['read_ceiling'] = {'us': ceiling['us'], 'GB/s': ceiling['GB/s'],
                                     'frac_of_peak': ceiling['GB/s'] / line_roof['peak'],
                                     'kernel_over_ceiling': achieved / ceiling['GB/s']}
        log(f'read ceiling: {ceiling["us"]:.2f} us, {ceiling["GB/s"]:.0f} GB/s')
        # Where the output is a large share of the bytes (the plane kernels
        # write a quarter), the same reads and writes streamed together.
        out_bytes = shape.planes * shape.n_q * shape.value_dim * shape.element_bytes
        if out_bytes * 10 >= fused:
            mixed = read_ceiling.measure_read_write(fused - out_bytes, out_bytes)
            line_roof['read_write_ceiling'] = {'us': mixed['us'], 'GB/s': mixed['GB/s'],
                                               'frac_of_peak': mixed['GB/s'] / line_roof['peak'],
                                               'kernel_over_ceiling': achieved / mixed['GB/s']}
            log(f'read + write ceiling: {mixed["us"]:.2f} us, {mixed["GB/s"]:.0f} GB/s')
    line_roof['algorithmic_bytes'] = fused

    result = {
        'metric': 'rbf_attention queries/s + % of HBM peak at B=1024 serving shape, bf16',
        'value': config.batch / seconds,
        'unit': 'queries/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': ms,
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': {torch.bfloat16: 'bf16', torch.float16: 'fp16', torch.float32: 'fp32'}[config.dtype],
        'data': 'synthetic',
        'config': {
            'workload': f'{config.name}: B={config.batch} H={config.heads} Lq={config.n_q} '
                        f'Lk={config.n_k} D={config.head_dim}',
            'batch': config.batch, 'heads': config.heads, 'n_q': config.n_q, 'n_k': config.n_k,
            'head_dim': config.head_dim, 'input_sets': n_sets,
            'timing': ('median over trials of %d launches, each %s, queued behind a graph replay of untimed '
                       'launches (%d before the first trial, ~12 ms before each later one)' %
                       (min(TRIAL_STEPS, args.steps),
                        {'capi': 'a host loop of C-ABI launches with the operator\'s arguments',
                         'graph': 'one HIP-graph replay of operator calls',
                         'op': 'a host loop of operator calls'}[mode], lead_steps)),
            'trials': len(trial_ms),
            'variant': variant,
        },
        'roofline': line_roof,
        'cpu_baseline': cpu,
        'native_libraries': [os.path.relpath(p, ROOT) for p in _native.loaded_libraries()],
    }
    print(json.dumps(result), flush=True)


if __name__ == '__main__':
    main()
