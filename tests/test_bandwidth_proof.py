"""The bandwidth-proof harness on the CPU: the SLO gate and the aggregation of
rocprofv3 output over the measured region.

Restates the reference's benchmark/harness_test.py:208-241
(test_nsight_csv_is_aggregated_over_the_region, test_bandwidth_gate) for
rocprofv3's kernel-stats and counter-collection CSVs.
"""

import csv

import pytest
import torch

from vectra_amd.benchmarks import bandwidth_proof
from vectra_amd.benchmarks import configs
from vectra_amd.benchmarks import roofline

BLIT = '__amd_rocclr_copyBuffer'


def _write(path, header, rows):
    with open(path, 'w', encoding='utf-8', newline='') as f:
        w = csv.writer(f, quoting=csv.QUOTE_ALL)
        w.writerow(header)
        w.writerows(rows)
    return str(path)


def _trace(path, dispatches):
    """A --kernel-trace CSV of (name, duration_ns) dispatches in launch order."""
    header = ['Kind', 'Agent_Id', 'Queue_Id', 'Stream_Id', 'Thread_Id', 'Dispatch_Id', 'Kernel_Id', 'Kernel_Name',
              'Correlation_Id', 'Start_Timestamp', 'End_Timestamp']
    rows, t = [], 1_000
    for i, (name, ns) in enumerate(dispatches, 1):
        rows.append(['KERNEL_DISPATCH', 1, 1, 0, 1, i, 1, name, i, t, t + ns])
        t += ns + 500
    return _write(path, header, rows)


def _counters(path, counter, dispatches):
    header = ['Correlation_Id', 'Dispatch_Id', 'Agent_Id', 'Queue_Id', 'Process_Id', 'Thread_Id',
              'Grid_Size', 'Kernel_Id', 'Kernel_Name', 'Workgroup_Size', 'LDS_Block_Size',
              'Scratch_Size', 'VGPR_Count', 'Accum_VGPR_Count', 'SGPR_Count', 'Counter_Name',
              'Counter_Value', 'Start_Timestamp', 'End_Timestamp']
    rows = [[i, i, 1, 1, 1, 1, 1, 1, name, 64, 0, 0, 0, 0, 0, counter, value, 0, 0]
            for i, (name, value) in enumerate(dispatches, 1)]
    return _write(path, header, rows)


def test_gate_restated_from_the_reference():
    good = {
        64: {
            'eager': {'dram_bytes': 300e6, 'dram_throughput_pct': 35.0},
            'fused': {'dram_bytes': 5e6, 'dram_throughput_pct': 20.0},
        },
        1024: {
            'eager': {'dram_bytes': 4.8e9, 'dram_throughput_pct': 41.0},
            'fused': {'dram_bytes': 70e6, 'dram_throughput_pct': 71.0},
        },
    }
    assert not bandwidth_proof.evaluate(good)
    slow = {64: good[64], 1024: dict(good[1024], fused={'dram_bytes': 70e6, 'dram_throughput_pct': 50.0})}
    failures = bandwidth_proof.evaluate(slow)
    assert len(failures) == 1 and '50.0% < 65%' in failures[0]


def test_gate_fails_on_bytes_at_any_batch_and_on_a_missing_utilisation_batch():
    heavy = {64: {'eager': {'dram_bytes': 10e6}, 'fused': {'dram_bytes': 6.5e6}}}
    failures = bandwidth_proof.evaluate(heavy)
    assert failures == ['batch 64: fused/eager bytes 0.650 > 0.6', 'batch 1024 was not profiled']
    # The ratio gate is inclusive: exactly 0.60 passes.
    edge = {1024: {'eager': {'dram_bytes': 10e6, 'dram_throughput_pct': 30.0},
                   'fused': {'dram_bytes': 6e6, 'dram_throughput_pct': 65.0}}}
    assert not bandwidth_proof.evaluate(edge)


def test_region_is_aggregated_over_the_measured_calls_but_not_the_runtime_blits(tmp_path):
    # A warm-up call and two measured calls of a two-kernel region, plus input
    # copies the runtime made; the warm-up call is slower and reads more.
    trace = _trace(tmp_path / 'trace.csv', [
        (BLIT, 9_999), ('kernel_a', 90_000), ('kernel_b', 50_000), (BLIT, 9_999),
        ('kernel_a', 30_000), ('kernel_b', 10_000), ('kernel_a', 30_000), ('kernel_b', 10_000),
    ])
    kib = 1024.0
    fetch = _counters(tmp_path / 'fetch.csv', 'FETCH_SIZE', [
        (BLIT, 512 * kib), ('kernel_a', 99_999 * kib), ('kernel_b', 99_999 * kib),
        ('kernel_a', 12_288 * kib), ('kernel_b', 4_096 * kib),
        ('kernel_a', 12_288 * kib), ('kernel_b', 4_096 * kib),
    ])
    write = _counters(tmp_path / 'write.csv', 'WRITE_SIZE', [
        (BLIT, 777 * kib), ('kernel_a', 5.0), ('kernel_b', 5.0),
        ('kernel_a', 0.0), ('kernel_b', 1_024 * kib),
        ('kernel_a', 0.0), ('kernel_b', 1_024 * kib),
    ])
    got = bandwidth_proof.region_counters(trace, fetch, write, calls=3, warmup=1, batch=8,
                                          scales={'fetch_scale': 2.0, 'write_scale': 1.0})
    read = 2.0 * (12_288 + 4_096) * kib * 1024
    written = 1_024 * kib * 1024
    assert got['dram_read_bytes'] == read
    assert got['dram_write_bytes'] == written
    assert got['dram_bytes'] == read + written
    assert got['dram_bytes_per_query'] == (read + written) / 8
    assert got['kernel_ns'] == 40_000
    # A dispatch count that does not divide into the calls is an error.
    with pytest.raises(ValueError):
        bandwidth_proof.measured_dispatches([1.0] * 5, calls=2, warmup=1)
    # Bytes over summed time: the time-weighted mean of the kernels' rates.
    want_pct = 100 * (read + written) / 40e-6 / roofline.MI355X.hbm_bytes_per_s
    assert got['dram_throughput_pct'] == pytest.approx(want_pct)


def test_time_weighted_throughput_equals_bytes_over_time():
    """The reference averages per-kernel throughput weighted by kernel time
    (collect_nsight_metrics.py:95-113); bytes over summed time is the same number."""
    kernels = [(30_000, 70.0), (10_000, 40.0)]  # (ns, % of peak)
    peak = roofline.MI355X.hbm_bytes_per_s
    total_bytes = sum(ns * 1e-9 * pct / 100 * peak for ns, pct in kernels)
    total_ns = sum(ns for ns, _ in kernels)
    assert 100 * total_bytes / (total_ns * 1e-9) / peak == pytest.approx(62.5)


def test_bandwidth_workload_is_the_reference_harness_shape():
    c = configs.BANDWIDTH
    inputs = configs.make_inputs(c, batch=2)
    assert inputs.q.shape == (2, 4, 65, 32) and inputs.q.dtype.itemsize == 2
    assert inputs.scale.shape == (1, 4, 1, 1)
    assert (inputs.scale == 1.0 / 64).all()
    padded = inputs.key_bias[0, 0, 0]
    assert padded[:57].eq(0).all() and padded[57:].eq(float('-inf')).all()
    # The harness's five rotating input sets do not fit the Infinity Cache.
    assert 5 * roofline.fused_bytes(c.shape()) > roofline.MI355X.infinity_cache_bytes
    assert 5 * roofline.fused_bytes(configs.SERVING.shape()) > roofline.MI355X.infinity_cache_bytes


def test_read_write_stream_checks_its_byte_mix():
    """The read + write ceiling's argument checks, before any launch."""
    from vectra_amd.benchmarks import read_ceiling
    sink = torch.zeros(256, dtype=torch.int32)
    for read_bytes, write_bytes in ((160, 16), (16, 32), (64, 8), (40, 24)):
        with pytest.raises(ValueError):
            read_ceiling.read_write_once(torch.zeros(read_bytes, dtype=torch.uint8),
                                         torch.zeros(write_bytes, dtype=torch.uint8), sink, 1, None)
