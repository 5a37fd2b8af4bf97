"""The MFMA-utilisation harness's arithmetic on synthetic rocprofv3 CSVs (CPU)."""

import csv

import pytest

from vectra_amd.benchmarks import configs
from vectra_amd.benchmarks import mfma_utilization as mu
from vectra_amd.benchmarks import roofline

KERNEL = 'void vectra::rbf_tile_kernel<__bf16, __bf16, 64, 64, 4, 2>(vectra::Problem, int)'


def _write(path, header, rows):
    with open(path, 'w', newline='', encoding='utf-8') as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def _profiles(tmp_path, grbm_factor):
    """A trace of three dispatches of 1.0-1.2 ms and a counter run whose
    dispatches last 1.25 ms at 2.0 GHz, the matrix cores busy 40% of it."""
    trace = tmp_path / 'trace.csv'
    _write(trace, ['Kernel_Name', 'Start_Timestamp', 'End_Timestamp'],
           [[KERNEL, 0, 1_100_000], [KERNEL, 2_000_000, 3_000_000], [KERNEL, 4_000_000, 5_200_000],
            ['other_kernel', 0, 5]])
    ns = 1_250_000
    active = 2.0 * ns
    simds = roofline.MI355X.compute_units * mu.SIMDS_PER_CU
    busy = 0.40 * simds * active
    counters = {'SQ_VALU_MFMA_BUSY_CYCLES': busy, 'SQ_INSTS_MFMA': busy / 16, 'SQ_INSTS_VALU': busy / 16 * 5,
                'SQ_WAVE_CYCLES': 1.0, 'SQ_BUSY_CYCLES': 1.0, 'GRBM_GUI_ACTIVE': active * grbm_factor}
    rows = []
    for dispatch in (7, 9):
        for name, value in counters.items():
            rows.append([dispatch, KERNEL, name, value, 10_000_000 * dispatch, 10_000_000 * dispatch + ns])
    pmc = tmp_path / 'pmc.csv'
    _write(pmc, ['Dispatch_Id', 'Kernel_Name', 'Counter_Name', 'Counter_Value', 'Start_Timestamp',
                 'End_Timestamp'], rows)
    return str(trace), str(pmc)


@pytest.mark.parametrize('grbm_factor', [1, roofline.MI355X.xcds])
def test_utilisation_from_counters(tmp_path, grbm_factor):
    trace, pmc = _profiles(tmp_path, grbm_factor)
    flops = roofline.matrix_flops(configs.LONG_KEY.shape())
    r = mu.summarize(trace, pmc, 'rbf_tile_kernel', flops)
    assert r['dispatches_traced'] == 3 and r['dispatches_counted'] == 2
    assert r['median_ns'] == 1_100_000
    assert r['grbm_summed_over_xcds'] == (grbm_factor > 1)
    assert r['clock_ghz'] == pytest.approx(2.0)
    assert r['mfma_busy_pct'] == pytest.approx(40.0)
    assert r['busy_cycles_per_mfma'] == pytest.approx(16.0)
    assert r['valu_per_mfma'] == pytest.approx(4.0)
    assert flops == 4 * 16 * 16 * 4096 * 4096 * 64
    assert r['flops_pct'] == pytest.approx(100 * flops / 1.1e-3 / 2.5e15)
    assert r['issued_flops'] == pytest.approx(r['counters_per_dispatch']['SQ_INSTS_MFMA'] * 16384)


def test_a_kernel_missing_from_the_profiles_is_an_error(tmp_path):
    trace, pmc = _profiles(tmp_path, 1)
    with pytest.raises(ValueError, match='no dispatch'):
        mu.summarize(trace, pmc, 'rbf_plane_kernel', 1.0)
