"""The matrix-core / vector-unit co-execution probe (vectra_amd/benchmarks/coexec_probe.hip)
and the issue model vectra_amd/benchmarks/coexec.py derives from it.

The model's arithmetic is checked on synthetic probe timings built from known
per-instruction costs (the model must recover them, and a mix's floor must be
the larger of its two sides); the library's entry points are checked for
their argument validation without touching a device; on a GPU the probe runs
and its costs are ordered as the hardware must order them.
"""

import ctypes
import os

import pytest
import torch

from vectra_amd.benchmarks import coexec


def _rows(fma, exp2, mfma, block, mfma32, block32):
    """Two-wave ticks per iteration that an exact issue model would produce."""
    def t(n_mfma, n_valu, has_exp, big):
        n_exp = n_valu // 4 if has_exp else 0
        vector = (n_valu - n_exp) * fma + n_exp * exp2 + n_mfma * (block32 if big else block)
        matrix = n_mfma * (mfma32 if big else mfma)
        return 2.0 * max(vector, matrix)  # two waves share the SIMD

    rows = []
    for n_mfma, n_valu, has_exp, big in ((8, 0, False, False), (0, 32, False, False), (0, 32, True, False),
                                         (8, 16, False, False), (8, 32, False, False), (8, 64, False, False),
                                         (8, 32, True, False), (4, 0, False, True), (4, 32, False, True)):
        rows.append({'mfma': n_mfma, 'valu': n_valu, 'exp2': has_exp, 'mfma_32x32x16': big,
                     'ticks_per_iter_1w': 0.0, 'ticks_per_iter_2w': t(n_mfma, n_valu, has_exp, big)})
    return rows


def test_issue_model_recovers_known_costs():
    model = coexec.issue_model(_rows(fma=2.5, exp2=8.0, mfma=12.0, block=9.5, mfma32=24.0, block32=12.0))
    assert model['fma'] == pytest.approx(2.5)
    assert model['exp2'] == pytest.approx(8.0)
    assert model['mfma'] == pytest.approx(12.0)
    assert model['mfma_valu_block'] == pytest.approx(9.5)
    assert model['mfma_32x32x16'] == pytest.approx(24.0)
    assert model['mfma_32x32x16_valu_block'] == pytest.approx(12.0)


def test_floor_is_the_larger_side():
    model = {'fma': 2.0, 'exp2': 6.0, 'mfma': 10.0, 'mfma_valu_block': 5.0}
    vector_bound = coexec.floor_ticks(model, valu=100, exp2=20, mfma=10)
    assert vector_bound['vector_side'] == pytest.approx(80 * 2.0 + 20 * 6.0 + 10 * 5.0)
    assert vector_bound['matrix_side'] == pytest.approx(100.0)
    assert vector_bound['floor'] == vector_bound['vector_side']
    matrix_bound = coexec.floor_ticks(model, valu=4, exp2=0, mfma=10)
    assert matrix_bound['floor'] == pytest.approx(100.0) == matrix_bound['matrix_side']


def _library_or_skip():
    if not os.path.exists(coexec.BENCH_LIBRARY):
        pytest.skip('libvectra_bench.so is not built')
    return coexec._library()


def test_probe_entry_points_validate_arguments():
    lib = _library_or_skip()
    n = lib.vectra_bench_coexec_variants()
    assert n == 9
    assert coexec.describe(lib, 0) == {'mfma': 8, 'valu': 0, 'exp2': False, 'mfma_32x32x16': False}
    assert coexec.describe(lib, 8) == {'mfma': 4, 'valu': 32, 'exp2': False, 'mfma_32x32x16': True}
    with pytest.raises(ValueError):
        coexec.describe(lib, n)
    per, ratio, iters = ctypes.c_double(), ctypes.c_double(), ctypes.c_int()
    # Rejected before any device call: bad variant, bad wave count, null buffers.
    for i, waves, buf in ((n, 1, 1), (-1, 1, 1), (0, 3, 1), (0, 1, None)):
        assert lib.vectra_bench_coexec(i, waves, buf, buf, ctypes.byref(per), ctypes.byref(ratio),
                                       ctypes.byref(iters)) == 1


@pytest.mark.gpu
def test_probe_costs_are_ordered_on_the_device():
    if not torch.cuda.is_available():
        pytest.skip('needs a GPU')
    _library_or_skip()
    rows = coexec.run_probes()
    model = coexec.issue_model(rows)
    assert all(r['ticks_per_iter_1w'] > 0 and r['ticks_per_iter_2w'] > 0 for r in rows)
    assert 1.0 < rows[0]['tick_ghz_2w'] < 4.0
    # An exp2 costs more than an FMA; an MFMA takes some vector issue but less
    # than its own matrix-pipe time; a 32x32x16 product is twice a 16x16x32 one
    # on the matrix pipe.
    assert model['exp2'] > model['fma'] > 0
    assert 0 < model['mfma_valu_block'] < model['mfma']
    assert model['mfma_32x32x16'] == pytest.approx(2 * model['mfma'], rel=0.2)
