"""The full-model throughput comparison's gate logic (CPU; the timing runs on the GPU)."""

from vectra_amd.benchmarks import model_throughput


def _run(mode, rps, error=0.0, **overrides):
    record = {'mode': mode, 'device': 'AMD Instinct MI355X', 'batch_size': 1024, 'block_dtype': 'float16',
              'num_candidates': 64, 'num_layers': 3, 'requests_per_s': rps,
              'max_abs_error_vs_eager': error, 'numerics_rtol': 1e-3}
    record.update(overrides)
    return record


def test_compare_passes_a_fast_matching_candidate():
    passed, problems, ratio = model_throughput.compare(_run('eager', 1e5), _run('vectra', 4e5, 0.004), 3.0)
    assert passed and not problems and ratio == 4.0


def test_compare_flags_slow_mismatched_or_inaccurate_candidates():
    passed, problems, _ = model_throughput.compare(_run('eager', 1e5), _run('vectra', 2e5), 3.0)
    assert not passed and any('ratio' in p for p in problems)
    passed, problems, _ = model_throughput.compare(_run('eager', 1e5),
                                                   _run('vectra', 5e5, batch_size=512), 3.0)
    assert not passed and any('batch_size' in p for p in problems)
    passed, problems, _ = model_throughput.compare(_run('eager', 1e5), _run('vectra', 5e5, 0.05), 3.0)
    assert not passed and any('numerics' in p for p in problems)


def test_config_5_shape():
    config = model_throughput.config_5(4)
    assert (config.d_model, config.num_heads, config.num_layers, config.attribute_dim,
            config.num_candidates) == (128, 8, 4, 16, 64)
