"""Benchmark workloads (CPU): the model-site layout and moving inputs."""

import torch

from vectra_amd.benchmarks import configs


def test_the_model_site_is_a_view_of_one_projection():
    c = configs.MODEL_SITE
    inputs = configs.make_inputs(c, seed=0, batch=3)
    q, k, v = inputs.q, inputs.k, inputs.v
    width = c.heads * c.head_dim
    assert q.shape == k.shape == v.shape == (3, c.heads, c.n_q, c.head_dim)
    # Rows of D elements, 3 H D apart; heads D apart; k and v a third further on.
    assert q.stride() == (c.n_q * 3 * width, c.head_dim, 3 * width, 1)
    assert k.storage_offset() - q.storage_offset() == width
    assert v.storage_offset() - q.storage_offset() == 2 * width
    assert q._base is k._base is v._base  # pylint: disable=protected-access
    projection = q._base  # pylint: disable=protected-access
    assert torch.equal(q[1, 2, 5], projection[1, 5, 2 * c.head_dim:3 * c.head_dim])
    assert torch.equal(v[2, 7, 64], projection[2, 64, 2 * width + 7 * c.head_dim:2 * width + 8 * c.head_dim])
    # The subject and 8-64 comparables are live; the rest are masked.
    assert inputs.key_bias.shape == (3, 1, 1, c.n_k) and inputs.key_bias.dtype == torch.float16
    assert ((inputs.counts >= 9) & (inputs.counts <= 65)).all()
    live = torch.isfinite(inputs.key_bias[:, 0, 0]).sum(-1)
    assert torch.equal(live, inputs.counts)


def test_moving_inputs_keeps_the_views():
    inputs = configs.make_inputs(configs.MODEL_SITE, seed=1, batch=2)
    moved = inputs.to('meta')
    for before, after in zip((inputs.q, inputs.k, inputs.v), (moved.q, moved.k, moved.v)):
        assert after.device.type == 'meta'
        assert after.stride() == before.stride() and after.storage_offset() == before.storage_offset()
    # Inputs that are not views of one tensor move as they are.
    plain = configs.make_inputs(configs.SERVING, seed=1, batch=2)
    assert plain.to('meta').q.is_contiguous()
