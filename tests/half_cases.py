"""The 16-bit edge cases shared by the GPU parity tests and the CPU model of
the plane and tile kernels (tests/kernel_model.py).

Each case is [2, 2, n_q, dim] queries and [2, 2, n_k, dim] keys and values
(normal draws from a seeded generator) with a coefficient and a key bias that
drive one of the kernels' branches: far points (weights that underflow unless
shifted), gamma < 0 and = 0, fully masked rows, one live key, biases far from
0, ragged masks.  The shapes select the plane kernel (D = 16 and 32) and the
tile kernel (D = 32 and 64).
"""

import math

import torch

HALF_CASES = ['far_points', 'negative_scale', 'zero_scale', 'fully_masked', 'one_live_key', 'large_biases',
              'ragged_mask']

HALF_KERNEL_SHAPES = {'plane16': (24, 70, 16), 'plane32': (40, 65, 32), 'tile32': (40, 200, 32),
                      'tile64': (33, 130, 64)}


def half_case(case, n_q, n_k, dim, gen):
    q = torch.randn(2, 2, n_q, dim, generator=gen)
    k = torch.randn(2, 2, n_k, dim, generator=gen)
    v = torch.randn(2, 2, n_k, dim, generator=gen)
    scale, bias = torch.tensor(0.5 / dim), None
    if case == 'far_points':
        # Every key far from every query (gamma d of a few hundred), so the
        # weights underflow unless each query's largest logit is subtracted;
        # distances stay where fp32 resolves them to the tolerance.
        q, k, scale = q * 3, k * 3, torch.tensor(0.3)
    elif case == 'negative_scale':
        scale = torch.tensor(-0.01)
    elif case == 'zero_scale':
        scale = torch.tensor(0.0)
        bias = torch.randn(2, 1, 1, n_k, generator=gen)
    elif case == 'fully_masked':
        bias = torch.zeros(2, 1, 1, n_k)
        bias[1] = -math.inf
    elif case == 'one_live_key':
        bias = torch.full((2, 1, 1, n_k), -math.inf)
        bias[..., n_k // 2] = 0.0
    elif case == 'large_biases':  # a per-key bias far above the distance term
        bias = 40.0 * torch.randn(2, 2, 1, n_k, generator=gen)
    elif case == 'ragged_mask':
        bias = torch.zeros(2, 1, 1, n_k)
        bias[0, ..., n_k // 3:] = -math.inf
    return q, k, v, scale, bias
