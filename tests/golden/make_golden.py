"""Writes tests/golden/rbf_golden.npz: small RBF-attention cases with their
expected outputs computed by brute force.

The reference ships no golden vectors for this path (its numerics tests draw
seeded inputs at run time and compare with its float64 oracle,
kernels/tests/test_parity.py:49-98).  These fixtures are computed here by
the most literal reading of the operator's definition
(kernels/vectra_kernels/custom_ops.py:52-72; reference.py:46-58), independent of oracle/: pure
Python float64 loops over b, h, i, j, d with math.exp, an explicit
maximum subtraction, NaN for a row whose keys are all masked, and zeros for an
empty key set.

  python tests/golden/make_golden.py

Inputs are drawn with numpy's PCG64 from fixed seeds; half-precision cases
store float32 arrays whose values are exactly representable in that dtype.
"""

import math
import os

import numpy as np
import torch

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'rbf_golden.npz')


def brute_force(q, k, v, scale, bias):
    """out[b,h,i,:] = sum_j softmax_j(-s*sum_d (q-k)^2 + bias_j) v_j, float64."""
    batch, heads, n_q, dim = q.shape
    n_k, dv = k.shape[2], v.shape[3]
    out = np.zeros((batch, heads, n_q, dv))
    for b in range(batch):
        for h in range(heads):
            s = float(scale[b, h])
            for i in range(n_q):
                logits = []
                for j in range(n_k):
                    sq = 0.0
                    for d in range(dim):
                        diff = float(q[b, h, i, d]) - float(k[b, h, j, d])
                        sq += diff * diff
                    x = -s * sq
                    if bias is not None:
                        x += float(bias[b, h, j])
                    logits.append(x)
                if n_k == 0:
                    continue
                m = max(logits)
                if m == -math.inf:
                    out[b, h, i, :] = math.nan
                    continue
                w = [math.exp(x - m) for x in logits]
                total = math.fsum(w)
                for c in range(dv):
                    out[b, h, i, c] = math.fsum(
                        w[j] * float(v[b, h, j, c]) for j in range(n_k)
                    ) / total
    return out


def _round(x, dtype):
    return torch.from_numpy(x).to(dtype).float().numpy()


def _case(rng, batch, heads, n_q, n_k, dim, dv, *, dtype=torch.float32, scale=None,
          counts=None, bias_per_head=False, qk_std=1.0):
    q = _round(rng.standard_normal((batch, heads, n_q, dim)) * qk_std, dtype)
    k = _round(rng.standard_normal((batch, heads, n_k, dim)) * qk_std, dtype)
    v = _round(rng.standard_normal((batch, heads, n_k, dv)), dtype)
    if scale is None:
        scale = 1.0 / (2.0 * dim * (0.5 + rng.random((1, heads, 1, 1))))
    scale = np.broadcast_to(np.asarray(scale, dtype=np.float64).reshape(
        (1,) * (4 - np.ndim(scale)) + np.shape(scale)), (batch, heads, 1, 1))
    scale = scale.astype(np.float32)
    bias = None
    if counts is not None:
        bh = heads if bias_per_head else 1
        bias = np.zeros((batch, bh, 1, n_k), dtype=np.float32)
        for b in range(batch):
            for h in range(bh):
                c = counts[b] if np.ndim(counts[b]) == 0 else counts[b][h]
                bias[b, h, 0, c:] = -np.inf
    return q, k, v, scale, bias


def cases():
    """name -> (q, k, v, scale [B,H,1,1] fp32, bias [B,1|H,1,Nk] fp32 or None, dtype)."""
    rng = np.random.default_rng(20251201)
    out = {}
    out['tiny'] = _case(rng, 1, 2, 3, 5, 4, 3, counts=[4]) + ('float32',)
    out['cpu_eager_like'] = _case(rng, 2, 4, 1, 32, 16, 16, scale=0.5 / 16,
                                  counts=[7, 32]) + ('float32',)
    out['serving_like_bf16'] = _case(rng, 3, 8, 1, 64, 32, 32, dtype=torch.bfloat16,
                                     scale=0.01 + 0.09 * rng.random((1, 8, 1, 1)),
                                     counts=[8, 37, 64]) + ('bfloat16',)
    out['self_attention_like_fp16'] = _case(rng, 1, 2, 9, 9, 32, 32, dtype=torch.float16,
                                            scale=1.0 / 32, counts=[5]) + ('float16',)
    out['ragged_dims'] = _case(rng, 1, 1, 5, 37, 3, 7) + ('float32',)
    out['single_key'] = _case(rng, 1, 2, 4, 1, 8, 8) + ('float32',)
    out['one_live_key'] = _case(rng, 2, 2, 3, 70, 16, 16, counts=[1, 1]) + ('float32',)
    out['per_head_bias'] = _case(rng, 2, 3, 2, 20, 8, 8, counts=[[20, 5, 11], [1, 20, 9]],
                                 bias_per_head=True) + ('float32',)
    out['fully_masked'] = _case(rng, 1, 1, 2, 6, 4, 4, counts=[0]) + ('float32',)
    out['zero_scale'] = _case(rng, 1, 2, 3, 12, 8, 8, scale=0.0, counts=[9]) + ('float32',)
    out['negative_scale'] = _case(rng, 1, 2, 3, 12, 8, 8, scale=-0.01) + ('float32',)
    out['far_points'] = _case(rng, 1, 2, 4, 20, 16, 16, scale=0.1, qk_std=20.0) + ('float32',)
    out['no_keys'] = _case(rng, 1, 2, 3, 0, 8, 4) + ('float32',)
    return out


def main():
    arrays = {}
    for name, (q, k, v, scale, bias, dtype) in cases().items():
        bias_b = None if bias is None else np.broadcast_to(
            bias, (q.shape[0], q.shape[1], 1, k.shape[2]))[:, :, 0, :]
        expected = brute_force(q, k, v, scale[:, :, 0, 0], bias_b)
        arrays[f'{name}/q'] = q
        arrays[f'{name}/k'] = k
        arrays[f'{name}/v'] = v
        arrays[f'{name}/scale'] = scale
        if bias is not None:
            arrays[f'{name}/bias'] = bias
        arrays[f'{name}/dtype'] = np.array(dtype)
        arrays[f'{name}/expected'] = expected
    np.savez_compressed(OUT, **arrays)
    print(f'wrote {OUT}: {len(cases())} cases')


if __name__ == '__main__':
    main()
