"""Loader for tests/golden/rbf_golden.npz (written by tests/golden/make_golden.py)."""

import functools
import os

import numpy as np
import torch

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden', 'rbf_golden.npz')

DTYPES = {'float32': torch.float32, 'float16': torch.float16, 'bfloat16': torch.bfloat16}


@functools.cache
def cases() -> dict:
    """name -> dict(q, k, v, scale, bias, dtype, expected) as torch CPU tensors.

    q, k, v are in the case's dtype (their stored float32 values are exact in
    it); scale is fp32 [B,H,1,1]; bias fp32 [B,1|H,1,Nk] or None; expected is
    float64.
    """
    data = np.load(PATH, allow_pickle=False)
    names = sorted({key.split('/')[0] for key in data.files})
    out = {}
    for name in names:
        dtype = DTYPES[str(data[f'{name}/dtype'])]

        def get(field, cast=None):
            key = f'{name}/{field}'
            if key not in data.files:
                return None
            t = torch.from_numpy(np.array(data[key]))
            return t.to(cast) if cast is not None else t

        out[name] = {
            'q': get('q', dtype),
            'k': get('k', dtype),
            'v': get('v', dtype),
            'scale': get('scale', torch.float32),
            'bias': get('bias', torch.float32),
            'dtype': dtype,
            'expected': get('expected'),
        }
    return out
