"""CPU restatements of the reference's RBF-attention formulations.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Every function takes
torch tensors or numpy arrays on any device and computes on the host.

Shapes: q [B, H, Nq, D], k [B, H, Nk, D], v [B, H, Nk, Dv]; scale broadcast
to [B, H, 1, 1]; key_bias (optional) broadcast to [B, 1|H, 1, Nk].
"""

import numpy as np
import torch

# Bound on the float64 [planes, Nq, Nk, D] difference tensor a chunk of the
# direct formulation may materialise.
_CHUNK_BYTES = 256 << 20


def _np64(x):
    if x is None:
        return None
    if isinstance(x, torch.Tensor):
        return x.detach().to('cpu', torch.float64).numpy()
    return np.asarray(x, dtype=np.float64)


def _operands(q, k, v, scale, key_bias):
    """float64 arrays with scale as [B,H,1,1] and bias as [B,H,1,Nk]."""
    q, k, v = _np64(q), _np64(k), _np64(v)
    batch, heads = q.shape[:2]
    n_k = k.shape[2]
    s = _np64(scale)
    s = np.broadcast_to(s.reshape((1,) * (4 - s.ndim) + s.shape), (batch, heads, 1, 1))
    bias = None
    if key_bias is not None:
        bias = _np64(key_bias)
        bias = bias.reshape((1,) * (4 - bias.ndim) + bias.shape)
        if bias.shape[-2] != 1:
            raise ValueError('key_bias must be constant across queries')
        bias = np.broadcast_to(bias, (batch, heads, 1, n_k))
    return q, k, v, s, bias


def _softmax_fp64(logits):
    """torch.softmax semantics in float64: an all -inf row gives NaN."""
    with np.errstate(invalid='ignore'):
        m = logits.max(axis=-1, keepdims=True)
        e = np.exp(logits - m)
        return e / e.sum(axis=-1, keepdims=True)


def _attend(logits, v):
    if logits.shape[-1] == 0:  # softmax over no keys contributes nothing
        return np.zeros((*logits.shape[:-1], v.shape[-1]))
    return _softmax_fp64(logits) @ v


def direct_fp64(q, k, v, scale, key_bias=None):
    """The eager chain of reference.py:46-58 in float64: sum_d (q_i - k_j)^2.

    Materialises the [.., Nq, Nk, D] difference, chunked over batches so the
    largest configs fit in memory.  Returns float64 [B, H, Nq, Dv].
    """
    q, k, v, s, bias = _operands(q, k, v, scale, key_bias)
    batch, heads, n_q, dim = q.shape
    n_k = k.shape[2]
    per_batch = max(1, heads * n_q * n_k * max(dim, 1) * 8)
    step = max(1, _CHUNK_BYTES // per_batch)
    out = np.empty((batch, heads, n_q, v.shape[-1]))
    for b0 in range(0, batch, step):
        sl = slice(b0, b0 + step)
        diff = q[sl, :, :, None, :] - k[sl, :, None, :, :]
        sq = np.einsum('bhijd,bhijd->bhij', diff, diff)
        logits = -sq * s[sl]
        if bias is not None:
            logits = logits + bias[sl]
        out[sl] = _attend(logits, v[sl])
    return out


def expanded_fp64(q, k, v, scale, key_bias=None):
    """The float64 Euclidean-expansion oracle of reference.py:61-76.

    |q|^2 + |k|^2 - 2 q.k, clamped at 0.  Returns float64 [B, H, Nq, Dv].
    """
    q, k, v, s, bias = _operands(q, k, v, scale, key_bias)
    q_norm = (q * q).sum(-1, keepdims=True)
    k_norm = (k * k).sum(-1)[..., None, :]
    sq = np.maximum(q_norm + k_norm - 2.0 * (q @ np.swapaxes(k, -1, -2)), 0.0)
    logits = -sq * s
    if bias is not None:
        logits = logits + bias
    return _attend(logits, v)


def eager_fp32(q, k, v, scale, key_bias=None, batch_chunk=None):
    """The eager operator chain of reference.py:54-58, in torch float32 on CPU.

    This is the comparator the parity gates name ("the eager formulation
    evaluated in fp32 on the same bf16-rounded inputs") and the CPU baseline
    bench.py times.  `batch_chunk` bounds the [.., Nq, Nk, D] intermediate.
    Returns a float32 CPU tensor [B, H, Nq, Dv].
    """

    def cpu32(t):
        return None if t is None else t.detach().to('cpu', torch.float32)

    q, k, v, scale, key_bias = map(cpu32, (q, k, v, scale, key_bias))

    def chain(q, k, v, scale, key_bias):
        sq_dist = (q.unsqueeze(-2) - k.unsqueeze(-3)).pow(2).sum(-1)
        logits = -sq_dist * scale
        if key_bias is not None:
            logits = logits + key_bias
        return torch.softmax(logits, dim=-1) @ v

    if batch_chunk is None or batch_chunk >= q.shape[0]:
        return chain(q, k, v, scale, key_bias)

    def rows(t, sl):
        # Batch-broadcast operands (leading dim 1, or fewer dims) stay whole.
        if t is None or t.dim() < 4 or t.shape[0] == 1:
            return t
        return t[sl]

    parts = []
    for b0 in range(0, q.shape[0], batch_chunk):
        sl = slice(b0, b0 + batch_chunk)
        parts.append(
            chain(q[sl], k[sl], v[sl], rows(scale, sl), rows(key_bias, sl))
        )
    return torch.cat(parts)


def tiled(q, k, v, scale, key_bias=None, block_q=64, block_k=64, dtype=np.float64):
    """The kernel's algorithm tile for tile (reference.py:102-161).

    Per query tile: resident query norms; per key tile: GEMM-form distances
    clamped at 0, logits, an online max with the -inf guard (safe_max = 0
    while the running max is -inf), rescaled running sum and accumulator.
    Arithmetic in `dtype`.  Returns [B, H, Nq, Dv] in `dtype`.
    """
    q, k, v, s, bias = _operands(q, k, v, scale, key_bias)
    q, k, v, s = (x.astype(dtype) for x in (q, k, v, s))
    if bias is not None:
        bias = bias.astype(dtype)
    batch, heads, n_q, _ = q.shape
    n_k, dv = k.shape[2], v.shape[-1]
    out = np.zeros((batch, heads, n_q, dv), dtype=dtype)
    for q0 in range(0, n_q, block_q):
        qt = q[:, :, q0 : q0 + block_q]
        q_norm = (qt * qt).sum(-1, keepdims=True)
        rows = qt.shape[2]
        run_max = np.full((batch, heads, rows, 1), -np.inf, dtype=dtype)
        run_sum = np.zeros_like(run_max)
        acc = np.zeros((batch, heads, rows, dv), dtype=dtype)
        for k0 in range(0, n_k, block_k):
            kt = k[:, :, k0 : k0 + block_k]
            vt = v[:, :, k0 : k0 + block_k]
            k_norm = (kt * kt).sum(-1)[..., None, :]
            sq = np.maximum(q_norm + k_norm - 2 * (qt @ np.swapaxes(kt, -1, -2)), 0)
            logits = -s * sq
            if bias is not None:
                logits = logits + bias[..., k0 : k0 + block_k]
            new_max = np.maximum(run_max, logits.max(-1, keepdims=True))
            safe = np.where(np.isneginf(new_max), 0, new_max)
            alpha = np.exp(run_max - safe)
            w = np.exp(logits - safe)
            run_sum = run_sum * alpha + w.sum(-1, keepdims=True)
            acc = acc * alpha + w @ vt
            run_max = new_max
        with np.errstate(invalid='ignore', divide='ignore'):
            out[:, :, q0 : q0 + rows] = (
                acc / run_sum if n_k else np.zeros_like(acc)
            )
    return out
