"""A CPU model of the 16-bit matrix-core kernels' own numerics (test
infrastructure; it models this repository's kernels, not the reference).

rbf_plane_kernel (vectra_amd/csrc/rbf_plane_impl.h) and rbf_tile_kernel
(rbf_tile_impl.h) do not follow the reference's online-softmax algorithm.
For bf16/fp16 inputs they compute, per (b, h) plane, in fp32:

  coef = (2 log2 e) * gamma
  c_j  = fma(-coef / 2, |k_j|^2, log2(e) * bias_j)              (-inf masked)
  plane: x_ij = fma(coef, q_i . k_j,               c_j - shift_i)
  tile:  x_ij = fma(coef, q_i . k_j - |q_i|^2 / 2, c_j) - shift_i
  w = exp2(x); hi = 16-bit(w); lo = 16-bit(w - hi)   (bf16 round to nearest,
                                                      fp16 round toward zero)
  acc_i = sum_j hi v_j + sum_j lo v_j
  total_i = sum_j w     (plane: the fp32 weights, added on the vector unit)
  total_i = sum_j (hi + lo)   (tile: a product of ones on the matrix core)
  out_i = acc_i * (1 / total_i)

with no clamp of the distance at 0 and no running maximum: shift_i = 0
unless the weight sums leave the range where the split is accurate
([2^-32, 2^32] for bf16, [2^-3, 2^15] for fp16).  The plane kernel tests the
16 queries of a block together and recomputes the whole block with each
query's own maximum logit subtracted; the tile kernel takes the exact passes
(a maximum pass, then a shifted pass) for every query of its work item when
a bias is present, gamma < 0, or any sum falls below the range.

The tile kernel's fast pass (no bias, gamma >= 0, at least FAST_KEYS keys)
comes first: each weight rounded once to fp16 (to nearest), no split, and the
values in fp16 (bf16 values converted to nearest, 2^16 and beyond to inf).
It stands if every sum T of the work item is at least FAST_SUM, every output
is finite, and at every output FAST_SIGMAS deviations of its rounding walk
fit the 16-bit accuracy contract:

  (FAST_WALK sqrt(sum_j w^_j^2) + 2^-25 Nk) / T * (max|v| + |o^|) + 2^-25
      <= GATE_ATOL + GATE_RTOL |o^|

(FAST_WALK = FAST_SIGMAS 2^-11 / sqrt(3); max|v| over the plane's values).
After the first eighth of the key tiles the pass checks its course with the
sums so far (the walk's term scaled to all keys, twice the allowance) and is
abandoned early where even that fails.  Otherwise the item takes the split
pass above.

Each query's path is reported as SPLIT (one unshifted split pass), SHIFTED
(recomputed with its maximum subtracted) or FAST.

Sums here are taken in float64 and rounded once (the matrix cores' order of
accumulation is not modelled), so the kernels match this model to ~1e-6
relative, not bit for bit.  tests/test_kernel_model.py bounds the model's
error against the fp64 oracle on the CPU, including both branches;
tests/test_kernel_model_gpu.py checks the kernels against the model.
"""

import numpy as np

F32 = np.float32
LOG2E = F32(1.4426950408889634)
TWO_LOG2E = F32(2.0) * LOG2E
SUM_RANGE = {'bf16': (F32(2.0 ** -32), F32(2.0 ** 32)), 'fp16': (F32(2.0 ** -3), F32(2.0 ** 15))}
# Query rows of one tile-kernel work item, by head dim: 4 waves x blocks of 16
# per wave (four blocks for 64-dim heads, two otherwise).
TILE_ITEM_ROWS = {32: 128, 64: 256, 128: 128}
FAST_KEYS = 1024      # the tile kernel tries its fast pass from this many keys
FAST_SUM = F32(256)   # and keeps it if every weight sum of the item is at least this
FAST_SIGMAS = 4.0     # and this many deviations of its rounding walk fit the contract
GATE_ATOL, GATE_RTOL = 1e-4, 1e-3  # the 16-bit paths' accuracy contract
FAST_WALK = FAST_SIGMAS * 2.0 ** -11 / np.sqrt(3.0)
TILE_KEYS = {32: 64, 64: 64, 128: 32}  # keys per tile, by head dim
SPLIT, SHIFTED, FAST = 0, 1, 2  # per-query paths


def to_bf16(x):
    """Round float32 values to bf16 (nearest, ties to even), as float32."""
    x = np.asarray(x, dtype=F32)
    bits = x.view(np.uint32).astype(np.uint64)
    rounded = ((bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    out = rounded.view(F32)
    return np.where(np.isnan(x), x, out).astype(F32)


def to_fp16_rtz(x):
    """Round float32 values to fp16 toward zero (v_cvt_pkrtz), as float32."""
    x = np.asarray(x, dtype=F32)
    with np.errstate(over='ignore'):
        h = x.astype(np.float16)
    too_far = np.abs(h.astype(F32)) > np.abs(x)
    h = np.where(too_far, np.nextafter(h, np.float16(0)), h)
    return h.astype(F32)


def split(w, kind):
    """(hi, lo) of the weights: hi + lo = w to ~2^-17 (bf16) / 2^-20 (fp16)."""
    rnd = to_bf16 if kind == 'bf16' else to_fp16_rtz
    hi = rnd(w)
    with np.errstate(invalid='ignore'):
        lo = rnd((w - hi).astype(F32))
    return hi, lo


def fma32(a, b, c):
    """fp32 fused multiply-add (the product is exact in float64)."""
    with np.errstate(invalid='ignore', over='ignore'):
        return (np.asarray(a, np.float64) * np.asarray(b, np.float64) + np.asarray(c, np.float64)).astype(F32)


def exp2_32(x):
    with np.errstate(over='ignore'):
        return np.exp2(np.asarray(x, np.float64)).astype(F32)


def _weighted_fast(x, v16):
    """(acc, total, sum of squared weights) of the fast pass: fp16 weights
    (nearest) against fp16 values."""
    w = exp2_32(x).astype(np.float16).astype(np.float64)
    with np.errstate(invalid='ignore', over='ignore'):
        acc = (w @ v16.astype(np.float64)).astype(F32)
        total = w.sum(-1).astype(F32)
        wsq = (w * w).sum(-1).astype(F32)
    return acc, total, wsq


def fast_misses(acc, total, wsq, vmax, seen, n_k, slack=1.0):
    """The tile kernel's check of its fast pass (rbf_tile_impl.h
    fast_misses): per query, whether the bound misses the contract at an
    output, a sum (scaled to n_k keys) is below FAST_SUM / slack, or an
    output is not finite.  `seen` keys of n_k have been summed."""
    grow = n_k / seen
    t = total.astype(np.float64)
    with np.errstate(invalid='ignore', over='ignore', divide='ignore'):
        o = np.abs(acc.astype(np.float64) / t[:, None])
        per_spread = (FAST_WALK * np.sqrt(wsq.astype(np.float64) / grow) + 2.0 ** -25 * seen) / t
        est = per_spread[:, None] * (vmax + o) + 2.0 ** -25
        ok = (est <= slack * (GATE_ATOL + GATE_RTOL * o)) & np.isfinite(o)
    return ~(ok.all(-1) & (t * grow * slack >= FAST_SUM))


def fast_pass(x0, v16, n_k, tile_keys=64):
    """The fast pass over one work item: (acc, total, kept).  It checks its
    course after the first eighth of the tiles (twice the allowance) and
    keeps its result only if its final sums pass."""
    tiles = -(-n_k // tile_keys)
    seen = min(tiles // 8 * tile_keys, n_k)
    acc, total, wsq = _weighted_fast(x0[:, :seen], v16[:seen])
    if fast_misses(acc, total, wsq, np.abs(v16[:seen]).max(), seen, n_k, slack=2.0).any():
        return None, None, False
    acc, total, wsq = _weighted_fast(x0, v16)
    kept = not fast_misses(acc, total, wsq, np.abs(v16).max(), n_k, n_k).any()
    return acc, total, kept


def _weighted(x, shift, v, kind, sum_of_weights=False):
    """(acc [n, dv], total [n]) of logits x [n, nk] with per-row shifts;
    total sums the split weights hi + lo, or the fp32 weights themselves."""
    w = exp2_32((x - shift[:, None]).astype(F32) if shift is not None else x)
    hi, lo = split(w, kind)
    v64 = v.astype(np.float64)
    with np.errstate(invalid='ignore', over='ignore'):
        acc = (hi.astype(np.float64) @ v64 + lo.astype(np.float64) @ v64).astype(F32)
        if sum_of_weights:
            total = w.astype(np.float64).sum(-1).astype(F32)
        else:
            total = (hi.astype(np.float64) + lo.astype(np.float64)).sum(-1).astype(F32)
    return acc, total


def _row_max(x):
    m = x.max(-1) if x.shape[-1] else np.full(x.shape[0], -np.inf, F32)
    return np.where(np.isneginf(m), F32(0), m).astype(F32)


def _in_range(total, kind):
    lo, hi = SUM_RANGE[kind]
    return (total >= lo) & (total <= hi)  # False for NaN


def _finish(acc, total):
    with np.errstate(divide='ignore', invalid='ignore'):
        inv = (F32(1) / total).astype(F32)
        return (acc * inv[:, None]).astype(F32)


def _folded_keys(k, gamma, bias):
    coef = F32(TWO_LOG2E * F32(gamma))
    sq = (k.astype(np.float64) ** 2).sum(-1).astype(F32)
    xb = np.zeros(k.shape[0], F32) if bias is None else (np.asarray(bias, F32) * LOG2E).astype(F32)
    return coef, fma32(F32(-0.5) * coef, sq, xb)


def plane(q, k, v, gamma, bias, kind, one_pass=False):
    """rbf_plane_kernel on one plane: q [nq, d], k [nk, d], v [nk, dv] (values
    already in the 16-bit type), gamma, bias [nk] or None.  Returns (out
    [nq, dv] float32, per-query paths: SPLIT or SHIFTED)."""
    q, k, v = (np.asarray(a, F32) for a in (q, k, v))
    coef, c = _folded_keys(k, gamma, bias)
    s = (q.astype(np.float64) @ k.astype(np.float64).T).astype(F32)
    nq = q.shape[0]
    out = np.zeros((nq, v.shape[1]), F32)
    path = np.full(nq, SPLIT, np.int8)
    for b0 in range(0, nq, 16):
        rows = slice(b0, min(b0 + 16, nq))
        x0 = fma32(coef, s[rows], c[None, :])
        acc, total = _weighted(x0, None, v, kind, sum_of_weights=True)
        if not one_pass and not _in_range(total, kind).all():
            shift = _row_max(x0)
            x = fma32(coef, s[rows], (c[None, :] - shift[:, None]).astype(F32))
            acc, total = _weighted(x, None, v, kind, sum_of_weights=True)
            path[rows] = SHIFTED
        out[rows] = _finish(acc, total)
    return out, path


def tile(q, k, v, gamma, bias, kind, one_pass=False, split_weights=False):
    """rbf_tile_kernel on one plane (work items of TILE_ITEM_ROWS query rows); same
    arguments as `plane`, paths SPLIT, SHIFTED or FAST.  `one_pass` models
    the split pass alone (no fast pass, no recompute); `split_weights` the
    VECTRA_FLAG_SPLIT_WEIGHTS flag (no fast pass)."""
    q, k, v = (np.asarray(a, F32) for a in (q, k, v))
    coef, c = _folded_keys(k, gamma, bias)
    nq = q.shape[0]
    half_q = (F32(-0.5) * (q.astype(np.float64) ** 2).sum(-1).astype(F32)).astype(F32)
    s = ((q.astype(np.float64) @ k.astype(np.float64).T) + half_q[:, None].astype(np.float64)).astype(F32)
    out = np.zeros((nq, v.shape[1]), F32)
    path = np.full(nq, SPLIT, np.int8)
    exact_always = bias is not None or not (coef >= 0)
    fast = not exact_always and not one_pass and not split_weights and k.shape[0] >= FAST_KEYS
    if fast:
        with np.errstate(over='ignore'):
            v16 = v.astype(np.float16).astype(F32)  # exact for fp16 inputs
    item_rows = TILE_ITEM_ROWS.get(q.shape[1], 128)
    for r0 in range(0, nq, item_rows):
        rows = slice(r0, min(r0 + item_rows, nq))
        x0 = fma32(coef, s[rows], c[None, :])
        if fast:
            acc, total, kept = fast_pass(x0, v16, k.shape[0], TILE_KEYS.get(q.shape[1], 64))
            if kept:
                out[rows] = _finish(acc, total)
                path[rows] = FAST
                continue
        exact = exact_always and not one_pass
        if not exact:
            acc, total = _weighted(x0, None, v, kind)
            lo = SUM_RANGE[kind][0]
            exact = not one_pass and not (total >= lo).all()
        if exact:
            acc, total = _weighted(x0, _row_max(x0), v, kind)
            path[rows] = SHIFTED
        out[rows] = _finish(acc, total)
    return out, path


def run(model, q, k, v, scale, bias, kind, one_pass=False, split_weights=False):
    """A model over [B, H, n, d] torch or numpy operands with the operator's
    broadcasting (scale [1|B, 1|H, 1, 1] or a scalar; bias [B, 1|H, 1, nk] or
    None).  Returns (out [B, H, nq, dv] float32, paths [B, H, nq])."""
    q, k, v = (np.asarray(a, F32) for a in (q, k, v))
    batch, heads, nq, _ = q.shape
    sc = np.asarray(scale, F32)
    sc = np.broadcast_to(sc.reshape(sc.shape[:2]) if sc.ndim == 4 else sc.reshape(1, 1), (batch, heads))
    bs = None if bias is None else np.broadcast_to(np.asarray(bias, F32)[:, :, 0, :], (batch, heads, k.shape[2]))
    extra = {'split_weights': split_weights} if model == 'tile' else {}
    out = np.zeros((batch, heads, nq, v.shape[-1]), F32)
    path = np.zeros((batch, heads, nq), np.int8)
    for b in range(batch):
        for h in range(heads):
            fn = plane if model == 'plane' else tile
            out[b, h], path[b, h] = fn(q[b, h], k[b, h], v[b, h], sc[b, h],
                                       None if bs is None else bs[b, h], kind, one_pass, **extra)
    return out, path
