"""Match validation and the replacement graph.

The subgraph matcher compares use-def topology with literals ignored, so one
template serves every shape.  Everything literals would have pinned down is
re-checked here from the matched nodes' fake-tensor metadata (as the
reference does in compiler/vectra_compiler/replacement.py:108-190), so
look-alikes that compute something else are refused: an exponent other than
2, reductions over another axis, a coefficient that varies per key or query,
a bias that varies per query, mismatched shapes or dtypes.

The replacement keeps the template's inputs and emits one call of
torch.ops.vectra.rbf_attention (replacement.py:193-235).
"""

import numbers
from collections.abc import Sequence

import torch
from torch import fx

from vectra_amd.compiler import pattern
from vectra_amd.kernels import custom_ops

aten = torch.ops.aten
SUPPORTED_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _meta(x) -> torch.Tensor | None:
    if isinstance(x, fx.Node):
        val = x.meta.get('val')
        if isinstance(val, torch.Tensor):
            return val
    return None


def bound_inputs(spec: pattern.PatternSpec, match) -> dict:
    """Graph values bound to each template placeholder, by name."""
    return dict(zip(spec.placeholder_names, match.placeholder_nodes, strict=True))


def _left_pad(shape: Sequence[int]) -> list[int] | None:
    if len(shape) > 4:
        return None
    return [1] * (4 - len(shape)) + list(shape)


def _per_head(shape: Sequence[int], lead: Sequence[int]) -> bool:
    """Broadcastable to [B, H, 1, 1]."""
    s = _left_pad(shape)
    return (
        s is not None
        and s[2] == 1
        and s[3] == 1
        and all(x in (1, n) for x, n in zip(s[:2], lead, strict=True))
    )


def _per_key(shape: Sequence[int], lead: Sequence[int], n_k: int) -> bool:
    """Broadcastable to [B, H, 1, Nk]."""
    s = _left_pad(shape)
    return (
        s is not None
        and s[2] == 1
        and s[3] in (1, n_k)
        and all(x in (1, n) for x, n in zip(s[:2], lead, strict=True))
    )


def _axes(dims, rank: int) -> list[int]:
    return sorted(d % rank for d in dims)


def _literals_agree(match) -> bool:
    """The checks literals would have made: squares, last-axis reductions."""
    for template_node, node in match.nodes_map.items():
        if template_node.op != 'call_function' or not isinstance(node, fx.Node):
            continue
        if node.target is aten.pow.Tensor_Scalar and node.args[1] != 2:
            return False
        if node.target in (aten.sum.dim_IntList, aten.amax.default):
            src = _meta(node.args[0])
            if src is None or len(node.args) < 2:
                return False
            if _axes(node.args[1], src.dim()) != [src.dim() - 1]:
                return False
            want = template_node.args[2] if len(template_node.args) > 2 else False
            got = node.args[2] if len(node.args) > 2 else False
            if bool(got) != bool(want):
                return False
    return True


def _pairs_every_query_with_every_key(match, lead, n_q, n_k, dim) -> bool:
    """The difference node must be [B, H, Nq, Nk, D]."""
    for template_node, node in match.nodes_map.items():
        if template_node.op != 'call_function' or template_node.target is not aten.sub.Tensor:
            continue
        if not all(
            isinstance(a, fx.Node) and a.target is aten.unsqueeze.default
            for a in template_node.args
        ):
            continue
        diff = _meta(node)
        if diff is None or tuple(diff.shape) != (*lead, n_q, n_k, dim):
            return False
    return True


def make_filter(spec: pattern.PatternSpec):
    """The semantic check for matches of `spec`."""

    def accept(match, original_graph, template_graph) -> bool:
        del original_graph, template_graph
        bound = bound_inputs(spec, match)
        q, k, v = _meta(bound[pattern.Q]), _meta(bound[pattern.K]), _meta(bound[pattern.V_BMM])
        if q is None or k is None or v is None:
            return False
        if (q.dim(), k.dim(), v.dim()) != (4, 4, 3):
            return False
        lead = tuple(q.shape[:2])
        n_q, dim, n_k = q.shape[2], q.shape[3], k.shape[2]
        if tuple(k.shape[:2]) != lead or k.shape[3] != dim:
            return False
        if v.shape[0] != lead[0] * lead[1] or v.shape[1] != n_k:
            return False
        if q.dtype not in SUPPORTED_DTYPES or not q.dtype == k.dtype == v.dtype:
            return False
        if not _pairs_every_query_with_every_key(match, lead, n_q, n_k, dim):
            return False
        if not _literals_agree(match):
            return False
        coefficient = bound[pattern.SCALE]
        if isinstance(coefficient, fx.Node):
            c = _meta(coefficient)
            if c is None or not _per_head(c.shape, lead):
                return False
        elif not isinstance(coefficient, numbers.Real) or (
            spec.coefficient == 'divisor' and coefficient == 0
        ):
            return False
        if spec.has_bias:
            bias = _meta(bound[pattern.BIAS])
            if bias is None or not _per_key(bias.shape, lead, n_k):
                return False
        out = _meta(match.returning_nodes[0])
        return out is not None and tuple(out.shape) == (*lead, n_q, v.shape[2])

    return accept


def make_replacement(spec: pattern.PatternSpec):
    """Builds the replacement graph for a match of `spec`."""

    def build(match, original_graph, template_graph) -> fx.Graph:
        del original_graph, template_graph
        bound = bound_inputs(spec, match)
        q, v = _meta(bound[pattern.Q]), _meta(bound[pattern.V_BMM])
        graph = fx.Graph()
        inputs = {name: graph.placeholder(name) for name in spec.placeholder_names}
        value = graph.call_function(
            aten.reshape.default,
            (inputs[pattern.V_BMM], [q.shape[0], q.shape[1], v.shape[1], v.shape[2]]),
        )
        coefficient = bound[pattern.SCALE]
        if isinstance(coefficient, fx.Node):
            scale = inputs[pattern.SCALE]
            if spec.coefficient == 'divisor':
                scale = graph.call_function(aten.reciprocal.default, (scale,))
        else:
            c = float(coefficient)
            scale = graph.call_function(
                aten.scalar_tensor.default,
                (1.0 / c if spec.coefficient == 'divisor' else c,),
                {'dtype': torch.float32, 'device': q.device},
            )
        bias = inputs[pattern.BIAS] if spec.has_bias else None
        out = graph.call_function(
            custom_ops.overload(),
            (inputs[pattern.Q], inputs[pattern.K], value, scale, bias),
        )
        graph.output(out)
        return graph

    return build
