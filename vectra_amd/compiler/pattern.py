"""Catalog of eager RBF-attention formulations and their ATen templates.

Behaviour follows the reference's compiler/vectra_compiler/pattern.py:65-400:

* Eight formulations (the CATALOG): coefficient as a divisor (-d / c) or a
  multiplier (-d * c), with or without an additive key bias, normalised by
  torch.softmax or by exp / sum.
* Each is captured as a template by running its eager function through
  TorchInductor's own front end and stopping at the joint-graph pre-pass,
  the hook the rewrite runs at, so templates track the installed torch.
* Templates are cut at the value operand of the final bmm (placeholder
  `v_bmm`), which keeps V's memory layout out of the match.
* Templates and model graphs are brought to one canonical form by rewrites
  that are exact in IEEE arithmetic: x * x -> x ** 2, and negations moved onto
  the distance operand of the logit products.

Precision tags: '[fp32]' and '[half]' (float16 and bfloat16 decompose alike)
for softmax, whose decomposition depends on the dtype; '[any]' where the fp32
and half templates are identical.  In addition to the reference's tags this
catalog captures '[autocast]' templates: the same formulations traced under
torch.autocast(bfloat16), whose graphs carry the casts autocast inserts
around pow, sum and softmax.
"""

import copy
import dataclasses
import functools
import itertools
import numbers
from collections.abc import Callable

import torch
from torch import fx
from torch._inductor import compile_fx
from torch._inductor import config as inductor_config
from torch._inductor.fx_passes import post_grad

aten = torch.ops.aten

# Template placeholder names, in graph order after the value cut.
Q, K, SCALE, BIAS, V_BMM = 'q', 'k', 'scale', 'bias', 'v_bmm'

COEFFICIENTS = ('divisor', 'multiplier')
NORMALIZATIONS = ('softmax', 'exp_sum')


@dataclasses.dataclass(frozen=True)
class PatternSpec:
    """One formulation of RBF attention."""

    coefficient: str  # 'divisor' (-d / c) or 'multiplier' (-d * c)
    has_bias: bool
    normalization: str  # 'softmax' or 'exp_sum'

    @property
    def name(self) -> str:
        middle = '_bias' if self.has_bias else ''
        return f'rbf_{self.coefficient}{middle}_{self.normalization}'

    @property
    def placeholder_names(self) -> tuple[str, ...]:
        return (Q, K, SCALE, BIAS, V_BMM) if self.has_bias else (Q, K, SCALE, V_BMM)

    def eager_fn(self) -> Callable[..., torch.Tensor]:
        """This formulation as plain eager PyTorch, v last."""
        divisor = self.coefficient == 'divisor'
        softmax = self.normalization == 'softmax'

        def attend(q, k, c, bias, v):
            sq_dist = (q.unsqueeze(-2) - k.unsqueeze(-3)).pow(2).sum(-1)
            logits = -sq_dist / c if divisor else -sq_dist * c
            if bias is not None:
                logits = logits + bias
            if softmax:
                weights = torch.softmax(logits, dim=-1)
            else:
                e = torch.exp(logits)
                weights = e / e.sum(-1, keepdim=True)
            return weights @ v

        if self.has_bias:
            def with_bias(q, k, c, bias, v):
                return attend(q, k, c, bias, v)
            return with_bias

        def without_bias(q, k, c, v):
            return attend(q, k, c, None, v)
        return without_bias


CATALOG = tuple(
    PatternSpec(coefficient, has_bias, normalization)
    for has_bias, coefficient, normalization in itertools.product(
        (True, False), COEFFICIENTS, NORMALIZATIONS
    )
)

# Precisions templates are captured at.  'autocast' traces bfloat16 q, k, v
# with a float32 coefficient and bias under torch.autocast(bfloat16).
PRECISIONS = ('fp32', 'half', 'autocast')


@dataclasses.dataclass(frozen=True)
class CapturedPattern:
    """A catalog entry's template for one precision tag."""

    spec: PatternSpec
    precision: str  # 'fp32' | 'half' | 'any' | 'autocast'
    graph_module: fx.GraphModule

    @property
    def name(self) -> str:
        return f'{self.spec.name}[{self.precision}]'


# ------------------------------------------------------------ canonical form


def canonicalize_squares(graph: fx.Graph) -> int:
    """mul(x, x) -> pow(x, 2), in place; returns the number of rewrites."""
    rewrites = 0
    for node in list(graph.nodes):
        if not (node.op == 'call_function' and node.target is aten.mul.Tensor):
            continue
        if len(node.args) != 2 or node.kwargs:
            continue
        x, y = node.args
        if not isinstance(x, fx.Node) or x is not y:
            continue
        with graph.inserting_before(node):
            square = graph.call_function(aten.pow.Tensor_Scalar, (x, 2))
        square.meta = dict(node.meta)
        node.replace_all_uses_with(square)
        graph.erase_node(node)
        rewrites += 1
    return rewrites


_SIGN_SINKS = {aten.exp.default, aten.amax.default}
_SIGN_CHAIN = {
    aten.neg.default,
    aten.mul.Tensor,
    aten.div.Tensor,
    aten.add.Tensor,
    aten.sub.Tensor,
}


def _sign_region(graph: fx.Graph) -> set[fx.Node]:
    """Pointwise mul/div/add/sub/neg nodes upstream of an exp or amax.

    Sign rewrites are confined to these logit chains so the rest of the
    graph reaches Inductor exactly as it was.
    """
    region: set[fx.Node] = set()
    frontier = [
        arg
        for node in graph.nodes
        if node.op == 'call_function' and node.target in _SIGN_SINKS
        for arg in node.args
        if isinstance(arg, fx.Node)
    ]
    while frontier:
        node = frontier.pop()
        if node in region or node.op != 'call_function' or node.target not in _SIGN_CHAIN:
            continue
        region.add(node)
        frontier.extend(arg for arg in node.args if isinstance(arg, fx.Node))
    return region


def _real(x) -> bool:
    return isinstance(x, numbers.Real) and not isinstance(x, bool)


def _numel(x) -> int:
    val = x.meta.get('val') if isinstance(x, fx.Node) else None
    return val.numel() if isinstance(val, torch.Tensor) else 1


def _is_neg(x) -> bool:
    return isinstance(x, fx.Node) and x.op == 'call_function' and x.target is aten.neg.default


def _negated(graph: fx.Graph, x: fx.Node, before: fx.Node) -> fx.Node:
    """-x as a node: unwraps an existing negation, else inserts one."""
    if _is_neg(x):
        return x.args[0]
    with graph.inserting_before(before):
        neg = graph.call_function(aten.neg.default, (x,))
    neg.meta = dict(x.meta)
    return neg


def _rewrite_sign(graph: fx.Graph, node: fx.Node) -> bool:
    """One exact sign rewrite at `node`, if any applies."""
    if node.kwargs or not node.users:
        return False
    if node.target is aten.neg.default:
        inner = node.args[0]
        if not isinstance(inner, fx.Node):
            return False
        if _is_neg(inner):  # --a -> a
            node.replace_all_uses_with(inner.args[0])
            return True
        if (
            inner.op == 'call_function'
            and inner.target in (aten.mul.Tensor, aten.div.Tensor)
            and len(inner.users) == 1
            and not inner.kwargs
            and isinstance(inner.args[0], fx.Node)
        ):  # -(a*b) -> (-a)*b ; -(a/b) -> (-a)/b
            inner.args = (_negated(graph, inner.args[0], inner), inner.args[1])
            node.replace_all_uses_with(inner)
            return True
        return False
    if node.target not in (aten.mul.Tensor, aten.div.Tensor) or len(node.args) != 2:
        return False
    a, b = node.args
    if not isinstance(a, fx.Node):
        return False
    if node.target is aten.mul.Tensor and isinstance(b, fx.Node) and _numel(b) > _numel(a):
        node.args = (b, a)  # the larger operand (the distances) first
        return True
    if _is_neg(b):  # a*(-b) -> (-a)*b ; a/(-b) -> (-a)/b
        node.args = (_negated(graph, a, node), b.args[0])
        return True
    if _real(b) and b < 0:  # a*(-c) -> (-a)*c ; a/(-c) -> (-a)/c
        node.args = (_negated(graph, a, node), -b)
        return True
    return False


def canonicalize_signs(graph: fx.Graph) -> int:
    """Moves negations onto the first operand of logit products, in place.

    Negation commutes with IEEE rounding and multiplication is commutative,
    so no rewrite changes a value, whether or not the graph then matches.
    Returns the number of rewrites.
    """
    total = 0
    while True:
        region = _sign_region(graph)
        changed = 0
        for node in [n for n in graph.nodes if n in region]:
            changed += _rewrite_sign(graph, node)
        graph.eliminate_dead_code()
        if not changed:
            return total
        total += changed


def canonicalize(graph: fx.Graph) -> None:
    """The normal form shared by templates and model graphs."""
    canonicalize_squares(graph)
    canonicalize_signs(graph)


# ------------------------------------------------------------------ capture


class _Captured(Exception):
    """Raised from the pre-pass hook once the template graph is recorded."""


def _cut_at_value(gm: fx.GraphModule) -> fx.GraphModule:
    """Makes the final bmm's value operand the `v_bmm` placeholder."""
    graph = gm.graph
    post_grad.remove_noop_ops(graph)
    bmm = next(n for n in reversed(graph.nodes) if n.target is aten.bmm.default)
    inputs = [n for n in graph.nodes if n.op == 'placeholder']
    v_input = inputs[-1]  # eager functions take v last
    with graph.inserting_after(v_input):
        v_bmm = graph.placeholder(V_BMM)
    bmm.args = (bmm.args[0], v_bmm)
    graph.eliminate_dead_code()
    if v_input.users:
        raise RuntimeError('template uses its value input outside the final bmm')
    graph.erase_node(v_input)
    canonicalize(graph)
    graph.lint()
    gm.recompile()
    return gm


def _template_inputs(spec: PatternSpec, device: torch.device, precision: str):
    gen = torch.Generator().manual_seed(0)
    q = torch.randn(2, 3, 5, 8, generator=gen)
    k = torch.randn(2, 3, 7, 8, generator=gen)
    v = torch.randn(2, 3, 7, 8, generator=gen)
    c = torch.rand(1, 3, 1, 1, generator=gen) + 0.5
    bias = torch.zeros(2, 1, 1, 7)
    io_dtype = {'fp32': torch.float32, 'half': torch.float16, 'autocast': torch.bfloat16}[precision]
    param_dtype = torch.float32 if precision == 'autocast' else io_dtype
    out = [q.to(device, io_dtype), k.to(device, io_dtype), c.to(device, param_dtype)]
    if spec.has_bias:
        out.append(bias.to(device, param_dtype))
    out.append(v.to(device, io_dtype))
    return out


def capture(spec: PatternSpec, device: torch.device, precision: str) -> fx.GraphModule:
    """Traces `spec` through Inductor up to the joint-graph pre-pass.

    Runs outside any enclosing Dynamo trace (static shapes, its own fake
    mode) and returns the canonical template cut at `v_bmm`.
    """
    traced = fx.symbolic_trace(spec.eager_fn())
    recorded: dict[str, fx.GraphModule] = {}

    def record(graph: fx.Graph) -> None:
        recorded['gm'] = copy.deepcopy(graph.owning_module)
        raise _Captured()

    autocast = (
        torch.autocast(device.type, dtype=torch.bfloat16)
        if precision == 'autocast'
        else torch.autocast(device.type, enabled=False)
    )
    with torch._guards.tracing(None), torch.no_grad(), autocast:  # pylint: disable=protected-access
        with inductor_config.patch(joint_custom_pre_pass=record, fx_graph_cache=False):
            try:
                compile_fx.compile_fx(traced, _template_inputs(spec, device, precision))
            except Exception:  # pylint: disable=broad-except
                # Inductor wraps the stop signal; only a missing graph is a failure.
                if 'gm' not in recorded:
                    raise
    return _cut_at_value(recorded['gm'])


@functools.cache
def load_catalog(device_type: str) -> tuple[CapturedPattern, ...]:
    """All templates for a device type, captured once per process.

    When a formulation's fp32 and half templates are the same graph it is
    kept once, tagged '[any]'.  Autocast templates identical to one already
    kept are dropped.
    """
    device = torch.device(device_type)
    entries: list[CapturedPattern] = []
    for spec in CATALOG:
        fp32 = capture(spec, device, 'fp32')
        half = capture(spec, device, 'half')
        kept = []
        if fp32.code == half.code:
            kept.append(CapturedPattern(spec, 'any', fp32))
        else:
            kept += [CapturedPattern(spec, 'fp32', fp32), CapturedPattern(spec, 'half', half)]
        mixed = capture(spec, device, 'autocast')
        if all(mixed.code != entry.graph_module.code for entry in kept):
            kept.append(CapturedPattern(spec, 'autocast', mixed))
        entries += kept
    return tuple(entries)
