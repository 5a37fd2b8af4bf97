"""After the rewrite, compiled code computes what the eager code computed
(CPU Inductor).

Behaviour restated from the reference's compiler/tests/test_rewrite_correctness.py:
every catalog formulation is rewritten to exactly one site at ordinary and
degenerate shapes; coefficients given as Python numbers work; half-precision
graphs and (added here) autocast graphs are rewritten; graphs that compute
gradients are left alone; the canonicalisation the pass applies first
changes no bit of any result; the pass's cache key is stable.
"""

import pytest
import torch
from torch import fx

from tests import compiler_helpers as ch
from vectra_amd.compiler import backend
from vectra_amd.compiler import pattern
from vectra_amd.compiler import rewrite_pass

aten = torch.ops.aten
TOL = {'rtol': 1e-4, 'atol': 1e-5}


@pytest.fixture(autouse=True)
def _fresh_dynamo():
    torch._dynamo.reset()  # pylint: disable=protected-access
    yield
    torch._dynamo.reset()  # pylint: disable=protected-access


def _arguments(spec: pattern.PatternSpec, ops: ch.Operands, mask_last_key=True) -> list:
    """Positional arguments of spec.eager_fn(): q, k, coefficient[, bias], v."""
    two_sigma_sq = 2 * ops.sigma**2
    args = [ops.q, ops.k, two_sigma_sq if spec.coefficient == 'divisor' else two_sigma_sq.reciprocal()]
    if spec.has_bias:
        bias = torch.zeros(ops.q.shape[0], 1, 1, ops.k.shape[2], dtype=ops.q.dtype)
        if mask_last_key:
            bias[-1, ..., -1] = float('-inf')
        args.append(bias)
    return args + [ops.v]


# (batch, heads, n_q, n_k, dim, dim_v)
SHAPES = {
    'model_like': (2, 3, 6, 9, 8, 8),
    'one_of_each': (1, 1, 1, 2, 1, 2),
    'odd_sizes': (3, 2, 5, 37, 3, 7),
    'lone_key': (1, 2, 17, 1, 16, 2),
}


@pytest.mark.parametrize('shape', sorted(SHAPES))
@pytest.mark.parametrize('spec', pattern.CATALOG, ids=lambda s: s.name)
def test_every_formulation_rewrites_to_one_site(spec, shape):
    b, h, n_q, n_k, d, dv = SHAPES[shape]
    if spec.has_bias and n_k == 1:
        pytest.skip('masking the lone key would leave a row with nothing to attend to')
    args = _arguments(spec, ch.operands(b, h, n_q, n_k, d, dv, seed=21))
    fn = spec.eager_fn()
    out, report = ch.run_vectra(fn, *args)
    assert report.sites == 1 and len(report.matches) == 1, report.matches
    (name,) = report.matches
    assert name.split('[')[0] == spec.name
    torch.testing.assert_close(out, fn(*args), **TOL)


def test_a_single_query_with_one_value_column_keeps_the_eager_graph():
    # With Nq = 1 and Dv = 1 Inductor's CPU lowering turns the value bmm into
    # a multiply and a sum, so the templates' bmm anchor is absent.
    spec = pattern.CATALOG[0]
    args = _arguments(spec, ch.operands(1, 1, 1, 3, 2, 1, seed=2))
    fn = spec.eager_fn()
    out, report = ch.run_vectra(fn, *args)
    assert report.sites == 0
    torch.testing.assert_close(out, fn(*args), **TOL)


@pytest.mark.parametrize('spec', pattern.CATALOG, ids=lambda s: s.name)
def test_a_python_number_coefficient_is_accepted(spec):
    ops = ch.operands(seed=4)
    number = 3.0 if spec.coefficient == 'divisor' else 1.0 / 3.0
    bias = [torch.zeros(2, 1, 1, ops.k.shape[2])] if spec.has_bias else []
    fn = spec.eager_fn()

    def literal(q, k, *rest):
        return fn(q, k, number, *rest)

    out, report = ch.run_vectra(literal, ops.q, ops.k, *bias, ops.v)
    assert report.sites == 1, report.matches
    torch.testing.assert_close(out, literal(ops.q, ops.k, *bias, ops.v), **TOL)


@pytest.mark.parametrize('dtype', [torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize('spec', pattern.CATALOG, ids=lambda s: s.name)
def test_half_precision_graphs_are_rewritten(spec, dtype):
    args = _arguments(spec, ch.operands(dtype=dtype, seed=8))
    fn = spec.eager_fn()
    out, report = ch.run_vectra(fn, *args)
    assert report.sites == 1, report.matches
    (name,) = report.matches
    assert name.endswith(('[half]', '[any]'))
    assert out.dtype == dtype
    # Against fp32 eager on the same rounded values: the compiled graph (like
    # eager) runs part of its arithmetic in the half dtype.
    want = fn(*(a.float() if isinstance(a, torch.Tensor) else a for a in args))
    tol = 1e-2 if dtype == torch.float16 else 4e-2
    torch.testing.assert_close(out.float(), want, rtol=tol, atol=tol)


@pytest.mark.parametrize('spec', pattern.CATALOG, ids=lambda s: s.name)
def test_autocast_graphs_are_rewritten(spec):
    # bf16 q, k, v (what autocast Linear layers hand on) with an fp32
    # coefficient and bias; autocast's own casts are part of the template.
    ops = ch.operands(seed=6)
    args = _arguments(spec, ops)
    args = [a.bfloat16() if a is ops.q or a is ops.k or a is ops.v else a for a in args]
    fn = spec.eager_fn()

    def autocast_region(*xs):
        with torch.autocast('cpu', dtype=torch.bfloat16):
            return fn(*xs)

    out, report = ch.run_vectra(autocast_region, *args)
    assert report.sites == 1, report.matches
    want = fn(*(a.float() if isinstance(a, torch.Tensor) else a for a in args))
    torch.testing.assert_close(out.float(), want, rtol=4e-2, atol=4e-2)


def test_graphs_that_compute_gradients_are_not_rewritten():
    ops = ch.operands(seed=9)
    leaves = [t.detach().clone().requires_grad_() for t in ops]
    fn = pattern.CATALOG[0].eager_fn()
    bias = torch.zeros(2, 1, 1, ops.k.shape[2])

    def loss(q, k, v, sigma):
        return fn(q, k, 2 * sigma**2, bias, v).pow(2).mean()

    torch._dynamo.reset()  # pylint: disable=protected-access
    report = backend.CompileReport()
    torch.compile(loss, backend=backend.make_backend(report))(*leaves).backward()
    assert report.sites == 0
    compiled_grads = [t.grad for t in leaves]
    eager_leaves = [t.detach().clone().requires_grad_() for t in ops]
    loss(*eager_leaves).backward()
    for got, t in zip(compiled_grads, eager_leaves):
        torch.testing.assert_close(got, t.grad, **TOL)


# ------------------------------------------------------ canonicalisation

class _Evaluate(fx.Interpreter):
    """Runs a graph, leaving each node's value in node.meta['val']."""

    def run_node(self, n):
        n.meta['val'] = super().run_node(n)
        return n.meta['val']


def _graph_of(*expressions) -> fx.GraphModule:
    """A graph over inputs a, b, c returning exp() of each expression; an
    expression is a function of (call, a, b, c) building aten nodes."""
    graph = fx.Graph()
    a, b, c = graph.placeholder('a'), graph.placeholder('b'), graph.placeholder('c')
    call = graph.call_function
    graph.output(tuple(call(aten.exp.default, (build(call, a, b, c),)) for build in expressions))
    return fx.GraphModule(torch.nn.Module(), graph)


SIGNED = (
    lambda call, a, b, c: call(aten.neg.default, (call(aten.mul.Tensor, (a, c)),)),
    lambda call, a, b, c: call(aten.mul.Tensor, (a, call(aten.neg.default, (c,)))),
    lambda call, a, b, c: call(aten.mul.Tensor, (c, call(aten.neg.default, (a,)))),
    lambda call, a, b, c: call(aten.mul.Tensor, (a, -0.625)),
    lambda call, a, b, c: call(aten.div.Tensor, (a, call(aten.neg.default, (c,)))),
    lambda call, a, b, c: call(aten.neg.default, (call(aten.div.Tensor, (b, -1.5)),)),
)


def test_moving_signs_changes_no_bit():
    gen = torch.Generator().manual_seed(17)
    a, b = torch.randn(2, 2, 3, 4, 5, generator=gen)
    c = 0.1 + torch.rand(1, 3, 1, 1, generator=gen)
    gm = _graph_of(*SIGNED)
    before = _Evaluate(gm).run(a, b, c)
    assert pattern.canonicalize_signs(gm.graph) > 0
    gm.recompile()
    for x, y in zip(before, gm(a, b, c)):
        assert torch.equal(x, y)
    # Normal form: a negation, if any, sits on the first operand of each
    # product or quotient; no literal operand is negative.
    for node in gm.graph.nodes:
        if node.target in (aten.mul.Tensor, aten.div.Tensor):
            lhs, rhs = node.args
            assert not (isinstance(rhs, (int, float)) and rhs < 0), node.format_node()
            assert not (isinstance(rhs, fx.Node) and rhs.target is aten.neg.default), node.format_node()
            assert lhs.op == 'placeholder' or lhs.target is aten.neg.default, node.format_node()


def test_arithmetic_outside_the_normal_form_is_untouched():
    graph = fx.Graph()
    a, c = graph.placeholder('a'), graph.placeholder('c')
    scaled = graph.call_function(aten.mul.Tensor, (c, -4.0))
    graph.output(graph.call_function(aten.sub.Tensor, (a, scaled)))
    text = str(graph)
    assert pattern.canonicalize_signs(graph) == 0
    assert str(graph) == text


def test_the_cache_key_depends_only_on_the_pass_sources():
    entries = pattern.load_catalog('cpu')
    key = rewrite_pass.RbfAttentionRewrite(entries).uuid()
    assert isinstance(key, bytes) and len(key) == 32
    assert key == rewrite_pass.RbfAttentionRewrite(entries[:1]).uuid()
