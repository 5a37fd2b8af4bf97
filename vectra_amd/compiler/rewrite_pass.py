"""Inductor joint-graph pre-pass that puts vectra::rbf_attention in place of
eager RBF-attention regions.

How one graph is rewritten (RbfAttentionRewrite.__call__):

1. A graph with `tangents_*` inputs computes gradients as well; the operator
   has no backward, so such a graph goes through unchanged.
2. The graph is brought to the templates' normal form: no-op views are
   dropped and pattern.canonicalize applies the exact algebraic rewrites the
   templates were captured under.
3. Template by template, in catalog order, fx's subgraph rewriter finds every
   non-overlapping occurrence; replacement.make_filter keeps only the
   occurrences that are RBF attention and replacement.make_replacement emits
   the operator call for each.
4. The nodes a template's rewrites created carry no fake value yet.  They get
   one before the next template runs, because a site whose q and k come from
   an earlier site's output (stacked layers) is filtered on those values.
5. Dead nodes are dropped and the graph is linted.

Running the pass again over its own output finds nothing new: the operator's
call matches no template.

Reference behaviour: compiler/vectra_compiler/rewrite_pass.py:37-122.
"""

import collections
import hashlib
import sys

from torch import fx
from torch._inductor import custom_graph_pass
from torch._inductor.fx_passes import post_grad
from torch._subclasses import fake_tensor
from torch.fx import subgraph_rewriter

from vectra_amd.compiler import pattern
from vectra_amd.compiler import replacement


def is_training_graph(graph: fx.Graph) -> bool:
    """Whether `graph` is a joint forward/backward graph (it takes tangents)."""
    return any(str(node.target).startswith('tangents') for node in graph.find_nodes(op='placeholder'))


def _graph_fake_mode(graph: fx.Graph):
    """The FakeTensorMode the graph's inputs were traced under, or None."""
    for node in graph.find_nodes(op='placeholder'):
        value = node.meta.get('val')
        if isinstance(value, fake_tensor.FakeTensor):
            return value.fake_mode
    return None


def _annotate_new_nodes(graph: fx.Graph) -> int:
    """Gives every call node without a fake value one, evaluated under the
    graph's fake mode in graph (topological) order; returns how many."""
    pending = [n for n in graph.nodes if n.op == 'call_function' and 'val' not in n.meta]
    mode = _graph_fake_mode(graph) if pending else None
    if mode is None:
        return 0

    def value_of(node):
        return node.meta['val']

    with mode:
        for node in pending:
            args, kwargs = fx.node.map_arg((node.args, node.kwargs), value_of)
            node.meta['val'] = node.target(*args, **kwargs)
    return len(pending)


class RbfAttentionRewrite(custom_graph_pass.CustomGraphPass):
    """The pre-pass, over one catalog of captured templates.

    Attributes:
      matches: sites rewritten so far, per catalog entry name, over every
        graph this instance has seen.
      graphs_seen / training_graphs_skipped: graphs handed to the pass, and
        how many of them were left alone as training graphs.
    """

    def __init__(self, catalog: tuple[pattern.CapturedPattern, ...]):
        self._catalog = tuple(catalog)
        self.matches: collections.Counter = collections.Counter()
        self.graphs_seen = 0
        self.training_graphs_skipped = 0

    @property
    def total_matches(self) -> int:
        return sum(self.matches.values())

    def _apply(self, module: fx.GraphModule, entry: pattern.CapturedPattern) -> int:
        found = subgraph_rewriter.replace_pattern_with_filters(
            module,
            entry.graph_module,
            match_filters=[replacement.make_filter(entry.spec)],
            ignore_literals=True,
            replacement_callback=replacement.make_replacement(entry.spec),
        )
        return len(found)

    def __call__(self, graph: fx.Graph) -> None:
        self.graphs_seen += 1
        if is_training_graph(graph):
            self.training_graphs_skipped += 1
            return
        post_grad.remove_noop_ops(graph)
        pattern.canonicalize(graph)
        rewritten = 0
        for entry in self._catalog:
            count = self._apply(graph.owning_module, entry)
            if count == 0:
                continue
            self.matches[entry.name] += count
            rewritten += count
            _annotate_new_nodes(graph)
        if rewritten:
            graph.eliminate_dead_code()
            graph.lint()

    def uuid(self) -> bytes:
        """Changes whenever this module, the templates or the filter change."""
        digest = hashlib.sha256()
        for module in (sys.modules[__name__], pattern, replacement):
            with open(module.__file__, 'rb') as f:
                digest.update(f.read())
        return digest.digest()
