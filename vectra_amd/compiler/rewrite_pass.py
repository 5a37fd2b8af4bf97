"""The joint-graph pre-pass that splices vectra::rbf_attention into graphs.

Behaviour follows compiler/vectra_compiler/rewrite_pass.py:37-122 of the
reference: graphs that take tangents (training graphs) are left alone since
the operator has no backward; the model graph is brought to the templates'
canonical form; every template of the catalog is matched with
torch.fx.subgraph_rewriter.replace_pattern_with_filters, validated by
replacement.make_filter and replaced by replacement.make_replacement; new
nodes get fake-tensor values so later Inductor passes can read them.  The
pass is idempotent (Inductor may run it more than once on a graph).
"""

import collections

import torch
from torch import fx
from torch._inductor import custom_graph_pass
from torch._inductor.fx_passes import post_grad
from torch.fx import subgraph_rewriter

from vectra_amd.compiler import pattern
from vectra_amd.compiler import replacement


def _fill_fake_values(graph: fx.Graph) -> None:
    """Evaluates nodes the rewrite created under the graph's fake mode."""
    inputs = [n.meta.get('val') for n in graph.nodes if n.op == 'placeholder']
    fake_mode = torch._guards.detect_fake_mode(inputs)  # pylint: disable=protected-access
    if fake_mode is None:
        return
    with fake_mode:
        for node in graph.nodes:
            if node.op != 'call_function' or 'val' in node.meta:
                continue
            args = fx.node.map_arg(node.args, lambda n: n.meta['val'])
            kwargs = fx.node.map_arg(node.kwargs, lambda n: n.meta['val'])
            node.meta['val'] = node.target(*args, **kwargs)  # pylint: disable=not-an-iterable,not-a-mapping


def is_training_graph(graph: fx.Graph) -> bool:
    """A joint forward-backward graph takes `tangents_*` inputs."""
    return any(n.op == 'placeholder' and str(n.target).startswith('tangents') for n in graph.nodes)


class RbfAttentionRewrite(custom_graph_pass.CustomGraphPass):
    """Replaces eager RBF attention with torch.ops.vectra.rbf_attention.

    Attributes:
      matches: sites rewritten so far, per catalog entry name.
    """

    def __init__(self, catalog: tuple[pattern.CapturedPattern, ...]):
        self._catalog = catalog
        self.matches: collections.Counter = collections.Counter()

    @property
    def total_matches(self) -> int:
        return sum(self.matches.values())

    def __call__(self, graph: fx.Graph) -> None:
        if is_training_graph(graph):
            return
        gm = graph.owning_module
        post_grad.remove_noop_ops(graph)
        pattern.canonicalize(graph)
        replaced_any = False
        for entry in self._catalog:
            replaced = subgraph_rewriter.replace_pattern_with_filters(
                gm,
                entry.graph_module,
                match_filters=[replacement.make_filter(entry.spec)],
                ignore_literals=True,
                replacement_callback=replacement.make_replacement(entry.spec),
            )
            if replaced:
                self.matches[entry.name] += len(replaced)
                replaced_any = True
                # A later site may consume this one's output (stacked
                # layers); its filter reads the new nodes' fake values.
                _fill_fake_values(graph)
        if replaced_any:
            graph.eliminate_dead_code()
            graph.lint()

    def uuid(self) -> bytes:
        """Cache key: the sources of the pass and its templates."""
        return custom_graph_pass.get_hash_for_files(
            (__file__, pattern.__file__, replacement.__file__)
        )
