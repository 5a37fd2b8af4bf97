"""Where the rewrite runs inside TorchInductor, and the one-graph check.

The rewrite is installed as Inductor's `joint_custom_pre_pass`, the first
custom hook to see the decomposed ATen graph and the last point before
Inductor's own pattern passes could split or fuse an attention region.  A
pre-pass that the caller had installed already keeps running, after ours.
While the rewrite is installed the FX graph cache is off: a cache hit would
skip the pass, and its match counts would then not describe the compile.

The one-graph check compiles the model once with a recording backend that
keeps every graph TorchDynamo hands it and runs the graph eagerly.  Each
graph carries the reason TorchDynamo ended it (`compile_subgraph_reason`);
a graph that ended at a break says so, with the break's cause, even when the
code resumed after the break traces no tensor op and so adds no graph.  A
serving model must come out as one graph with no break, because a break
inside an attention region hides the region from the rewrite.

Reference behaviour: compiler/vectra_compiler/inductor_hook.py:41-95.
"""

import contextlib
import dataclasses
import hashlib

import torch
from torch._inductor import config as inductor_config
from torch._inductor import custom_graph_pass

from vectra_amd.compiler import rewrite_pass


class GraphBreakError(RuntimeError):
    """The model does not capture as a single graph."""


class _PassChain(custom_graph_pass.CustomGraphPass):
    """Runs several pre-passes in order, with one combined cache key."""

    def __init__(self, *passes):
        self.passes = passes

    def __call__(self, graph):
        for one in self.passes:
            one(graph)

    def uuid(self):
        digest = hashlib.sha256()
        for one in self.passes:
            key = one.uuid() if hasattr(one, 'uuid') else repr(one)
            digest.update(key if isinstance(key, bytes) else str(key).encode())
        return digest.digest()


@contextlib.contextmanager
def installed(rewrite: rewrite_pass.RbfAttentionRewrite):
    """Inside the block, Inductor compiles run `rewrite` as their joint-graph
    pre-pass (before any pre-pass already installed), with the FX graph cache
    off."""
    earlier = inductor_config.joint_custom_pre_pass
    chosen = rewrite if earlier is None else _PassChain(rewrite, earlier)
    with inductor_config.patch({'joint_custom_pre_pass': chosen, 'fx_graph_cache': False}):
        yield rewrite


@dataclasses.dataclass(frozen=True)
class CaptureReport:
    """How one call of a model captures under TorchDynamo.

    graph_count: graphs the call was split into;
    graph_break_count: breaks TorchDynamo recorded (at least graph_count - 1;
      a break whose resumed code traces no tensor op adds a reason but no
      graph);
    break_reasons: the distinct reasons, as TorchDynamo words them;
    op_count: call nodes over all graphs.
    """

    graph_count: int
    graph_break_count: int
    break_reasons: tuple[str, ...]
    op_count: int = 0


def _break_reason(gm: torch.fx.GraphModule) -> str | None:
    """Why TorchDynamo ended `gm` at a graph break, or None if it did not."""
    reason = getattr(gm, 'compile_subgraph_reason', None)
    if reason is None or not getattr(reason, 'graph_break', False):
        return None
    return str(reason.reason)


def explain(model: torch.nn.Module, *inputs) -> CaptureReport:
    """Captures one call of `model` and reports its graphs and breaks.

    TorchDynamo's state is reset before and after, so the capture neither
    reuses nor leaves behind compiled frames.
    """
    graphs = []

    def recording_backend(gm: torch.fx.GraphModule, example_inputs):
        del example_inputs
        graphs.append(gm)
        return gm.forward

    torch._dynamo.reset()  # pylint: disable=protected-access
    try:
        with torch.no_grad():
            torch.compile(model, backend=recording_backend, dynamic=False)(*inputs)
    finally:
        torch._dynamo.reset()  # pylint: disable=protected-access
    reasons = [r for r in map(_break_reason, graphs) if r is not None]
    breaks = max(len(reasons), len(graphs) - 1)
    ops = sum(1 for gm in graphs for node in gm.graph.nodes
              if node.op in ('call_function', 'call_method', 'call_module'))
    return CaptureReport(graph_count=len(graphs), graph_break_count=breaks,
                         break_reasons=tuple(dict.fromkeys(reasons)), op_count=ops)


def assert_single_graph(model: torch.nn.Module, *inputs) -> CaptureReport:
    """The capture report of one call, or GraphBreakError if the call does
    not capture as exactly one graph with no break."""
    report = explain(model, *inputs)
    if report.graph_count != 1 or report.graph_break_count:
        detail = '; '.join(report.break_reasons) or 'no reason recorded'
        raise GraphBreakError(f'the model captures as {report.graph_count} graph(s) with '
                              f'{report.graph_break_count} break(s): {detail}')
    return report
