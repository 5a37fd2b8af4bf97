"""Installing the pass in TorchInductor, and single-graph capture checks.

Behaviour follows compiler/vectra_compiler/inductor_hook.py:41-95 of the
reference: the rewrite is Inductor's joint-graph pre-pass (the first hook on
the decomposed ATen graph, before Inductor's own algebraic rewrites), the FX
graph cache is off while it is installed so every compile runs the pass, and
a model that TorchDynamo captures as more than one graph is refused.
"""

import contextlib
import dataclasses

import torch
from torch._inductor import config as inductor_config

from vectra_amd.compiler import rewrite_pass


class GraphBreakError(RuntimeError):
    """The model does not compile to a single graph."""


@contextlib.contextmanager
def installed(rewrite: rewrite_pass.RbfAttentionRewrite):
    """Runs `rewrite` as Inductor's joint-graph pre-pass inside the block."""
    with inductor_config.patch(joint_custom_pre_pass=rewrite, fx_graph_cache=False):
        yield


@dataclasses.dataclass(frozen=True)
class CaptureReport:
    """TorchDynamo's capture summary for one call.

    graph_break_count counts recorded break reasons as well, since
    graph_count - 1 misses a break whose resumed code traces no tensor op.
    """

    graph_count: int
    graph_break_count: int
    break_reasons: tuple[str, ...]


def explain(model: torch.nn.Module, *inputs) -> CaptureReport:
    """torch._dynamo.explain over one call."""
    result = torch._dynamo.explain(model)(*inputs)  # pylint: disable=protected-access
    reasons = tuple(str(r.reason) for r in result.break_reasons)
    return CaptureReport(
        graph_count=result.graph_count,
        graph_break_count=max(result.graph_break_count, len(reasons)),
        break_reasons=reasons,
    )


def assert_single_graph(model: torch.nn.Module, *inputs) -> CaptureReport:
    """Raises GraphBreakError unless the call captures as exactly one graph."""
    report = explain(model, *inputs)
    if report.graph_break_count or report.graph_count != 1:
        raise GraphBreakError(
            f'{report.graph_count} graph(s), {report.graph_break_count} graph break(s): '
            + '; '.join(report.break_reasons)
        )
    return report
