"""Fuse elementwise add/mul chains that follow zentorch_woq_linear.

Binary-binary, as the reference (src/cpu/python/zentorch/_woq_linear_binary_binary_fusion.py:136-225):
``(woq * m) + a`` -> ``zentorch_woq_linear_mul_add`` and ``(woq + a1) + a2``
-> ``zentorch_woq_linear_add_add``, in every operand order of the two ops
(each op is commutative, so the four orders are the same value).

Extension, applied after the binary-binary patterns so those take
precedence: a single ``woq + a`` / ``a + woq`` -> ``zentorch_woq_linear_add``
(the Llama down projection's residual add); the reference registers the op
but no pass for it.

Every extra operand must have the output's shape and dtype: the fused ops
neither broadcast nor promote (the reference checks the shape, :38-59).
"""
import functools
from typing import Any, Callable, Iterable

import torch
from torch._inductor import config
from torch._inductor.pattern_matcher import (
    CallFunction,
    KeywordArg,
    Match,
    PatternMatcherPass,
    register_graph_pattern,
    stable_topological_sort,
)
from torch.fx.graph import Graph

from ._utils import counters, on_gpu, tensor_meta
from ._woq_linear_unary_fusion import _OPERANDS, woq_call

aten = torch.ops.aten

binary_binary_pass = PatternMatcherPass(pass_name="zentorch_woq_linear_binary_binary_pass")
binary_pass = PatternMatcherPass(pass_name="zentorch_woq_linear_binary_pass")

_ATEN = {"add": aten.add.Tensor, "mul": aten.mul.Tensor}


def _either_order(op: Any, a: Any, b: Any) -> Iterable[CallFunction]:
    yield CallFunction(op, a, b)
    yield CallFunction(op, b, a)


def _operands_match_output(names: tuple) -> Callable[[Match], bool]:
    def check(match: Match) -> bool:
        out = tensor_meta(match.output_node())
        if out is None or not on_gpu(out) or out.dtype not in (torch.bfloat16, torch.float32):
            return False
        woq = [n for n in match.nodes
               if n.target is torch.ops.zentorch.zentorch_woq_linear.default]
        wv = tensor_meta(woq[0]) if len(woq) == 1 else None
        # the fused op returns the woq output's dtype and shape
        if wv is None or not on_gpu(wv) or wv.dtype != out.dtype \
                or tuple(wv.shape) != tuple(out.shape):
            return False
        for name in names:
            v = tensor_meta(match.kwargs.get(name))
            if v is None or not on_gpu(v) or tuple(v.shape) != tuple(out.shape) \
                    or v.dtype != out.dtype:
                return False
        return True

    return check


def _replacement(op_name: str, extra: tuple) -> Callable:
    def handler(match: Match, **kw: Any) -> None:
        names = [n for n in _OPERANDS if n in kw]

        def repl(*vals: Any) -> torch.Tensor:
            ops = dict(zip(names, vals[:len(names)]))
            counters["zentorch"][op_name] += 1
            return getattr(torch.ops.zentorch, op_name)(
                ops["input"], ops["weight"], ops["weight_scales"],
                ops["weight_zero_points"], *vals[len(names):], ops.get("bias"))

        match.replace_by_example(repl, [kw[n] for n in names] + [kw[e] for e in extra])

    return handler


@functools.cache
def register_woq_linear_binary_fusions() -> None:
    for n in (4, 5):
        # (woq <inner> b1) <outer> b2 with the op's buffer order (b1, b2)
        for inner, outer, op_name in (("mul", "add", "zentorch_woq_linear_mul_add"),
                                      ("add", "add", "zentorch_woq_linear_add_add")):
            for inner_call in _either_order(_ATEN[inner], woq_call(n), KeywordArg("b1")):
                for pattern in _either_order(_ATEN[outer], inner_call, KeywordArg("b2")):
                    register_graph_pattern(
                        pattern, pass_dict=binary_binary_pass,
                        extra_check=_operands_match_output(("b1", "b2")),
                    )(_replacement(op_name, ("b1", "b2")))
        for pattern in _either_order(_ATEN["add"], woq_call(n), KeywordArg("b1")):
            register_graph_pattern(
                pattern, pass_dict=binary_pass,
                extra_check=_operands_match_output(("b1",)),
            )(_replacement("zentorch_woq_linear_add", ("b1",)))


def _apply(fx_graph: Graph, p: PatternMatcherPass, name: str) -> None:
    if config.pattern_matcher:
        assert fx_graph.owning_module is not None, "Graph has no owning module"
        torch.fx.passes.graph_transform_observer.GraphTransformObserver(
            fx_graph.owning_module, name, subsystem=name).apply_graph_pass(p.apply)
    stable_topological_sort(fx_graph)
    fx_graph.lint()


def woq_linear_binary_binary_post_op_fusions(fx_graph: Graph) -> Graph:
    """Apply the binary-binary fusions, then the single-add fusion."""
    register_woq_linear_binary_fusions()
    _apply(fx_graph, binary_binary_pass, "woq_linear_binary_binary_post_op_fusions")
    _apply(fx_graph, binary_pass, "woq_linear_binary_post_op_fusions")
    return fx_graph
