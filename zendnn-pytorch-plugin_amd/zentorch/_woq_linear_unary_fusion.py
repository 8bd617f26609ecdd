"""Fuse an activation that follows zentorch_woq_linear into the op.

GELU follows the reference (src/cpu/python/zentorch/_woq_linear_unary_fusion.py:142-261):
``aten.gelu(woq, approximate=...)`` and Inductor's decomposed erf/tanh GELU,
with or without the fp32 round trip Inductor inserts around it for bf16
(``bf16(gelu(fp32(woq)))``), become ``zentorch_woq_linear_gelu_erf`` /
``_gelu_tanh``.

Extensions (the reference registers the ops but no pass for them):

* ``silu(woq) * m`` and ``m * silu(woq)`` -> ``zentorch_woq_linear_silu_mul``
  (the gate half of a Llama MLP; silu in any of its decomposed forms);
* ``relu(woq)`` -> ``zentorch_woq_linear_relu``;
* ``sigmoid(woq)`` (also inside the bf16 fp32 round trip) ->
  ``zentorch_woq_linear_sigmoid``.

The woq_linear node is matched with 4 operands (no bias) or 5, keyword
operands (``zentorch_op_name``) are ignored.  Counter keys are
``zentorch_woq_linear_<post-op>``.
"""
import functools
from typing import Any, Callable, Dict, Optional

import torch
from torch._inductor import config
from torch._inductor.fx_passes.mkldnn_fusion import _gelu_fusion_1, _gelu_fusion_2
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

aten = torch.ops.aten
prims = torch.ops.prims

matcher_pass = PatternMatcherPass(pass_name="zentorch_woq_linear_unary_fusion_pass")

_OPERANDS = ("input", "weight", "weight_scales", "weight_zero_points", "bias")


def woq_call(n_operands: int, users: int = 1) -> CallFunction:
    """zentorch_woq_linear with its operands bound to keyword names."""
    return CallFunction(torch.ops.zentorch.zentorch_woq_linear.default,
                        *[KeywordArg(n) for n in _OPERANDS[:n_operands]], _users=users)


def _to(dtype, inner, users: int = 1) -> CallFunction:
    return CallFunction(prims.convert_element_type.default, inner, dtype, _users=users)


def _woq_node(match: Match):
    for n in match.nodes:
        if n.target is torch.ops.zentorch.zentorch_woq_linear.default:
            return n
    return None


def _woq_on_gpu(match: Match) -> bool:
    node = _woq_node(match)
    return node is not None and on_gpu(tensor_meta(node))


def _replace_with(op_name: str, extra: tuple = ()) -> Callable:
    """Handler that swaps the matched subgraph for zentorch.<op_name>(woq
    operands, *extra buffers, bias)."""

    def handler(match: Match, **kw: Any) -> None:
        names = [n for n in _OPERANDS if n in kw]
        buffers = [kw[e] for e in extra]

        def repl(*vals: Any) -> torch.Tensor:
            ops = dict(zip(names, vals[:len(names)]))
            bufs = list(vals[len(names):])
            counters["zentorch"][op_name] += 1
            return getattr(torch.ops.zentorch, op_name)(
                ops["input"], ops["weight"], ops["weight_scales"],
                ops["weight_zero_points"], *bufs, ops.get("bias"))

        match.replace_by_example(repl, [kw[n] for n in names] + buffers)

    return handler


def _register(pattern: CallFunction, op_name: str,
              check: Callable[[Match], bool], extra: tuple = ()) -> None:
    register_graph_pattern(pattern, pass_dict=matcher_pass, extra_check=check)(
        _replace_with(op_name, extra))


# ------------------------------------------------------------------ checks
def _gpu_only(match: Match) -> bool:
    return _woq_on_gpu(match)


def _gelu_approximate(approximate: str) -> Callable[[Match], bool]:
    """aten.gelu node whose ``approximate`` (keyword or second positional
    operand, default "none") is ``approximate``.  The pattern itself cannot
    tell: the matcher ignores node keywords a pattern does not name."""

    def check(match: Match) -> bool:
        if not _woq_on_gpu(match):
            return False
        node = match.output_node()
        got = node.kwargs.get("approximate", node.args[1] if len(node.args) > 1 else "none")
        return got == approximate

    return check


def _mul_operand_check(match: Match) -> bool:
    """The multiplier must have the output's shape and dtype (no broadcast,
    no type promotion), so the fused op returns what the graph returned."""
    if not _woq_on_gpu(match):
        return False
    m = tensor_meta(match.kwargs.get("mul_input"))
    out = tensor_meta(match.output_node())
    w = tensor_meta(_woq_node(match))
    return (m is not None and out is not None and w is not None and on_gpu(m)
            and tuple(m.shape) == tuple(out.shape) == tuple(w.shape)
            and m.dtype == out.dtype == w.dtype
            and m.dtype in (torch.bfloat16, torch.float32))


# ---------------------------------------------------------------- patterns
def _silu_forms(n: int):
    """silu(woq) as it can appear after Inductor's decompositions."""
    yield CallFunction(aten.silu, woq_call(n))
    c = woq_call(n, users=2)
    yield CallFunction(aten.mul, c, CallFunction(aten.sigmoid, c))
    c = _to(torch.float32, woq_call(n), users=2)
    yield _to(torch.bfloat16, CallFunction(aten.mul, c, CallFunction(aten.sigmoid, c)))


@functools.cache
def register_woq_linear_unary_fusions() -> None:
    for n in (4, 5):
        # GELU, not decomposed
        gelu = CallFunction(aten.gelu, woq_call(n))
        _register(gelu, "zentorch_woq_linear_gelu_erf", _gelu_approximate("none"))
        _register(gelu, "zentorch_woq_linear_gelu_tanh", _gelu_approximate("tanh"))
        # GELU, decomposed: erf form uses the output twice, tanh form four times
        for op_name, form, users in (("zentorch_woq_linear_gelu_erf", _gelu_fusion_1, 2),
                                     ("zentorch_woq_linear_gelu_tanh", _gelu_fusion_2, 4)):
            _register(form(woq_call(n, users)), op_name, _gpu_only)
            _register(_to(torch.bfloat16, form(_to(torch.float32, woq_call(n), users))),
                      op_name, _gpu_only)
        # relu / sigmoid
        _register(CallFunction(aten.relu, woq_call(n)), "zentorch_woq_linear_relu",
                  _gpu_only)
        _register(CallFunction(aten.sigmoid, woq_call(n)), "zentorch_woq_linear_sigmoid",
                  _gpu_only)
        _register(_to(torch.bfloat16, CallFunction(aten.sigmoid, _to(torch.float32, woq_call(n)))),
                  "zentorch_woq_linear_sigmoid", _gpu_only)
        # silu(woq) * m, either operand order
        for silu in _silu_forms(n):
            for pattern in (CallFunction(aten.mul, silu, KeywordArg("mul_input")),
                            CallFunction(aten.mul, KeywordArg("mul_input"), silu)):
                _register(pattern, "zentorch_woq_linear_silu_mul", _mul_operand_check,
                          extra=("mul_input",))


def woq_linear_unary_post_op_fusions(fx_graph: Graph) -> Graph:
    """Apply the WOQ unary fusions to ``fx_graph`` in place."""
    register_woq_linear_unary_fusions()
    if config.pattern_matcher:
        assert fx_graph.owning_module is not None, "Graph has no owning module"
        torch.fx.passes.graph_transform_observer.GraphTransformObserver(
            fx_graph.owning_module, "zentorch_woq_linear_unary_fusion_pass",
            subsystem="woq_linear_unary_post_op_fusions",
        ).apply_graph_pass(matcher_pass.apply)
    stable_topological_sort(fx_graph)
    fx_graph.lint()
    return fx_graph
