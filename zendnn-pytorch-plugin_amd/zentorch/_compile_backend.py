"""The ``"zentorch"`` torch.compile backend.

The reference's backend (src/cpu/python/zentorch/_compile_backend.py:19-95)
installs the zentorch graph passes as Inductor's ``joint_custom_post_pass``
and compiles the rest of the graph with Inductor's CPU code generation.  On
MI355X the hot ops are the hand-written HIP kernels, so this backend keeps
Inductor's front half and drops its code generation:

1. AOT autograd traces the dynamo graph to aten ops with Inductor's
   decomposition table (the graph form the reference's patterns are written
   against: ``prims.convert_element_type``, decomposed GELU/SiLU, ...);
2. the WOQ replacement and fusion passes rewrite it (``optimize``);
3. repacks (and the scale copies) of module parameters and buffers go
   through the packed-weight cache (``_weight_cache``), so a forward
   repacks a weight only when it changed;
4. the rewritten graph runs op by op: the zentorch ops on their HIP
   kernels, everything else on PyTorch's own kernels.  No Triton code is
   generated.  Launch-bound callers capture the compiled forward in a HIP
   graph (``torch.cuda.CUDAGraph``).

The passes only rewrite GPU subgraphs; a CPU graph runs unchanged.
"""
from typing import Any, Callable, List

import torch
from torch._dynamo import register_backend
from torch._functorch.aot_autograd import aot_module_simplified, make_boxed_func
from torch._inductor.decomposition import select_decomp_table

from ._logging import get_logger
from ._optimize import optimize
from ._weight_cache import (cached_clone, cached_clone_offset, cached_repack_from_int4pack,
                            cached_repack_weight, cached_repack_weight_offset)

logger = get_logger(__name__)

_CACHED = {
    torch.ops.zentorch.zentorch_woq_repack_weight.default: cached_repack_weight,
    torch.ops.zentorch.zentorch_woq_repack_from_int4pack.default: cached_repack_from_int4pack,
    # the [G, N] scale / zero-point copies the replacement makes
    torch.ops.aten.clone.default: cached_clone,
}

# aten ops that return a view of their first operand without copying
_VIEW_OPS = {
    torch.ops.aten.view.default, torch.ops.aten._unsafe_view.default,
    torch.ops.aten.permute.default, torch.ops.aten.t.default,
    torch.ops.aten.transpose.int, torch.ops.aten.alias.default,
    torch.ops.aten.select.int, torch.ops.aten.slice.Tensor,
}


def _weight_placeholders(graph: torch.fx.Graph) -> set:
    """Placeholders that carry module parameters or buffers: AOT autograd
    marks them static (the same tensors on every call)."""
    ctx = torch._guards.TracingContext.try_get()
    idx = getattr(getattr(ctx, "fw_metadata", None), "static_input_indices", None) or []
    ph = [n for n in graph.nodes if n.op == "placeholder"]
    return {ph[i] for i in idx if i < len(ph)}


def _from_weight(node: torch.fx.Node, weights: set) -> bool:
    """True if ``node`` is a weight placeholder or a view chain of one."""
    while node.op == "call_function" and node.target in _VIEW_OPS:
        node = node.args[0]
    return node in weights


def _only_feeds_zentorch_ops(node: torch.fx.Node) -> bool:
    """True if every use of ``node`` (through views) is an operand of a
    zentorch op, so a cached tensor never leaves the graph where a caller
    could modify it."""
    for user in node.users:
        if user.op == "call_function" and user.target in _VIEW_OPS:
            if not _only_feeds_zentorch_ops(user):
                return False
        elif not (user.op == "call_function"
                  and getattr(user.target, "namespace", None) == "zentorch"):
            return False
    return True


_ADD_OPS = {torch.ops.aten.add.Tensor, torch.ops.aten.add.Scalar}


def _const_offset(node) -> "int | None":
    """The integer c when ``node`` is add(v, c) with a Python int c (alpha 1)."""
    if not (isinstance(node, torch.fx.Node) and node.op == "call_function"
            and node.target in _ADD_OPS and len(node.args) == 2 and not node.kwargs):
        return None
    c = node.args[1]
    return c if isinstance(c, int) and not isinstance(c, bool) else None


def use_weight_cache(graph: torch.fx.Graph, weights: set) -> int:
    """Route repacks (and contiguous copies) of module weights through the
    packed-weight cache, including the offset forms the WOQ replacement
    emits for weights with zero points: repack(add(w, c)) and
    add(clone(zero points), c).  Other inputs change from call to call and
    are never cached."""
    n = 0
    repack = torch.ops.zentorch.zentorch_woq_repack_weight.default
    for node in graph.nodes:
        if node.op != "call_function":
            continue
        if node.target in _CACHED and _from_weight(node.args[0], weights) \
                and _only_feeds_zentorch_ops(node):
            node.target = _CACHED[node.target]
            n += 1
        elif node.target is repack and _const_offset(node.args[0]) is not None \
                and _from_weight(node.args[0].args[0], weights) and _only_feeds_zentorch_ops(node):
            add = node.args[0]
            node.args = (add.args[0], _const_offset(add))
            node.target = cached_repack_weight_offset
            n += 1
        elif _const_offset(node) is not None and isinstance(node.args[0], torch.fx.Node) \
                and node.args[0].op == "call_function" \
                and node.args[0].target is torch.ops.aten.clone.default \
                and _from_weight(node.args[0].args[0], weights) and _only_feeds_zentorch_ops(node):
            clone, offset = node.args[0], _const_offset(node)
            node.target = cached_clone_offset
            node.kwargs = dict(clone.kwargs)
            node.args = (clone.args[0], offset)
            n += 1
    return n


def _static_values(graph: torch.fx.Graph, weights: set, real_inputs: List[Any]) -> dict:
    """Real tensors of the weight placeholders: the forward graph's
    placeholders are the flattened inputs dynamo handed the backend, in
    order (inference, no lifted parameters); matched only when every shape
    and dtype of the weight placeholders agrees.

    Only weight placeholders are compared, and only those whose sizes are
    plain ints: comparing a symbolic size (an activation's token count under
    ``dynamic=True`` or automatic dynamic shapes) with a real one would
    install a guard that specialises the graph to that count, so every new
    token count would recompile."""
    ph = [n for n in graph.nodes if n.op == "placeholder"]
    if len(ph) != len(real_inputs):
        return {}
    out = {}
    for node, real in zip(ph, real_inputs):
        if node not in weights:
            continue
        val = node.meta.get("val", None)
        if not isinstance(real, torch.Tensor) or not isinstance(val, torch.Tensor):
            continue
        shape = tuple(val.shape)
        if not all(type(d) is int for d in shape):
            continue
        if shape != tuple(real.shape) or val.dtype != real.dtype:
            return {}
        out[node] = real
    return out


def _compile_forward(gm: torch.fx.GraphModule, example_inputs: List[Any],
                     real_inputs: List[Any] = ()) -> Callable:
    weights = _weight_placeholders(gm.graph)
    static = _static_values(gm.graph, weights, list(real_inputs))
    if isinstance(real_inputs, list):
        real_inputs.clear()  # hold no references to the caller's inputs
    optimize(gm.graph, static)
    cached = use_weight_cache(gm.graph, weights)
    gm.graph.eliminate_dead_code()
    gm.recompile()
    logger.info("zentorch graph ready (%d cached weight transforms)", cached)
    return make_boxed_func(gm.forward)


def zentorch_compile(gm: torch.fx.GraphModule, example_inputs: List[torch.Tensor]) -> Callable:
    logger.info("Called the zentorch backend.")
    real_inputs = list(example_inputs)
    return aot_module_simplified(
        gm, example_inputs,
        fw_compiler=lambda g, ex: _compile_forward(g, ex, real_inputs),
        decompositions=select_decomp_table(), keep_inference_input_mutations=True)


@register_backend
def zentorch(model, inputs):
    return zentorch_compile(model, inputs)
