"""Fuse a merged gate_up WOQ linear and its SiLU-and-mul into one op.

The reference fuses the bf16 form of this MLP head: a view -> mm -> view ->
split -> silu / mul chain becomes mm + mm_silu_mul on the two halves of the
weight (``_split_mm_pattern``, src/cpu/python/zentorch/_fusion_patterns.py:
72-109).  Here the weight-only-quantised form is rewritten: a
``zentorch_woq_linear`` whose [*, 2I] output is split into halves along the
last dimension, followed by ``silu(gate) * up`` (vLLM's merged gate_up +
SiluAndMul), becomes one ``zentorch_woq_linear_gate_up_silu_mul`` call,
which runs the whole [2I, K] weight in one kernel launch with the silu·mul
epilogue.  The fused op rounds ``up`` to the output dtype before the
product, as the unfused graph does.

Matched forms, after Inductor's decompositions:

* the woq output, optionally ``view``-ed (the 3-D [bs, sl, 2I] form);
* the split as ``aten.split.Tensor(h, I, -1)`` / ``split_with_sizes(h, [I, I],
  -1)`` with ``getitem`` 0 and 1, or as two ``aten.slice.Tensor`` over
  [0, I) and [I, 2I) of the last dimension;
* ``silu(gate)`` as ``aten.silu``, ``gate * sigmoid(gate)`` or that inside
  the bf16 -> fp32 -> bf16 round trip;
* ``silu * up`` in either operand order.

Every intermediate node must have no other user, the tensors must be on the
GPU with bf16 / fp32 outputs of one dtype, and the product must have the
half's shape (no broadcasting).  Counter key:
``zentorch_woq_linear_gate_up_silu_mul``.
"""
import operator
from typing import List, Optional

import torch
from torch.fx.graph import Graph

from ._utils import counters, on_gpu, tensor_meta

aten = torch.ops.aten
prims = torch.ops.prims
_WOQ = torch.ops.zentorch.zentorch_woq_linear.default
_GATE_UP = torch.ops.zentorch.zentorch_woq_linear_gate_up_silu_mul.default
_BIG = 2 ** 62


def _only_user(node: torch.fx.Node) -> Optional[torch.fx.Node]:
    users = list(node.users)
    return users[0] if len(users) == 1 else None


def _last_dim(node: torch.fx.Node, dim) -> bool:
    v = tensor_meta(node)
    return v is not None and isinstance(dim, int) and dim in (-1, v.dim() - 1)


def _halves(h: torch.fx.Node, I: int):
    """(gate, up, split nodes) when h's users split it into [0, I) and
    [I, 2I) along the last dimension, else None."""
    users = list(h.users)
    if len(users) == 1 and users[0].op == "call_function":
        sp = users[0]
        ok = False
        if sp.target is aten.split.Tensor and len(sp.args) >= 2:
            ok = sp.args[1] == I and _last_dim(h, sp.args[2] if len(sp.args) > 2 else
                                               sp.kwargs.get("dim", 0))
        elif sp.target is aten.split_with_sizes.default and len(sp.args) >= 2:
            ok = list(sp.args[1]) == [I, I] and _last_dim(h, sp.args[2] if len(sp.args) > 2 else
                                                           sp.kwargs.get("dim", 0))
        if not ok:
            return None
        gets = {}
        for u in sp.users:
            if u.target is not operator.getitem or u.args[1] not in (0, 1) or u.args[1] in gets:
                return None
            gets[u.args[1]] = u
        if set(gets) != {0, 1}:
            return None
        return gets[0], gets[1], [sp]
    if len(users) == 2 and all(u.target is aten.slice.Tensor for u in users):
        gate = up = None
        for u in users:
            dim = u.args[1] if len(u.args) > 1 else 0
            start = u.args[2] if len(u.args) > 2 else 0
            end = u.args[3] if len(u.args) > 3 else _BIG
            step = u.args[4] if len(u.args) > 4 else 1
            if not _last_dim(h, dim) or step != 1:
                return None
            if start == 0 and end == I:
                gate = u
            elif start == I and isinstance(end, int) and end >= 2 * I:
                up = u
        if gate is None or up is None:
            return None
        return gate, up, []
    return None


def _convert(node, dtype) -> bool:
    return (isinstance(node, torch.fx.Node) and node.target is prims.convert_element_type.default
            and node.args[1] == dtype)


def _silu_of(gate: torch.fx.Node):
    """(silu output node, its internal nodes) when gate's users compute
    silu(gate) and nothing else, else None."""
    users = list(gate.users)
    if len(users) == 1 and users[0].target is aten.silu.default:
        return users[0], []
    src, inner = gate, []
    if len(users) == 1 and _convert(users[0], torch.float32):
        src = users[0]
        inner.append(src)
        users = list(src.users)
    # src * sigmoid(src): users are the sigmoid and the mul
    if len(users) != 2:
        return None
    sig = next((u for u in users if u.target is aten.sigmoid.default), None)
    mul = next((u for u in users if u.target is aten.mul.Tensor), None)
    if sig is None or mul is None or _only_user(sig) is not mul or set(mul.args) != {src, sig}:
        return None
    inner += [sig]
    if src is not gate:  # back to bf16
        out = _only_user(mul)
        if out is None or not _convert(out, torch.bfloat16):
            return None
        return out, inner + [mul]
    return mul, inner


def _fuse_one(woq: torch.fx.Node, graph: Graph) -> bool:
    out = tensor_meta(woq)
    if out is None or out.dim() != 2 or not on_gpu(out) or out.shape[1] % 2:
        return False
    if out.dtype not in (torch.bfloat16, torch.float32):
        return False
    if any(v is not None and not isinstance(v, torch.fx.Node) for v in woq.args[4:5]):
        return False
    I = out.shape[1] // 2
    h, view = woq, None
    u = _only_user(woq)
    if u is not None and u.target in (aten.view.default, aten.reshape.default,
                                      aten._unsafe_view.default):
        h, view = u, u
    halves = _halves(h, I)
    if halves is None:
        return False
    gate, up, split_nodes = halves
    silu = _silu_of(gate)
    if silu is None:
        return False
    silu_out, silu_inner = silu
    prod = _only_user(silu_out)
    if prod is None or prod.target is not aten.mul.Tensor or set(prod.args) != {silu_out, up}:
        return False
    if list(up.users) != [prod]:
        return False
    pv, uv = tensor_meta(prod), tensor_meta(up)
    if pv is None or uv is None or tuple(pv.shape) != tuple(uv.shape) or pv.dtype != out.dtype:
        return False
    args = list(woq.args[:4]) + [woq.args[4] if len(woq.args) > 4 else woq.kwargs.get("bias")]
    with graph.inserting_before(prod):
        fused = graph.call_function(_GATE_UP, tuple(args),
                                    {"zentorch_op_name": "zentorch_woq_linear_gate_up_silu_mul"})
        fused.meta["val"] = torch.empty_like(pv.reshape(-1, I)) if pv.dim() != 2 else pv
        res = fused
        if view is not None:
            res = graph.call_function(aten.view.default, (fused, list(pv.shape)))
            res.meta["val"] = pv
    prod.replace_all_uses_with(res)
    dead: List[torch.fx.Node] = [prod, silu_out] + silu_inner + [gate, up] + split_nodes
    if view is not None:
        dead.append(view)
    dead.append(woq)
    for n in dead:
        if n in graph.nodes and not n.users:
            graph.erase_node(n)
    counters["zentorch"]["zentorch_woq_linear_gate_up_silu_mul"] += 1
    return True


def woq_linear_gate_up_fusion(fx_graph: Graph) -> Graph:
    """Apply the merged gate_up fusion to ``fx_graph`` in place."""
    for node in list(fx_graph.nodes):
        if node.op == "call_function" and node.target is _WOQ and node in fx_graph.nodes:
            _fuse_one(node, fx_graph)
    fx_graph.eliminate_dead_code()
    fx_graph.lint()
    return fx_graph
