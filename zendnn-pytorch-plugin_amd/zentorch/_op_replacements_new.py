"""WOQ op replacement: dequantise-then-matmul subgraphs -> zentorch_woq_linear.

Matches the post-grad graphs the reference's pass matches
(src/cpu/python/zentorch/_op_replacements_new.py:316-799) and rewrites them
into ``repack -> transpose -> zentorch_woq_linear``:

* IntxWeightOnly per channel (:330-394 mm, :408-482 addmm)::

      mm(x, permute(mul(sub(bf16(w), bf16(zp)), scale), [1, 0]))

  with ``w`` int8 ``[N, K]`` and ``scale`` ``[N, 1]``; per group
  (:499-578 mm, :594-677 addmm) the product is viewed to ``[N, K]`` first,
  with ``w`` ``[N, G, gs]`` and ``scale`` ``[N, G, 1]``.  The reference
  drops the zero-point operand (:370,386), so a non-zero zero point would be
  computed as zero there.  Here the compile-time values decide: with every
  zero point 0 and the weight in [-8, 7] the operand is dropped (signed int4,
  as the reference) behind a run-time guard that the zero points stay zero;
  with integer zero points that are not all zero the rewrite keeps them and
  takes the unsigned int4 path of the op (``WOQ_Linear.cpp:44-49``): it packs
  ``u = w + 8`` and passes ``zp + 8``, so ``(u - zp') = (w - zp)`` and the op
  computes the graph's ``bf16((w - zp) * scale)``.
* Int4OpaqueTensor (:684-736 and +bias :746-799)::

      _weight_int4pack_mm_for_cpu(x, packed, groupsize, scale_and_zero)

  rewritten to ``repack_from_int4pack`` and a float zero point taken from
  ``scale_and_zero[..., 1]`` (tinygemm convention).

Differences from the reference, all narrowing what is rewritten: every
tensor operand must be on the GPU (the ops here have no CPU kernel; the
reference gates on AVX-512 instead, _optimize.py:87-91), the permute must
be the 2-D transpose, and the shapes the op would reject (K % 8 != 0,
scales of the wrong shape) leave the graph unchanged instead of failing at
run time.  Inductor may have turned the per-group ``view`` into
``reshape``; both are matched.
"""
import functools
from typing import Any, Callable, List, Optional

import torch
from torch._inductor import config
from torch._subclasses.fake_tensor import unset_fake_temporarily
from torch._inductor.pattern_matcher import (
    Arg,
    CallFunction,
    Match,
    PatternMatcherPass,
    register_graph_pattern,
    stable_topological_sort,
)
from torch.fx.graph import Graph

from ._utils import counters, on_gpu, placeholder_of, static_value, tensor_meta

aten = torch.ops.aten
prims = torch.ops.prims

pass_pattern = PatternMatcherPass(pass_name="zentorch_woq_replacement_pass")

# (zero-point placeholder, weight placeholder) pairs of the rewrites of the
# last pass that dropped all-zero zero points (signed int4 in [-8, 7])
ASSUMED_ZERO_ZP = []


# u4 packing of a signed int4 weight with integer zero points: u = w + U4_OFFSET
U4_OFFSET = 8


def _int4_kind(w_node, zp_node) -> Optional[str]:
    """What the compile-time values of the weight and zero points show:
    "symmetric" (every zero point 0, every weight value in [-8, 7]),
    "zero_points" (weight in [-8, 7], integer zero points not all zero whose
    offset by U4_OFFSET stays in the zero points' dtype), or None (leave the
    subgraph to PyTorch)."""
    zp, w = static_value(zp_node), static_value(w_node)
    if zp is None or w is None or placeholder_of(zp_node) is None or \
            placeholder_of(w_node) is None:
        return None
    # the passes run under the compile's fake mode; these are real tensors
    with unset_fake_temporarily():
        if not bool(((w >= -8) & (w <= 7)).all()):
            return None
        if not bool(zp.any()):
            return "symmetric"
        if zp.dtype not in (torch.int8, torch.int32):
            return None
        if int(zp.max()) > torch.iinfo(zp.dtype).max - U4_OFFSET:
            return None
        return "zero_points"


def _bf16(arg):
    return CallFunction(prims.convert_element_type.default, arg, torch.bfloat16)


def _dequant_transposed(view_op: Optional[Any]) -> CallFunction:
    """permute([view](mul(sub(bf16(w), bf16(zp)), scale), shape), dims).

    Arguments in match order: w, zp, scale, [shape], dims."""
    dq = CallFunction(aten.mul, CallFunction(aten.sub, _bf16(Arg()), _bf16(Arg())), Arg())
    if view_op is not None:
        dq = CallFunction(view_op, dq, Arg())
    return CallFunction(aten.permute, dq, Arg())


def _is_transpose(dims) -> bool:
    return isinstance(dims, (list, tuple)) and list(dims) == [1, 0]


def _dequant_check(has_bias: bool, per_group: bool) -> Callable[[Match], bool]:
    """Operand checks for the dequant patterns (match.args in pattern order)."""

    def check(match: Match) -> bool:
        args = list(match.args)
        bias = args.pop(0) if has_bias else None
        x, w, zp, scale = args[:4]
        shape = args[4] if per_group else None
        dims = args[-1]
        xv, wv, sv = tensor_meta(x), tensor_meta(w), tensor_meta(scale)
        if xv is None or wv is None or sv is None:
            return False
        if wv.dtype != torch.int8 or not _is_transpose(dims):
            return False
        if not on_gpu(xv, wv, sv):
            return False
        if per_group:
            if wv.dim() != 3 or sv.dim() != 3:
                return False
            N, G, gs = wv.shape
            if tuple(sv.shape) != (N, G, 1):
                return False
            if not isinstance(shape, (list, tuple)) or list(shape) != [N, G * gs]:
                return False
            K = G * gs
        else:
            if wv.dim() != 2 or sv.dim() != 2:
                return False
            N, K = wv.shape
            if tuple(sv.shape) != (N, 1):
                return False
        if K % 8 != 0 or xv.dim() != 2 or xv.shape[1] != K:
            return False
        if bias is not None:
            bv = tensor_meta(bias)
            if bv is None or bv.dim() != 1 or bv.shape[0] != N or not on_gpu(bv):
                return False
        zv = tensor_meta(zp)
        if zv is None or not on_gpu(zv) or zv.numel() != sv.numel():
            return False
        return _int4_kind(w, zp) is not None

    return check


def _register_dequant(matmul: Any, per_group: bool, view_op: Optional[Any]) -> None:
    has_bias = matmul is aten.addmm
    if has_bias:
        pattern = CallFunction(aten.addmm, Arg(), Arg(), _dequant_transposed(view_op))
    else:
        pattern = CallFunction(aten.mm, Arg(), _dequant_transposed(view_op))

    @register_graph_pattern(pattern, pass_dict=pass_pattern,
                            extra_check=_dequant_check(has_bias, per_group))
    def _replace(match: Match, *args: Any) -> None:
        w_node, zp_node = match.args[2:4] if has_bias else match.args[1:3]
        symmetric = _int4_kind(w_node, zp_node) == "symmetric"
        if symmetric:
            # recorded only for a rewrite that is applied
            ASSUMED_ZERO_ZP.append((placeholder_of(zp_node), placeholder_of(w_node)))

        def repl(*vals: Any) -> torch.Tensor:
            vals = list(vals)
            bias = vals.pop(0) if has_bias else None
            x, w, zp, scale = vals[:4]
            if per_group:
                w = w.reshape(vals[4])
            # [N, G(, 1)] scales and zero points -> [G, N]
            scales = scale.reshape(scale.shape[0], -1).transpose(0, 1).contiguous()
            if symmetric:
                # [N, K] int8 -> [N, K/8] int32 -> the op's [K/8, N] view
                packed = torch.ops.zentorch.zentorch_woq_repack_weight(w).transpose(0, 1)
                zeros = None
            else:
                # unsigned int4 u = w + 8 with zero points zp + 8
                packed = torch.ops.zentorch.zentorch_woq_repack_weight(
                    torch.ops.aten.add.Tensor(w, U4_OFFSET)).transpose(0, 1)
                zeros = torch.ops.aten.add.Tensor(
                    zp.reshape(zp.shape[0], -1).transpose(0, 1).contiguous(), U4_OFFSET)
            counters["zentorch"]["zentorch_woq_linear"] += 1
            return torch.ops.zentorch.zentorch_woq_linear(
                x, packed, scales, zeros, bias, zentorch_op_name="zentorch_woq_linear")

        match.replace_by_example(repl, list(args))


def _int4pack_check(bias_index: Optional[int]) -> Callable[[Match], bool]:
    def check(match: Match) -> bool:
        x, packed, _gs, sz = match.args[:4]
        xv, pv, szv = tensor_meta(x), tensor_meta(packed), tensor_meta(sz)
        if xv is None or pv is None or szv is None:
            return False
        if not on_gpu(xv, pv, szv) or pv.dtype != torch.uint8 or pv.dim() != 2:
            return False
        N = pv.shape[0]
        if N % 64 != 0 or szv.dim() != 3 or szv.shape[1] != N or szv.shape[2] != 2:
            return False
        if bias_index is not None:
            bv = tensor_meta(match.args[bias_index])
            if bv is None or bv.dim() != 1 or bv.shape[0] != N or not on_gpu(bv):
                return False
        return True

    return check


def _register_int4pack(with_bias: bool) -> None:
    mm = CallFunction(aten._weight_int4pack_mm_for_cpu, Arg(), Arg(), Arg(), Arg())
    pattern = CallFunction(aten.add.Tensor, mm, Arg()) if with_bias else mm

    @register_graph_pattern(pattern, pass_dict=pass_pattern,
                            extra_check=_int4pack_check(4 if with_bias else None))
    def _replace(match: Match, *args: Any) -> None:
        def repl(*vals: Any) -> torch.Tensor:
            x, packed, _groupsize, scale_and_zero = vals[:4]
            bias = vals[4] if with_bias else None
            repacked = torch.ops.zentorch.zentorch_woq_repack_from_int4pack(packed)
            scales = scale_and_zero.select(2, 0).contiguous()
            zeros = scale_and_zero.select(2, 1).contiguous()
            counters["zentorch"]["zentorch_woq_linear"] += 1
            return torch.ops.zentorch.zentorch_woq_linear(
                x, repacked.transpose(0, 1), scales, zeros, bias,
                zentorch_op_name="zentorch_woq_linear")

        match.replace_by_example(repl, list(args))


@functools.cache
def _register_all() -> None:
    for matmul in (aten.mm, aten.addmm):
        _register_dequant(matmul, per_group=False, view_op=None)
        for view_op in (aten.view, aten.reshape):
            _register_dequant(matmul, per_group=True, view_op=view_op)
    _register_int4pack(with_bias=False)
    _register_int4pack(with_bias=True)


def replace_with_zentorch_ops_new(fx_graph: Graph) -> Graph:
    """Apply the WOQ replacement patterns to ``fx_graph`` in place; the
    zero-point placeholders its rewrites assumed zero are in
    ``ASSUMED_ZERO_ZP`` afterwards."""
    _register_all()
    ASSUMED_ZERO_ZP.clear()
    if config.pattern_matcher:
        assert fx_graph.owning_module is not None, "Graph has no owning module"
        torch.fx.passes.graph_transform_observer.GraphTransformObserver(
            fx_graph.owning_module, "zentorch_woq_replacement_pass",
            subsystem="replace_with_zentorch_ops_new",
        ).apply_graph_pass(pass_pattern.apply)
    stable_topological_sort(fx_graph)
    fx_graph.lint()
    return fx_graph
