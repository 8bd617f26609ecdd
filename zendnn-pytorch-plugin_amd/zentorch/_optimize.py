"""Pass orchestrator for the quantized-linear hot path.

Order follows the reference's optimize() (src/cpu/python/zentorch/_optimize.py:80-160)
restricted to the WOQ passes: the WOQ op replacement (:104), the merged
gate_up SiLU-and-mul fusion (the WOQ form of the reference's split-mm
pattern, _fusion_patterns.py:72-109, applied there in the fusion passes),
then the binary-binary (:117) and unary (:118) post-op fusions.  The reference skips
all passes without AVX-512 (:87-91); here the gate is the graph's device: the
passes only rewrite subgraphs whose tensors live on the GPU.
"""
import torch

from . import _utils
from ._logging import get_logger
from ._op_replacements_new import ASSUMED_ZERO_ZP, replace_with_zentorch_ops_new
from ._woq_linear_binary_binary_fusion import woq_linear_binary_binary_post_op_fusions
from ._woq_linear_gate_up_fusion import woq_linear_gate_up_fusion
from ._woq_linear_unary_fusion import woq_linear_unary_post_op_fusions

logger = get_logger(__name__)


def zero_points_guard(zp: torch.Tensor, weight: torch.Tensor = None) -> None:
    """Raise if the zero points a compiled graph assumed zero are not, or if
    the int8 weight it packed as signed int4 left [-8, 7].  Each tensor is
    checked once per version (the version is remembered on the tensor object
    itself, so a new tensor is always checked), so a forward pays a device
    synchronisation only the first time and after an in-place update."""
    if getattr(zp, "_zentorch_zero_checked", None) != zp._version:
        if bool(zp.any()):
            raise RuntimeError(
                "zentorch: this graph was compiled for all-zero weight zero points "
                "(symmetric int4) and they have changed since; recompile the model")
        zp._zentorch_zero_checked = zp._version
    if weight is not None and getattr(weight, "_zentorch_int4_checked", None) != weight._version:
        if weight.numel() and not bool(((weight >= -8) & (weight <= 7)).all()):
            raise RuntimeError(
                "zentorch: this graph was compiled for a signed int4 weight in [-8, 7] and "
                "the weight has left that range since; recompile the model")
        weight._zentorch_int4_checked = weight._version


torch.fx.node._side_effectful_functions.add(zero_points_guard)


def _insert_zero_point_guards(fx_graph) -> None:
    placeholders = [n for n in fx_graph.nodes if n.op == "placeholder"]
    if not placeholders:
        return
    with fx_graph.inserting_after(placeholders[-1]):
        for zp, w in dict.fromkeys(ASSUMED_ZERO_ZP):
            fx_graph.call_function(zero_points_guard, (zp, w))


def optimize(fx_graph, static_values=None):
    """Run the WOQ passes on ``fx_graph`` in place.  ``static_values`` maps
    placeholder nodes to the real tensors they carry when known at compile
    time (module weights and buffers); the replacement reads zero points
    from it."""
    logger.info("Optimizing the fx_graph with zentorch ops.")
    _utils.STATIC_VALUES.clear()
    _utils.STATIC_VALUES.update(static_values or {})
    try:
        g = replace_with_zentorch_ops_new(fx_graph)
        _insert_zero_point_guards(g)
        g = woq_linear_gate_up_fusion(g)
        g = woq_linear_binary_binary_post_op_fusions(g)
        g = woq_linear_unary_post_op_fusions(g)
    finally:
        _utils.STATIC_VALUES.clear()
    return g
