"""Pass orchestrator for the quantized-linear hot path.

Order follows the reference's optimize() (src/cpu/python/zentorch/_optimize.py:80-160)
restricted to the WOQ passes: the WOQ op replacement (:104), then the
binary-binary (:117) and unary (:118) post-op fusions.  The reference skips
all passes without AVX-512 (:87-91); here the gate is the graph's device: the
passes only rewrite subgraphs whose tensors live on the GPU.
"""
from ._logging import get_logger
from ._op_replacements_new import replace_with_zentorch_ops_new
from ._woq_linear_binary_binary_fusion import woq_linear_binary_binary_post_op_fusions
from ._woq_linear_unary_fusion import woq_linear_unary_post_op_fusions

logger = get_logger(__name__)


def optimize(fx_graph):
    logger.info("Optimizing the fx_graph with zentorch ops.")
    g = replace_with_zentorch_ops_new(fx_graph)
    g = woq_linear_binary_binary_post_op_fusions(g)
    g = woq_linear_unary_post_op_fusions(g)
    return g
