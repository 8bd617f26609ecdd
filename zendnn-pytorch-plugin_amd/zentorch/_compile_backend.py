"""The ``"zentorch"`` torch.compile backend.

As in the reference (src/cpu/python/zentorch/_compile_backend.py:19-95) the
backend installs the zentorch graph passes as Inductor's
``joint_custom_post_pass`` and hands the FX graph to ``compile_fx``.  The
reference's CPU-only pre-passes (mkldnn conv fusion, :79-84) have no GPU
counterpart and are not run.
"""
import base64
from typing import Any, Callable, List

import torch
from torch._dynamo import register_backend
from torch._inductor import config
from torch._inductor.compile_fx import compile_fx
from torch._inductor.custom_graph_pass import CustomGraphPass, get_hash_for_files

from ._logging import get_logger
from ._optimize import optimize

logger = get_logger(__name__)


class OptimizePass(CustomGraphPass):
    def __call__(self, graph: torch.fx.Graph):
        optimize(graph)

    def uuid(self) -> Any:
        # Inductor's FX-graph cache keys on this: hash the pass sources.
        import os
        here = os.path.dirname(os.path.abspath(__file__))
        files = tuple(os.path.join(here, f) for f in (
            "_optimize.py", "_op_replacements_new.py",
            "_woq_linear_unary_fusion.py", "_woq_linear_binary_binary_fusion.py"))
        return base64.b64encode(get_hash_for_files(files)).decode()


optimize_pass = OptimizePass()


def zentorch_compile(gm: torch.fx.GraphModule, example_inputs: List[torch.Tensor]) -> Callable:
    logger.info("Called the zentorch backend.")
    config.joint_custom_post_pass = optimize_pass
    return compile_fx(gm, example_inputs)


@register_backend
def zentorch(model, inputs):
    return zentorch_compile(model, inputs)
