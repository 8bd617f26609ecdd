"""Replacement counters shared by the graph passes and the tests.

``counters["zentorch"][op]`` is incremented once per replaced node, as in the
reference (src/cpu/python/zentorch/_utils.py:23; incremented e.g. at
_op_replacements_new.py:381).  ZENTORCH_DUMP_COUNTERS=1 writes them to a JSON
file at exit (_utils.py:114-134).
"""
import atexit
import json
import os
from collections import Counter, defaultdict

counters = defaultdict(Counter)


def _dump_counters():
    if os.environ.get("ZENTORCH_DUMP_COUNTERS", "0") != "1":
        return
    path = os.environ.get("ZENTORCH_COUNTERS_FILE", f"zentorch_counters_{os.getpid()}.json")
    with open(path, "w") as f:
        json.dump({k: dict(v) for k, v in counters.items()}, f, indent=2)


atexit.register(_dump_counters)


def tensor_meta(node):
    """The example value (FakeTensor) an FX node carries, or None."""
    import torch

    if not isinstance(node, torch.fx.Node):
        return None
    val = node.meta.get("val", None)
    return val if isinstance(val, torch.Tensor) else None


# Device types the graph passes rewrite for.  The ops have kernels for the
# GPU only, so a subgraph on any other device is left to stock torch.
PASS_DEVICE_TYPES = ("cuda",)


def on_gpu(*vals):
    """True if every example tensor lives on a device the ops run on."""
    return all(v is not None and v.device.type in PASS_DEVICE_TYPES for v in vals)


# Real values of graph inputs known at compile time (module weights and
# buffers), keyed by placeholder node; set by optimize() for the duration of
# the passes.  A pass that needs a value it cannot see leaves its subgraph
# alone.
STATIC_VALUES = {}


def static_value(node):
    """The real tensor behind ``node`` (a placeholder, possibly through
    views), or None when it is not known at compile time."""
    import torch

    view_ops = (torch.ops.aten.view.default, torch.ops.aten.reshape.default,
                torch.ops.aten._unsafe_view.default)
    while isinstance(node, torch.fx.Node) and node.op == "call_function" \
            and node.target in view_ops:
        node = node.args[0]
    if not isinstance(node, torch.fx.Node) or node.op != "placeholder":
        return None
    return STATIC_VALUES.get(node)


def placeholder_of(node):
    """The placeholder ``node`` is a view chain of, or None."""
    import torch

    view_ops = (torch.ops.aten.view.default, torch.ops.aten.reshape.default,
                torch.ops.aten._unsafe_view.default)
    while isinstance(node, torch.fx.Node) and node.op == "call_function" \
            and node.target in view_ops:
        node = node.args[0]
    return node if isinstance(node, torch.fx.Node) and node.op == "placeholder" else None
