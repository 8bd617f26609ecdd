"""zentorch for MI355X: zentorch's quantized-linear hot path on gfx950.

Importing the package loads the two in-tree native libraries
(libzentorch_hip.so: HIP kernels + C-ABI; _C.so: TORCH_LIBRARY(zentorch) +
AOTInductor shims) with RTLD_GLOBAL, as the reference loads libzentorch.so
(src/cpu/python/zentorch/__init__.py:69-78), then registers the Meta kernels
the ``"zentorch"`` torch.compile backend and the Inductor lowerings that
call the ops' AOTInductor shims.  A missing library is an
ImportError: there is no CPU fallback.
"""
import ctypes
import os

import torch

__version__ = "0.1.0"

_HERE = os.path.dirname(os.path.abspath(__file__))
HIP_LIBRARY = os.path.join(_HERE, "libzentorch_hip.so")
OPS_LIBRARY = os.path.join(_HERE, "_C.so")


def _load_native():
    for path in (HIP_LIBRARY, OPS_LIBRARY):
        if not os.path.exists(path):
            raise ImportError(
                f"zentorch: native library {path} is missing; build it with "
                "`python zendnn-pytorch-plugin_amd/build.py` (or "
                "__graft_entry__.build())")
    mode = os.RTLD_GLOBAL | os.RTLD_NOW
    hip = ctypes.CDLL(HIP_LIBRARY, mode=mode)
    ctypes.CDLL(OPS_LIBRARY, mode=mode)
    torch.ops.loaded_libraries.add(OPS_LIBRARY)
    return hip


_hip = _load_native()

from . import _meta_registrations  # noqa: E402,F401
from ._utils import counters  # noqa: E402,F401
from ._compile_backend import zentorch  # noqa: E402,F401
from . import _lowerings  # noqa: E402,F401


def native_libraries():
    """Paths of the native libraries this package loaded."""
    return [HIP_LIBRARY, OPS_LIBRARY]
