"""Cache of repacked weights for compiled graphs.

A rewritten graph calls ``zentorch_woq_repack_weight(w)`` (or
``_repack_from_int4pack``) on a module buffer every forward; on the GPU the
repack reads twice the packed bytes, more than the linear itself.  The
reference avoids the same cost by reordering a constant weight once and
caching it inside ZenDNNL (``is_weights_const=true``,
src/cpu/cpp/WOQ_Linear.cpp:107).  Here a compiled graph calls
:func:`cached_repack` instead, which returns the packed tensor computed for
the same weight storage, view and version counter.

The entry holds a reference to the source weight, so its storage (and
address) cannot be reused by another tensor while the entry exists; an
in-place update of the weight bumps its version counter and the next call
repacks.  :func:`clear_weight_cache` drops every entry.
"""
import threading
from typing import Callable, Dict, Tuple

import torch

_lock = threading.Lock()
_entries: Dict[Tuple, Tuple[torch.Tensor, int, torch.Tensor]] = {}


def _key(op_name: str, w: torch.Tensor) -> Tuple:
    return (op_name, w.device, w.dtype, w.data_ptr(), tuple(w.shape), tuple(w.stride()))


def cached_repack(op: Callable[[torch.Tensor], torch.Tensor], op_name: str,
                  w: torch.Tensor) -> torch.Tensor:
    key = _key(op_name, w)
    with _lock:
        hit = _entries.get(key)
        if hit is not None and hit[1] == w._version:
            return hit[2]
    out = op(w)
    with _lock:
        _entries[key] = (w, w._version, out)
    return out


def cached_repack_weight(w: torch.Tensor) -> torch.Tensor:
    return cached_repack(torch.ops.zentorch.zentorch_woq_repack_weight, "repack_weight", w)


def cached_repack_from_int4pack(w: torch.Tensor) -> torch.Tensor:
    return cached_repack(torch.ops.zentorch.zentorch_woq_repack_from_int4pack,
                         "repack_from_int4pack", w)


def cached_clone(w: torch.Tensor, *, memory_format=torch.preserve_format) -> torch.Tensor:
    return cached_repack(lambda t: t.clone(memory_format=memory_format),
                         f"clone:{memory_format}", w)


def clear_weight_cache() -> None:
    with _lock:
        _entries.clear()


def cache_size() -> int:
    with _lock:
        return len(_entries)
