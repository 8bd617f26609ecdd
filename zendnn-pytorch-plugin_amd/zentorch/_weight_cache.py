"""Cache of repacked weights for compiled graphs.

A rewritten graph calls ``zentorch_woq_repack_weight(w)`` (or
``_repack_from_int4pack``) on a module buffer every forward; on the GPU the
repack reads twice the packed bytes, more than the linear itself.  The
reference avoids the same cost by reordering a constant weight once and
caching it inside ZenDNNL (``is_weights_const=true``,
src/cpu/cpp/WOQ_Linear.cpp:107).  Here a compiled graph calls
:func:`cached_repack` instead, which returns the packed tensor computed for
the same weight storage, view and version counter.  A repack checks the
weight's value range when it packs (a miss), so an in-place update that
leaves the int4 range raises instead of being truncated.

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


def _checked_int4(w: torch.Tensor, lo: int, hi: int, what: str) -> torch.Tensor:
    """``w`` after checking that every value lies in [lo, hi] (run on a cache
    miss only: when a weight is packed the first time or after it changed);
    a value outside would be truncated to its low nibble by the packing."""
    if w.numel() and not bool(((w >= lo) & (w <= hi)).all()):
        raise RuntimeError(
            f"zentorch: {what} holds values outside [{lo}, {hi}], which int4 packing "
            f"cannot represent; this graph was compiled for an int4 weight in that range")
    return w


def cached_repack_weight(w: torch.Tensor) -> torch.Tensor:
    return cached_repack(
        lambda t: torch.ops.zentorch.zentorch_woq_repack_weight(
            _checked_int4(t, -8, 15, "a weight packed by zentorch_woq_repack_weight")),
        "repack_weight", w)


def cached_repack_weight_offset(w: torch.Tensor, offset: int) -> torch.Tensor:
    """zentorch_woq_repack_weight(w + offset), packed once per weight version:
    the unsigned int4 packing u = w + offset of a signed int4 weight whose
    zero points are kept (the offset keeps u in [0, 15])."""
    return cached_repack(
        lambda t: torch.ops.zentorch.zentorch_woq_repack_weight(
            _checked_int4(t, -offset, 15 - offset, "an int4 weight with zero points") + offset),
        f"repack_weight+{offset}", w)


def cached_clone_offset(w: torch.Tensor, offset: int, *,
                        memory_format=torch.preserve_format) -> torch.Tensor:
    """w.clone() + offset once per version of w (the zero points zp + 8 that
    go with cached_repack_weight_offset)."""
    return cached_repack(lambda t: t.clone(memory_format=memory_format) + offset,
                         f"clone+{offset}:{memory_format}", w)


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
