"""Prepacked-weight cache of the drop-ins that receive raw NK MXFP4 tensors
(MXT16) or FP8 e4m3 weights at decode sizes (T16).

The reference's GEMV drop-ins accept raw ``packed``/``scale`` tensors and a
``prepacked`` argument; a caller that passes only the raw tensors would
otherwise pay a prepack (a full read and write of the weight) on every call.

An entry is keyed by the caller's source tensors: each one's data pointer,
shape, strides, dtype and device.  A hit also needs every source's storage
to be the same live storage object as when the entry was made (torch keeps
one Python object per live storage, shared by every view of it, dtype views
included), and its in-place version counter unchanged (views share it, so an
in-place update through any view re-prepacks).  A fresh ``.view()`` of the
same weight therefore hits, and a freed tensor whose memory is reused never
matches.  The entry is dropped as soon as any of its storages is freed, so the
prepacked copy lives exactly as long as the weight it was made from.  No
device data is read back.
"""
from __future__ import annotations

import weakref
from typing import Callable, Sequence

import torch

from .. import ops

_CACHE: "dict[tuple, tuple]" = {}


def _root(t: torch.Tensor):
    return t.untyped_storage()


def _key(srcs: Sequence[torch.Tensor]) -> tuple:
    return tuple((t.data_ptr(), tuple(t.shape), tuple(t.stride()), t.dtype, t.device) for t in srcs)


def cached(srcs: Sequence[torch.Tensor], make: Callable[[], object]):
    """``make()``, reused while every tensor of ``srcs`` is alive and unmodified."""
    key = _key(srcs)
    roots = [_root(t) for t in srcs]
    hit = _CACHE.get(key)
    if hit is not None:
        refs, versions, value = hit
        if all(r() is t for r, t in zip(refs, roots)) and versions == tuple(t._version for t in srcs):
            return value
        del _CACHE[key]
    value = make()

    def _drop(_ref, key=key):
        # only the entry made with these roots: a newer one under the same key has other refs
        entry = _CACHE.get(key)
        if entry is not None and any(r is _ref for r in entry[0]):
            del _CACHE[key]

    refs = tuple(weakref.ref(t, _drop) for t in roots)
    _CACHE[key] = (refs, tuple(t._version for t in srcs), value)
    return value


def mxt16(packed: torch.Tensor, scale: torch.Tensor) -> ops.MXT16:
    """ops.mxt16_prepack(packed, scale), reused while both tensors are alive and unmodified."""
    return cached((packed, scale), lambda: ops.mxt16_prepack(packed, scale))


def fp8_t16(b: torch.Tensor) -> ops.FP8T16:
    """ops.fp8_t16_prepack(b), reused while ``b`` is alive and unmodified."""
    return cached((b,), lambda: ops.fp8_t16_prepack(b))


def size() -> int:
    return len(_CACHE)


def clear() -> None:
    _CACHE.clear()
