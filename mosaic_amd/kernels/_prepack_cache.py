"""Prepacked-weight cache of the drop-ins that receive raw NK MXFP4 tensors.

The reference's GEMV drop-ins accept raw ``packed``/``scale`` tensors and a
``prepacked`` argument; a caller that passes only the raw tensors would
otherwise pay an MXT16 prepack (a full read and write of the weight) on every
call.  Entries are keyed by the tensors' identity: a weak reference to each
raw tensor (so a freed tensor whose memory is reused never matches) plus its
in-place version counter (so an in-place update re-prepacks).  No device data
is read back.
"""
from __future__ import annotations

import weakref
from collections import OrderedDict

import torch

from .. import ops

_MAX_ENTRIES = 64
_CACHE: "OrderedDict[tuple, tuple]" = OrderedDict()


def mxt16(packed: torch.Tensor, scale: torch.Tensor) -> ops.MXT16:
    """ops.mxt16_prepack(packed, scale), reused while both tensors are alive and unmodified."""
    key = (packed.data_ptr(), scale.data_ptr(), tuple(packed.shape), tuple(scale.shape), packed.device)
    hit = _CACHE.get(key)
    if hit is not None:
        pref, sref, pver, sver, w = hit
        if pref() is packed and sref() is scale and packed._version == pver and scale._version == sver:
            _CACHE.move_to_end(key)
            return w
    w = ops.mxt16_prepack(packed, scale)
    _CACHE[key] = (weakref.ref(packed), weakref.ref(scale), packed._version, scale._version, w)
    _CACHE.move_to_end(key)
    while len(_CACHE) > _MAX_ENTRIES:
        _CACHE.popitem(last=False)
    return w


def clear() -> None:
    _CACHE.clear()
