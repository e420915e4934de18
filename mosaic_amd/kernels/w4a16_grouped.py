"""Tile list for grouped expert GEMMs (reference ``kernels/w4a16_grouped.py:151-169``)."""
from __future__ import annotations

import torch

from .. import ops
from ._launches import LaunchCounter

BLOCK_M = 16
_LAUNCHES = LaunchCounter()


def last_launch_count() -> int:
    """Kernel launches of this module's operators so far (``kernels/w4a16_grouped.py:15-16``)."""
    return _LAUNCHES.n


def emit_tiles(counts: torch.Tensor, block_m: int = BLOCK_M, max_tiles: int | None = None):
    """counts [E] int32 -> (expert_index [Tcap], m_start [Tcap], n_tiles [1], tile_rows [Tcap]).
    No per-expert cap: the reference stops at MAX_TILES=32 per expert (``:55-60``)."""
    e = counts.numel()
    t_cap = int(max_tiles) if max_tiles is not None else max(e, 1)
    with _LAUNCHES.track():
        ei, ms, nt, rows = ops.emit_tiles(counts, block_m, t_cap)
    return ei, ms, nt, rows
