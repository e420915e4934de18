"""Shared plumbing of the A8 drop-ins: activation prequant and weight prepack."""
from __future__ import annotations

import torch

from .. import ops
from . import _prepack_cache


def prequant(x: torch.Tensor | None, prequant) -> tuple[torch.Tensor, torch.Tensor]:
    """(e4m3 codes, fp32 pow2 scales) from ``prequant`` or act_quant_ref(x)
    (``kernels/xsimt.py:284-289``)."""
    if prequant is not None:
        x_fp8, sa = prequant
        return ops._u8(x_fp8, "x_fp8"), ops._cuda(sa, "sA").to(torch.float32).contiguous()
    return ops.act_quant(x, 128, "pow2")


def weight(packed: torch.Tensor, scale_w: torch.Tensor, prepacked) -> ops.MXT16:
    if prepacked is not None:
        if not isinstance(prepacked, ops.MXT16):
            raise TypeError("prepacked must be an MXT16 weight (mosaic_amd.ops.mxt16_prepack)")
        return prepacked
    return _prepack_cache.mxt16(packed, scale_w)


def linear(x, packed, scale_w, n_out, prequant_=None, prepacked=None) -> torch.Tensor:
    """x [M, K] bf16, packed [N, K/2], scale [N, K/32] -> [M, N] bf16 (A8)."""
    n = packed.shape[0] if prepacked is None else prepacked.n
    if n != n_out:
        raise ValueError(f"n_out={n_out} != packed N={n}")
    xq, sa = prequant(x, prequant_)
    return ops.mxt16_linear_a8(None, weight(packed, scale_w, prepacked), prequant=(xq, sa))
