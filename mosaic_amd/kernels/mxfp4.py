"""MXFP4 pack / dequant (reference ``kernels/mxfp4.py``).

``pack_mxfp4`` quantizes along the LAST dim in blocks of 32 with the reference
packer's FLOOR e8m0 recipe (``kernels/mxfp4.py:32-43,91-127``; the quack
``to_mxfp4`` it prefers is not importable, so the reference takes this path);
``quantize_mxfp4`` offers the benchmark spec's ceil recipe.  Low nibble = even index."""
from __future__ import annotations

import torch

from .. import ops

E2M1_LUT = (
    0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
    -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0,
)
MX_BLOCK = 32


def pack_mxfp4(w_bf16: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """w [R, C] -> packed uint8 [R, C/2], scale float8_e8m0fnu [R, C/32] (``kernels/mxfp4.py:91``)."""
    if w_bf16.dim() != 2:
        raise ValueError(f"pack_mxfp4 expects [K, N], got {tuple(w_bf16.shape)}")
    if w_bf16.shape[1] % MX_BLOCK != 0:
        raise ValueError(f"N={w_bf16.shape[1]} must be a multiple of MX_BLOCK={MX_BLOCK}")
    if w_bf16.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError(f"pack_mxfp4 expects bf16/fp16/fp32, got {w_bf16.dtype}")
    p, s = ops.mx_quantize(w_bf16, "floor")
    return p, s.view(torch.float8_e8m0fnu)


def quantize_mxfp4(w: torch.Tensor, recipe: str = "ceil") -> tuple[torch.Tensor, torch.Tensor]:
    """The benchmark spec's recipe (scale 2^ceil(log2(amax/6)), upstream fp4_quant_kernel) or 'floor'."""
    p, s = ops.mx_quantize(w, recipe)
    return p, s.view(torch.float8_e8m0fnu)


def dequant_mxfp4(packed: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """packed [R, C/2] uint8 + e8m0 [R, C/32] -> bf16 [R, C] (``kernels/mxfp4.py:130-160``)."""
    if packed.dtype != torch.uint8:
        raise ValueError(f"dequant_mxfp4 expects uint8 packed, got {packed.dtype}")
    r, ch = packed.shape
    if tuple(scale.shape) != (r, 2 * ch // MX_BLOCK):
        raise ValueError(f"scale shape {tuple(scale.shape)} != ({r}, {2 * ch // MX_BLOCK})")
    return ops.mx_dequant(packed, scale, torch.bfloat16)
