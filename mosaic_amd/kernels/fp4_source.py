"""Source-semantic FP4 layout helpers (reference ``kernels/fp4_source.py``).

Weights are NK: packed uint8 [N, K/2] + e8m0 [N, K/32]; activations use the
1x128 power-of-two act_quant; ``reference_fp4_linear_source_semantics`` is the
A8 linear, here run on the scaled MFMA."""
from __future__ import annotations

import torch

from .. import ops
from . import _prepack_cache
from .mxfp4 import MX_BLOCK

ACT_BLOCK = 128
ACT_FP8_MAX = 448.0


def pack_mxfp4_nk(w_nk: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """w [N, K] -> packed [N, K/2], e8m0 [N, K/32], FLOOR recipe (``kernels/fp4_source.py:35-64``)."""
    if w_nk.dim() != 2:
        raise ValueError(f"pack_mxfp4_nk expects [N, K], got {tuple(w_nk.shape)}")
    if w_nk.shape[1] % MX_BLOCK != 0:
        raise ValueError(f"K={w_nk.shape[1]} must be a multiple of MX_BLOCK={MX_BLOCK}")
    p, s = ops.mx_quantize(w_nk, "floor")
    return p, s.view(torch.float8_e8m0fnu)


def e8m0_to_fp32(scale: torch.Tensor) -> torch.Tensor:
    """e8m0 (or uint8) -> fp32 2^(b-127) by exponent insertion (``kernels/fp4_source.py:67-75``)."""
    b = ops._u8(scale, "scale")
    return (b.to(torch.int32) << 23).view(torch.float32)


def decode_e2m1_nk(packed: torch.Tensor) -> torch.Tensor:
    """packed [..., K/2] -> fp32 E2M1 values [..., K] without scale (``kernels/fp4_source.py:78-84``)."""
    p = ops._u8(packed, "packed")
    flat = p.reshape(-1, p.shape[-1])
    ones = torch.full((flat.shape[0], flat.shape[1] * 2 // MX_BLOCK), 127, dtype=torch.uint8, device=p.device)
    return ops.mx_dequant(flat, ones, torch.float32).reshape(*p.shape[:-1], p.shape[-1] * 2)


def decode_e4m3(x_fp8: torch.Tensor) -> torch.Tensor:
    """e4m3fn or uint8 -> fp32 (``kernels/fp4_source.py:87-91``)."""
    return ops.e4m3_decode(x_fp8)


def act_quant_ref(x: torch.Tensor, block: int = ACT_BLOCK) -> tuple[torch.Tensor, torch.Tensor]:
    """x [M, K] -> (e4m3fn [M, K], pow2 fp32 scale [M, K/block]) (``kernels/fp4_source.py:110-129``)."""
    if x.dim() != 2:
        raise ValueError(f"act_quant_ref expects [M, K], got {tuple(x.shape)}")
    if x.shape[1] % block != 0:
        raise ValueError(f"K={x.shape[1]} must be a multiple of act block {block}")
    return ops.act_quant(x, block, "pow2")


def act_quant_legacy_phase27(x: torch.Tensor, block: int = ACT_BLOCK) -> tuple[torch.Tensor, torch.Tensor]:
    """x [M, K] -> (e4m3fn [M, K], fp32 scale [M, K/block]) with s = amax/448, 1 for an
    all-zero block; kept for comparison with ``act_quant_ref`` (``kernels/fp4_source.py:94-107``)."""
    if x.dim() != 2:
        raise ValueError(f"act_quant_legacy_phase27 expects [M, K], got {tuple(x.shape)}")
    if x.shape[1] % block != 0:
        raise ValueError(f"K={x.shape[1]} must be a multiple of act block {block}")
    return ops.act_quant(x, block, "legacy")


def reference_fp4_linear_source_semantics(x_bf16: torch.Tensor, packed: torch.Tensor,
                                          scale_w: torch.Tensor) -> torch.Tensor:
    """A8 linear, x [M, K] -> [M, N] bf16 (``kernels/fp4_source.py:132-156``)."""
    m, k = x_bf16.shape
    n, kh = packed.shape
    if kh * 2 != k:
        raise ValueError(f"packed K {kh * 2} != x K {k}")
    return ops.mxt16_linear_a8(x_bf16, _prepack_cache.mxt16(packed, scale_w))
