"""A16 MXFP4 linear on the reference's KN layout (``kernels/skinny_fp4.py``).

The KN layout blocks the e8m0 scales along N, so it cannot be re-blocked into
the NK tiles without requantizing; this compatibility path dequantizes the KN
weight exactly on the GPU and runs the library GEMM with fp32 accumulation
(dequant-then-matmul, the contract of ``tests/test_skinny_fp4.py:16-25``).
The NK path (``mosaic_amd.ops.mx_linear_a16`` / ``mxt16_linear_a16``) is the
hand-written kernel."""
from __future__ import annotations

import torch

from .. import ops


def last_launch_count() -> int:
    return 2


def skinny_mxfp4_gemm(x: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, n_out: int) -> torch.Tensor:
    """x [M, K] bf16, packed [K, N/2], scale [K, N/32] -> [M, N] bf16 (``kernels/skinny_fp4.py:113-144``)."""
    m, k = x.shape
    k_p, n_half = packed.shape
    n = n_half * 2
    if n != n_out:
        raise ValueError(f"n_out={n_out} != packed N={n}")
    if k_p != k:
        raise ValueError(f"packed K={k_p} != x K={k}")
    w = ops.mx_dequant(packed, scale, torch.bfloat16)  # [K, N], exact
    return torch.matmul(ops._bf16(x, "x"), w)
