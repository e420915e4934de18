"""A8 MXFP4 GEMV with the reference ``kernels/xsimt.py`` signatures."""
from __future__ import annotations

import torch

from .. import ops
from . import _a8
from ._launches import LaunchCounter

_LAUNCHES = LaunchCounter()


def last_launch_count() -> int:
    """Kernel launches of this module's operators so far (``kernels/xsimt.py:31-32``)."""
    return _LAUNCHES.n


def prepack_xsimt(packed: torch.Tensor, scale: torch.Tensor) -> ops.MXT16:
    """Bit-exact invertible repack for the GEMV (``kernels/xsimt.py:39-53``): MXT16 tile order."""
    return ops.mxt16_prepack(packed, scale)


def inverse_prepack_xsimt(w: ops.MXT16, n: int | None = None, k: int | None = None):
    """Inverse of ``prepack_xsimt`` (``kernels/xsimt.py:56-63``)."""
    return ops.mxt16_unpack(w)


def xsimt_gemm(x: torch.Tensor, packed: torch.Tensor, scale_w: torch.Tensor, n_out: int, backend: str = "native",
               prequant=None, prepacked=None) -> torch.Tensor:
    """x [M, K] bf16, packed [N, K/2], scale [N, K/32] -> [M, N] bf16, A8 (``kernels/xsimt.py:292-325``)."""
    if backend not in ("native", "triton"):
        raise ValueError(f"backend {backend}")
    with _LAUNCHES.track():
        return _a8.linear(x, packed, scale_w, n_out, prequant, prepacked)
