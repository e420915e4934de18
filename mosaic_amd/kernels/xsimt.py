"""A8 MXFP4 GEMV with the reference ``kernels/xsimt.py`` signatures."""
from __future__ import annotations

import torch

from .. import ops
from . import _a8, _prepack_cache
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


def prepack_expert_bank(packed_e: torch.Tensor, scale_e: torch.Tensor) -> ops.MXT16:
    """Stacked experts packed [E, N, K/2] + scale [E, N, K/32] -> one MXT16 bank, cached
    while the source tensors live and are unmodified (``kernels/xsimt.py:380-394``, whose
    cache is keyed on the tensor's id; the bank is one object here, not a codes/scales pair)."""
    if packed_e.dim() != 3 or scale_e.dim() != 3:
        raise ValueError("prepack_expert_bank expects [E, N, K/2] and [E, N, K/32]")
    return _prepack_cache.mxt16(packed_e, scale_e)


def decode_activation_exact(pair) -> torch.Tensor:
    """(x e4m3fn [M, K], unused scale) or x -> f16 [M, K], each code's exact value
    (``kernels/xsimt.py:96-113``; every e4m3 value is an fp16 value)."""
    x = pair[0] if isinstance(pair, tuple) else pair
    with _LAUNCHES.track():
        return ops.e4m3_decode(x).to(torch.float16)


def xsimt_gemm(x: torch.Tensor, packed: torch.Tensor, scale_w: torch.Tensor, n_out: int, backend: str = "native",
               prequant=None, prepacked=None) -> torch.Tensor:
    """x [M, K] bf16, packed [N, K/2], scale [N, K/32] -> [M, N] bf16, A8 (``kernels/xsimt.py:292-325``)."""
    if backend not in ("native", "triton"):
        raise ValueError(f"backend {backend}")
    with _LAUNCHES.track():
        return _a8.linear(x, packed, scale_w, n_out, prequant, prepacked)
