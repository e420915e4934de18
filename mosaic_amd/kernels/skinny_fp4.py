"""A16 MXFP4 linear and MoE on the reference's KN layout (``kernels/skinny_fp4.py``).

KN: packed uint8 [K, N/2] (low nibble = even n) with one e8m0 scale per 32
consecutive N at each k ([K, N/32]).  Both operators run the hand-written
KN kernel of ``csrc/mx_kn.hip`` (decode to exact bf16 in registers, LDS
transposing reads into the bf16 MFMA), keeping the reference's arithmetic:
``skinny_mxfp4_gemm`` is fp32-accumulated dequant-then-matmul to bf16;
``fused_moe_skinny`` runs its bf16 SwiGLU, weight-after-down and bf16
index-add combine."""
from __future__ import annotations

import torch

from .. import ops
from ._launches import LaunchCounter

_LAUNCHES = LaunchCounter()


def last_launch_count() -> int:
    """Kernel launches since ``fused_moe_skinny`` last started (``kernels/skinny_fp4.py:17-22``):
    each ``skinny_mxfp4_gemm`` adds its GEMM (plus a split-K sum when K is split)."""
    return _LAUNCHES.n


def skinny_mxfp4_gemm(x: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, n_out: int) -> torch.Tensor:
    """x [M, K] bf16, packed [K, N/2], scale [K, N/32] -> [M, N] bf16 (``kernels/skinny_fp4.py:113-144``)."""
    m, k = x.shape
    k_p, n_half = packed.shape
    n = n_half * 2
    if n != n_out:
        raise ValueError(f"n_out={n_out} != packed N={n}")
    if k_p != k:
        raise ValueError(f"packed K={k_p} != x K={k}")
    with _LAUNCHES.track():
        return ops.mx_kn_linear_a16(x, packed, scale)


def pack_gate_up_mxfp4(w_gate: torch.Tensor, w_up: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """KN gate [K, I] and up [K, I] -> one KN gate|up weight: the two concatenated along N,
    then ``pack_mxfp4`` -> packed [K, I] (2I nibbles) + e8m0 [K, 2I/32] (``kernels/skinny_fp4.py:231-234``);
    I % 32 == 0 keeps every 32-column scale block inside gate or up."""
    from .mxfp4 import pack_mxfp4
    if w_gate.dim() != 2 or tuple(w_gate.shape) != tuple(w_up.shape):
        raise ValueError(f"gate {tuple(w_gate.shape)} and up {tuple(w_up.shape)} must be equal [K, I]")
    return pack_mxfp4(torch.cat([w_gate, w_up], dim=1))


def _stack(t):
    if torch.is_tensor(t):
        return t if t.dim() == 3 else t.unsqueeze(0)
    return torch.stack(list(t), dim=0)


def fused_moe_skinny(x, expert_ids, expert_weights, packed_gate_up, scale_gate_up, packed_down, scale_down):
    """``kernels/skinny_fp4.py:267-322``: x [k_tok, H] bf16, expert_ids [k_tok, top_k]
    (or [k_tok]), expert_weights of the same shape (None = ones); KN banks
    packed_gate_up [E, H, 2I/2] + [E, H, 2I/32] (gate | up along N),
    packed_down [E, I, H/2] + [E, I, H/32] -> [k_tok, H] in x.dtype."""
    _LAUNCHES.reset()
    ids = expert_ids if expert_ids.dim() == 2 else expert_ids.reshape(-1, 1)
    w = (torch.ones(ids.shape, dtype=torch.float32, device=x.device) if expert_weights is None
         else expert_weights.reshape(ids.shape).to(torch.float32))
    with _LAUNCHES.track():
        y = ops.moe_skinny_forward(x.to(torch.bfloat16), ids, w, _stack(packed_gate_up), _stack(scale_gate_up),
                                   _stack(packed_down), _stack(scale_down))
    return y.to(x.dtype)
