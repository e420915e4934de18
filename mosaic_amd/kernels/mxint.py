"""A8 MXFP4 GEMV and the fused MoE with the reference ``kernels/mxint.py`` signatures.

The reference's integer-exact limb arithmetic (qA split into three s8 limbs on
dp4a / mma.s8) has no counterpart here: gfx950's scaled MFMA consumes the e4m3
activations and E2M1 weights directly with both power-of-two scales, so the
banks are simply MXT16-prepacked MXFP4 (``weight_repr`` is accepted and
ignored)."""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .. import ops
from . import _a8, _prepack_cache
from ._launches import LaunchCounter

_LAUNCHES = LaunchCounter()


def last_launch_count() -> int:
    """Kernel launches since ``fused_moe_mxint`` last started (``kernels/mxint.py:33-34,1460``)."""
    return _LAUNCHES.n


@dataclass
class MXT16Bank:
    """Prepacked expert bank: gate|up [E, 2I, H/2] and down [E, H, I/2] in MXT16."""
    gate_up: ops.MXT16
    down: ops.MXT16

    @property
    def n_out_gu(self) -> int:
        return self.gate_up.n

    @property
    def n_out_d(self) -> int:
        return self.down.n


def prepack_expert_bank_mxint(packed_g, scale_g, packed_u=None, scale_u=None, packed_d=None, scale_d=None,
                              chunk: int = 32) -> MXT16Bank:
    """NK packed expert tensors (gate|up concatenated, or gate and up separately)
    -> MXT16Bank (``kernels/mxint.py:165-206``)."""
    if packed_d is None or scale_d is None:
        raise TypeError("packed_d/scale_d are required")
    if packed_u is not None:
        packed_g = torch.cat([ops._u8(packed_g, "packed_g"), ops._u8(packed_u, "packed_u")], dim=1)
        scale_g = torch.cat([ops._u8(scale_g, "scale_g"), ops._u8(scale_u, "scale_u")], dim=1)
    return MXT16Bank(ops.mxt16_prepack(packed_g, scale_g), ops.mxt16_prepack(packed_d, scale_d))


prepack_expert_bank_mxint_packed4 = prepack_expert_bank_mxint


def mxint_dp4a_gemm(x, packed, scale_w, n_out, prequant=None, xint=None, prepacked=None,
                    weight_repr: str = "hot8") -> torch.Tensor:
    """x [M, K] bf16 -> [M, N] bf16, A8 (``kernels/mxint.py:362-401``)."""
    with _LAUNCHES.track():
        return _a8.linear(x, packed, scale_w, n_out, prequant, prepacked)


def mxint_imma_gemm(x, packed, scale_w, n_out, prequant=None, xint=None, qpa_k=8, ordered=True, prepacked=None,
                    weight_repr: str = "hot8") -> torch.Tensor:
    """x [M, K] bf16 -> [M, N] bf16, A8 (``kernels/mxint.py:1014-1054``)."""
    with _LAUNCHES.track():
        return _a8.linear(x, packed, scale_w, n_out, prequant, prepacked)


def fused_moe_mxint(x, expert_ids, expert_weights, packed_gate_up=None, scale_gate_up=None, packed_down=None,
                    scale_down=None, bank: MXT16Bank | None = None, crossover: int = 0, imma_k: int = 8,
                    swiglu_limit: float = 10.0, stage_times: dict | None = None, weight_repr: str = "hot8",
                    epilogue: str = "torch", gu_bank=None, down_bank=None, masked_bank=None) -> torch.Tensor:
    """A8 routed MoE -> [k_tok, H] bf16 (``kernels/mxint.py:1435-1739``).

    x [k_tok, H] bf16; expert_ids [k_tok, top_k] (or [k_tok]); expert_weights
    fp32 of the same shape (None = ones).  Weights come from ``bank`` (MXT16Bank)
    or raw NK tensors (their MXT16 prepack cached while the tensors live).
    Sync-free unless ``stage_times`` is given: then the stage boundaries are
    timed with HIP events and the call waits for them, as the reference does."""
    if weight_repr not in ("hot8", "packed4", "hybrid"):
        raise ValueError(f"weight_repr must be hot8|packed4|hybrid, got {weight_repr}")
    _LAUNCHES.reset()
    with _LAUNCHES.track():
        return _fused_moe_a8(x, expert_ids, expert_weights, packed_gate_up, scale_gate_up, packed_down, scale_down,
                             bank, swiglu_limit, stage_times)


def _fused_moe_a8(x, expert_ids, expert_weights, packed_gate_up, scale_gate_up, packed_down, scale_down,
                  bank: MXT16Bank | None, swiglu_limit: float, stage_times: dict | None) -> torch.Tensor:
    if bank is None:
        if packed_gate_up is None or packed_down is None:
            raise TypeError("fused_moe_mxint requires bank= or packed_gate_up/packed_down")
        bank = MXT16Bank(_prepack_cache.mxt16(packed_gate_up, scale_gate_up), _prepack_cache.mxt16(packed_down, scale_down))
    ids = expert_ids if expert_ids.dim() == 2 else expert_ids.reshape(-1, 1)
    k_tok, top_k = ids.shape
    w = (torch.ones(k_tok, top_k, dtype=torch.float32, device=x.device) if expert_weights is None
         else expert_weights.reshape(k_tok, top_k).to(torch.float32))
    se = ops.StageEvents(ops.MOE_A8_STAGES) if stage_times is not None else None
    y, _, _ = ops.moe_a8_forward(x, bank.gate_up, bank.down, ids=ids, weights=w, swiglu_limit=swiglu_limit,
                                 stage_events=se)
    if se is not None:  # the reference synchronizes to fill stage_times (kernels/mxint.py:1702-1714)
        t = se.times()
        stage_times.update(t)
        stage_times["decode_int_sec"] = 0.0  # no integer limb split on gfx950
        stage_times["swiglu_sec"] = 0.0      # fused into the gate/up kernels
    return y


def mxint_swiglu_quant_down(gu, w_a, inter: int, swiglu_limit: float):
    """gu [A, 2*inter] bf16 + route weights [A] -> (e4m3fn codes [A, inter], f32 scales
    [A, inter/128]): clamps, SiLU, route weight, bf16, 1x128 pow2 act_quant in one pass
    (``kernels/mxint.py:1387-1408``).  The reference returns the codes as three int8 limb
    planes for its dp4a GEMMs; the codes and scales here are the ``prequant=`` input of
    this module's GEMMs."""
    if gu.dim() != 2 or gu.shape[1] != 2 * inter or inter % 128 != 0 or swiglu_limit <= 0:
        raise ValueError("mxint_swiglu_quant_down requires [A,2*inter], inter%128==0, limit>0")
    with _LAUNCHES.track():
        return ops.swiglu_act_quant(gu, w_a, inter, swiglu_limit)


def mxint_routed_reduce(yd, slot_rows, order, h: int):
    """Packed-order down partials bf16 [A, h] -> bf16 [k_tok, h], each token's top_k
    partials summed in fp32 in ascending expert-id order (``kernels/mxint.py:1411-1429``)."""
    with _LAUNCHES.track():
        return ops.routed_reduce(yd, slot_rows, order, h)
