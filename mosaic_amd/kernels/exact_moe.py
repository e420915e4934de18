"""Exact-target MoE entry point (reference ``kernels/exact_moe.py``)."""
from __future__ import annotations

import os

from .mxint import fused_moe_mxint
from .qpa_mma import fused_moe_qpa

_FALSE = ("0", "false", "False", "no", "")


def exact_target() -> bool:
    """True unless ``MOSAICVM_EXACT_TARGET`` is explicitly disabled (``runtime/exact.py:19-21``)."""
    return os.environ.get("MOSAICVM_EXACT_TARGET", "1") not in _FALSE


def exact_moe(x, expert_ids, expert_weights, packed_gate_up, scale_gate_up, packed_down, scale_down):
    """A8 routed MoE; requires the exact target (``kernels/exact_moe.py:12-19``)."""
    if not exact_target():
        raise RuntimeError("exact_moe requires MOSAICVM_EXACT_TARGET=1")
    return fused_moe_qpa(x, expert_ids, expert_weights, packed_gate_up, scale_gate_up, packed_down, scale_down)


def exact_moe_mxint(x, expert_ids, expert_weights, packed_gate_up, scale_gate_up, packed_down, scale_down, bank=None):
    """A8 routed MoE through ``fused_moe_mxint``; requires the exact target
    (``kernels/exact_moe.py:22-31``)."""
    if not exact_target():
        raise RuntimeError("exact_moe_mxint requires MOSAICVM_EXACT_TARGET=1")
    return fused_moe_mxint(x, expert_ids, expert_weights, packed_gate_up, scale_gate_up, packed_down, scale_down,
                           bank=bank)
