"""A8 MXFP4 GEMV / MoE with the reference ``kernels/qpa_mma.py`` signatures."""
from __future__ import annotations

import torch

from .. import ops
from . import _a8
from ._launches import LaunchCounter
from .mxint import MXT16Bank, _fused_moe_a8, prepack_expert_bank_mxint

_LAUNCHES = LaunchCounter()


def last_launch_count() -> int:
    """Kernel launches since ``fused_moe_qpa`` last started (``kernels/qpa_mma.py:58-59,698``)."""
    return _LAUNCHES.n


def prepack_qpa(packed: torch.Tensor, scale: torch.Tensor, stage: str = "qpa_k32_fragment"):
    """Bit-exact invertible repack (``kernels/qpa_mma.py:90-126``): MXT16 tile order."""
    return ops.mxt16_prepack(packed, scale), stage


def inverse_prepack_qpa(tiles: ops.MXT16, n: int | None = None, k: int | None = None):
    """Inverse of ``prepack_qpa`` (``kernels/qpa_mma.py:129-150``)."""
    return ops.mxt16_unpack(tiles)


def qpa_mma_gemm(x, packed, scale_w, n_out, backend="native", qpa_k=1, prequant=None, prepacked=None,
                 prepack_stage="qpa_k32_fragment", x_norm=None, sA=None, ordered=True) -> torch.Tensor:
    """x [M, K] bf16, packed [N, K/2], scale [N, K/32] -> [M, N] bf16, A8 (``kernels/qpa_mma.py:498-541``).
    ``x_norm``/``sA`` (pre-decoded activations of the reference) are accepted as
    e4m3 codes + scales."""
    if x_norm is not None and sA is not None:
        prequant = (x_norm, sA)
    with _LAUNCHES.track():
        return _a8.linear(x, packed, scale_w, n_out, prequant, prepacked)


def prepack_expert_bank_qpa(packed_g, scale_g, packed_u=None, scale_u=None, packed_d=None, scale_d=None,
                            chunk: int = 32) -> MXT16Bank:
    """``kernels/qpa_mma.py:577-612``: the same MXT16 bank as the MXINT prepack."""
    return prepack_expert_bank_mxint(packed_g, scale_g, packed_u, scale_u, packed_d, scale_d, chunk)


def fused_moe_qpa(x, expert_ids, expert_weights, packed_gate_up=None, scale_gate_up=None, packed_down=None,
                  scale_down=None, bank: MXT16Bank | None = None, crossover: int = 3, qpa_k: int = 8,
                  xsimt_k: int = 4, swiglu_limit: float = 10.0) -> torch.Tensor:
    """A8 routed MoE (``kernels/qpa_mma.py:681-784``); same contract as ``fused_moe_mxint``."""
    _LAUNCHES.reset()
    with _LAUNCHES.track():
        return _fused_moe_a8(x, expert_ids, expert_weights, packed_gate_up, scale_gate_up, packed_down, scale_down,
                             bank, swiglu_limit, None)


def launch_census(fn) -> dict:
    """GPU kernel launches of one call of ``fn`` (``kernels/qpa_mma.py:833-856``), counted by
    the torch profiler: ``total_cuda_launches`` every kernel; ``custom_qpa_launches`` this
    build's kernels (the library's, which serve every A8 entry) other than routing/layout;
    ``layout_launches`` kernels whose name mentions emit, bincount, sort, route or layout;
    ``epilogue_launches`` the rest (torch's own).  ``custom_xsimt_launches`` and
    ``custom_mxint_launches`` are 0: there are no separate xsimt/mxint kernels.  When the
    profiler is unavailable: {"launch_census": "custom_only", "custom_launches": n} with n
    from the library's own launch counter."""
    from ._launches import LaunchCounter
    counter = LaunchCounter()
    try:
        with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CUDA]) as prof:
            fn()
            torch.cuda.synchronize()
        names = [e.name for e in prof.events() if e.device_type == torch.autograd.DeviceType.CUDA and e.name]
    except Exception:
        with counter.track():
            fn()
            torch.cuda.synchronize()
        return {"launch_census": "custom_only", "custom_launches": counter.n}
    low = [n.lower() for n in names]
    layout = sum(1 for n in low if any(t in n for t in ("emit", "bincount", "sort", "route", "layout")))
    custom = sum(1 for n, l in zip(names, low) if "mosaic::" in n and not any(
        t in l for t in ("emit", "bincount", "sort", "route", "layout")))
    total = len(names)
    return {"total_cuda_launches": total, "custom_qpa_launches": custom, "custom_xsimt_launches": 0,
            "custom_mxint_launches": 0, "layout_launches": layout,
            "epilogue_launches": max(0, total - custom - layout)}
