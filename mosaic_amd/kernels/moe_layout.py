"""Device-side MoE assignment layout (reference ``kernels/moe_layout.py``)."""
from __future__ import annotations

import torch

from .. import ops


def layout_assignments(expert_ids: torch.Tensor, n_experts: int):
    """expert_ids [A] -> (sorted_ids [A], perm [A] int64, offsets [E+1] int32, counts [E] int32)
    (``kernels/moe_layout.py:8-27``).  The order is STABLE: inside one expert,
    ascending flat assignment index (the reference's argsort leaves it open)."""
    if expert_ids.device.type != "cuda":
        raise ValueError("layout_assignments requires CUDA expert_ids")
    ids = expert_ids.reshape(-1, 1)
    out = ops.moe_layout(ids, None, n_experts, has_shared=False, block_m=16)
    return (out["sorted_ids"].to(torch.int64), out["perm"].to(torch.int64), out["offsets"], out["counts"])
