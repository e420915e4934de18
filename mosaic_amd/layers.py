"""MoE layer entry points with the reference model's signatures, on the HIP kernels.

* ``Router`` -- ``model/layers.py:118-150``: fp32 router projection
  (``mosaic_router_logits``), sqrtsoftplus scores, ``e_score_correction_bias``
  for selection only, top-k with ties to the lower expert index, renormalized
  (sum clamped at 1e-9) and scaled by ``routed_scaling_factor``; returns
  (weights fp32 [M, k], ids int64 [M, k]).
* ``Gate`` -- ``.mosaicvm/source/inference_model.py:550-589``: the upstream gate
  (softmax | sigmoid | sqrtsoftplus, optional bias, renormalized unless
  softmax, times ``route_scale``); returns (weights, indices).  Hash layers
  (ids looked up from ``tid2eid``) raise: hash routing is not on this path.
* ``grouped_expert_forward`` -- ``model/layers.py:329-373``: the A16 routed
  expert sum (fp32 SwiGLU with the clamps, route weight before down, bf16 z,
  ascending-expert fp32 combine) over MXFP4 experts.

Scores are the fp32 rounding of the exact function of an fp32 logit, and each
logit is the exact dot product rounded once to fp32, so ids do not depend on
a summation order.  Nothing here synchronizes the host.
"""
from __future__ import annotations

import torch

from . import ops
from .kernels import _prepack_cache


def _exact_target() -> bool:
    from .kernels.exact_moe import exact_target
    return exact_target()


class Router(torch.nn.Module):
    """``model/layers.py:118-150``.  ``cfg`` needs ``n_routed_experts``,
    ``hidden_size``, ``scoring_func``, ``num_experts_per_tok``,
    ``norm_topk_prob`` and ``routed_scaling_factor`` (the reference's V4Config)."""

    def __init__(self, cfg, device=None):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.zeros(cfg.n_routed_experts, cfg.hidden_size, device=device))
        self.e_score_correction_bias = torch.nn.Parameter(torch.zeros(cfg.n_routed_experts, device=device))
        self.cfg = cfg

    def forward(self, x: torch.Tensor):
        cfg = self.cfg
        if cfg.scoring_func != "sqrtsoftplus":
            raise ValueError(f"unknown scoring_func {cfg.scoring_func}")
        if _exact_target():
            max_k = cfg.num_experts_per_tok
        else:
            if getattr(self, "aed", False):
                raise NotImplementedError("adaptive expert dropping (runtime/aed.py) is not part of this build")
            max_k = getattr(self, "active_k", None) or cfg.num_experts_per_tok
        logits = ops.router_logits(x.reshape(-1, x.shape[-1]), self.weight.detach())
        ids, w = ops.moe_route_topk(logits, max_k, "sqrtsoftplus", renorm=bool(cfg.norm_topk_prob),
                                    route_scale=float(cfg.routed_scaling_factor),
                                    bias=self.e_score_correction_bias.detach())
        return w, ids.to(torch.int64)


class Gate(torch.nn.Module):
    """``.mosaicvm/source/inference_model.py:550-589``.  ``args`` needs ``dim``,
    ``n_activated_experts``, ``score_func``, ``route_scale``, ``n_hash_layers``,
    ``n_routed_experts`` and ``vocab_size``."""

    def __init__(self, layer_id: int, args, device=None):
        super().__init__()
        self.dim = args.dim
        self.topk = args.n_activated_experts
        self.score_func = args.score_func
        self.route_scale = args.route_scale
        self.hash = layer_id < args.n_hash_layers
        self.weight = torch.nn.Parameter(torch.empty(args.n_routed_experts, args.dim, device=device))
        if self.hash:
            self.tid2eid = torch.nn.Parameter(
                torch.empty(args.vocab_size, args.n_activated_experts, dtype=torch.int32, device=device),
                requires_grad=False)
            self.bias = None
        else:
            self.bias = torch.nn.Parameter(torch.empty(args.n_routed_experts, dtype=torch.float32, device=device))

    def forward(self, x: torch.Tensor, input_ids: torch.Tensor | None = None):
        if self.hash:
            # hash routing (ids looked up from tid2eid by token id) is not on the quantized matrix path
            raise NotImplementedError("hash-routed Gate layers (layer_id < n_hash_layers) are not part of this build")
        logits = ops.router_logits(x.reshape(-1, x.shape[-1]), self.weight.detach())
        ids, w = ops.moe_route_topk(logits, self.topk, self.score_func, renorm=self.score_func != "softmax",
                                    route_scale=float(self.route_scale),
                                    bias=None if self.bias is None else self.bias.detach())
        return w, ids.to(torch.int64)


def _as_mxt16_bank(w, what: str) -> ops.MXT16:
    if isinstance(w, ops.MXT16):
        return w
    if isinstance(w, (tuple, list)) and len(w) == 2 and all(isinstance(t, torch.Tensor) for t in w) and \
            w[0].dtype in (torch.uint8, torch.int8) and w[0].dim() == 3:
        return _prepack_cache.mxt16(w[0], w[1])
    raise TypeError(f"{what}: expected an MXT16 bank or (packed [E, N, K/2] uint8, scale [E, N, K/32] e8m0) MXFP4 "
                    "experts in the checkpoint [out, in] layout; dense float expert weights are not run by this build")


def grouped_expert_forward(x: torch.Tensor, scores: torch.Tensor, idx: torch.Tensor, gate_up, down, n_experts: int,
                           swiglu_limit: float = 0.0) -> torch.Tensor:
    """``model/layers.py:329-373`` over MXFP4 experts.

    ``gate_up``: an MXT16 bank of [E, 2I, H/2] (gate rows then up rows), or
    ((packed_gate, scale_gate), (packed_up, scale_up)) with packed [E, I, H/2]
    and scale [E, I, H/32] in the checkpoint's [out, in] layout; ``down``: an
    MXT16 bank of [E, H, I/2] or (packed [E, H, I/2], scale [E, H, I/32]).
    fp32 gate/up, SwiGLU with the clamps when ``swiglu_limit`` > 0, x route
    weight before the down projection, bf16 z, fp32 down, per-token sum in
    ascending expert id, one rounding to x.dtype."""
    bt, h = x.shape
    k = idx.shape[-1]
    if isinstance(gate_up, (tuple, list)) and len(gate_up) == 2 and isinstance(gate_up[0], (tuple, list)):
        (pg, sg), (pu, su) = gate_up
        # keyed on the caller's four tensors, not on the concatenation (a new tensor every call)
        gu = _prepack_cache.cached(
            (pg, sg, pu, su),
            lambda: ops.mxt16_prepack(torch.cat([ops._u8(pg, "packed_gate"), ops._u8(pu, "packed_up")], dim=1),
                                      torch.cat([ops._u8(sg, "scale_gate"), ops._u8(su, "scale_up")], dim=1)))
    else:
        gu = _as_mxt16_bank(gate_up, "gate_up")
    dn = _as_mxt16_bank(down, "down")
    if gu.lead != (n_experts,) or dn.lead != (n_experts,):
        raise ValueError(f"expert banks hold {gu.lead}/{dn.lead} experts, n_experts={n_experts}")
    w = scores.reshape(bt, k).float()
    y, _, _ = ops.moe_a16_forward(x.to(torch.bfloat16), gu, dn, ids=idx.reshape(bt, k), weights=w,
                                  swiglu_limit=swiglu_limit)
    return y.to(x.dtype)
