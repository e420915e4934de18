"""GPU parity of the router projection and of the model-level drop-ins:
``Router`` (model/layers.py:118-150), ``Gate`` (.mosaicvm/source/inference_model.py:550-589),
``grouped_expert_forward`` (model/layers.py:329-373) and ``exact_moe_mxint``
(kernels/exact_moe.py:22-31).

Bars: router logits bit-exact against the exact dot product rounded once to
fp32; ids and weights bit-exact against the oracle's routing of those logits;
layer outputs within |got - ref| <= 2e-2 * max(1, |ref|) of the oracle.
"""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import codecs as C
from oracle import moe as MO

pytestmark = pytest.mark.gpu

TOL = 2e-2


def assert_close(got, ref, tol=TOL, what=""):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref) / np.maximum(1.0, np.abs(ref))
    worst = float(err.max()) if err.size else 0.0
    assert worst <= tol, f"{what}: max scaled error {worst:.3e} > {tol}"


@pytest.mark.parametrize("m,e,h,xdt,wdt", [(1, 256, 7168, "bf16", "bf16"), (5, 256, 7168, "bf16", "f32"),
                                           (70, 64, 512, "f32", "bf16"), (9, 33, 384, "f32", "f32")])
def test_router_logits_exact(dev, m, e, h, xdt, wdt):
    from mosaic_amd import ops
    rng = np.random.default_rng(m + e + h)
    dt = {"bf16": torch.bfloat16, "f32": torch.float32}
    x = torch.from_numpy(rng.standard_normal((m, h)).astype(np.float32)).to(dt[xdt])
    w = torch.from_numpy((rng.standard_normal((e, h)) * 0.02).astype(np.float32)).to(dt[wdt])
    got = ops.router_logits(x.to(dev), w.to(dev)).cpu().numpy()
    ref = MO.router_logits(x.float().numpy(), w.float().numpy())
    np.testing.assert_array_equal(got, ref)


def _v4_cfg(e=256, h=1024, k=8):
    return SimpleNamespace(n_routed_experts=e, hidden_size=h, scoring_func="sqrtsoftplus", num_experts_per_tok=k,
                           norm_topk_prob=True, routed_scaling_factor=1.5)


def test_router_drop_in(dev):
    """Router.forward: projection + sqrtsoftplus + bias + renorm x 1.5."""
    from mosaic_amd.layers import Router
    rng = np.random.default_rng(3)
    cfg = _v4_cfg()
    r = Router(cfg, device=dev)
    with torch.no_grad():
        r.weight.copy_(torch.from_numpy((rng.standard_normal((256, 1024)) * 0.05).astype(np.float32)))
        r.e_score_correction_bias.copy_(torch.from_numpy((rng.standard_normal(256) * 0.1).astype(np.float32)))
    x = torch.from_numpy(rng.standard_normal((12, 1024)).astype(np.float32)).to(torch.bfloat16)
    w, ids = r(x.to(dev))
    assert ids.dtype == torch.int64 and w.dtype == torch.float32
    lg = MO.router_logits(x.float().numpy(), r.weight.detach().cpu().numpy())
    ids_ref, w_ref = MO.route_topk(lg, 8, "sqrtsoftplus", bias=r.e_score_correction_bias.detach().cpu().numpy(),
                                   route_scale=1.5)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy(), w_ref)


@pytest.mark.parametrize("func,with_bias", [("sigmoid", True), ("softmax", False), ("sqrtsoftplus", True)])
def test_gate_drop_in(dev, func, with_bias):
    from mosaic_amd.layers import Gate
    rng = np.random.default_rng(5)
    args = SimpleNamespace(dim=768, n_activated_experts=6, score_func=func, route_scale=2.5, n_hash_layers=0,
                           n_routed_experts=64, vocab_size=100)
    g = Gate(3, args, device=dev)
    with torch.no_grad():
        g.weight.copy_(torch.from_numpy((rng.standard_normal((64, 768)) * 0.05).astype(np.float32)))
        if not with_bias:
            g.bias = None
        else:
            g.bias.copy_(torch.from_numpy((rng.standard_normal(64) * 0.1).astype(np.float32)))
    x = torch.from_numpy(rng.standard_normal((7, 768)).astype(np.float32)).to(torch.bfloat16)
    w, ids = g(x.to(dev))
    lg = MO.router_logits(x.float().numpy(), g.weight.detach().cpu().numpy())
    ids_ref, w_ref = MO.route_topk(lg, 6, func, bias=None if g.bias is None else g.bias.detach().cpu().numpy(),
                                   renorm=func != "softmax", route_scale=2.5)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(w.cpu().numpy(), w_ref, rtol=2e-7, atol=0)


def test_gate_hash_layer_raises(dev):
    """Hash routing (tid2eid lookups) is outside this build's path: the hash
    layers of Gate raise instead of running a torch fallback."""
    from mosaic_amd.layers import Gate
    args = SimpleNamespace(dim=256, n_activated_experts=4, score_func="sqrtsoftplus", route_scale=1.5,
                           n_hash_layers=3, n_routed_experts=32, vocab_size=50)
    g = Gate(0, args, device=dev)
    x = torch.zeros((5, 256), dtype=torch.bfloat16, device=dev)
    with pytest.raises(NotImplementedError):
        g(x, torch.tensor([3, 9, 9, 40, 0], device=dev))


def _nk_bank(rng, e, h, inter):
    def q(n, k):
        return C.quantize_mxfp4_ceil(C.round_bf16((rng.standard_normal((n, k)) * 0.03).astype(np.float32)))
    g = [q(inter, h) for _ in range(e)]
    u = [q(inter, h) for _ in range(e)]
    d = [q(h, inter) for _ in range(e)]
    st = lambda lst, j: np.stack([t[j] for t in lst])
    return (st(g, 0), st(g, 1)), (st(u, 0), st(u, 1)), (st(d, 0), st(d, 1))


def test_grouped_expert_forward_drop_in(dev):
    """model/layers.py:329-373 over MXFP4 experts given as raw NK (gate, up) and down tensors."""
    from mosaic_amd.layers import grouped_expert_forward
    rng = np.random.default_rng(7)
    e, h, inter, m, k = 8, 512, 256, 6, 3
    (pg, sg), (pu, su), (pd, sd) = _nk_bank(rng, e, h, inter)
    x = torch.from_numpy(rng.standard_normal((m, h)).astype(np.float32)).to(torch.bfloat16)
    idx = np.stack([rng.choice(e, k, replace=False) for _ in range(m)])
    scores = rng.uniform(0.05, 1.0, size=(m, k)).astype(np.float32)
    scores[2, 1] = 0.0  # a zero weight contributes nothing
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    from mosaic_amd.kernels import _prepack_cache
    _prepack_cache.clear()
    bank = ((T(pg), T(sg)), (T(pu), T(su))), (T(pd), T(sd))
    y = grouped_expert_forward(x.to(dev), T(scores), T(idx), *bank, e, swiglu_limit=10.0)
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == (m, h)
    gu_p, gu_s = np.concatenate([pg, pu], axis=1), np.concatenate([sg, su], axis=1)
    ref = MO.moe_layer_a16(x.float().numpy(), idx, scores, gu_p, gu_s, pd, sd, swiglu_limit=10.0)
    assert_close(y.float().cpu().numpy(), ref, what="grouped_expert_forward")
    # the second call reuses both prepacked banks; freeing the weights frees them
    assert _prepack_cache.size() == 2
    y2 = grouped_expert_forward(x.to(dev), T(scores), T(idx), *bank, e, swiglu_limit=10.0)
    assert _prepack_cache.size() == 2 and torch.equal(y, y2)
    del bank
    import gc
    gc.collect()
    assert _prepack_cache.size() == 0
    with pytest.raises(TypeError):
        grouped_expert_forward(x.to(dev), T(scores), T(idx), (torch.zeros(e, h, inter, device=dev),) * 2,
                               torch.zeros(e, inter, h, device=dev), e)


def test_exact_moe_mxint_drop_in(dev, monkeypatch):
    from mosaic_amd.kernels.exact_moe import exact_moe_mxint
    rng = np.random.default_rng(8)
    e, h, inter, m, k = 8, 256, 128, 4, 2
    (pg, sg), (pu, su), (pd, sd) = _nk_bank(rng, e, h, inter)
    gu_p, gu_s = np.concatenate([pg, pu], axis=1), np.concatenate([sg, su], axis=1)
    x = torch.from_numpy(rng.standard_normal((m, h)).astype(np.float32)).to(torch.bfloat16)
    ids = np.stack([rng.choice(e, k, replace=False) for _ in range(m)])
    w = rng.uniform(0.1, 1.0, size=(m, k)).astype(np.float32)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    monkeypatch.setenv("MOSAICVM_EXACT_TARGET", "1")
    y = exact_moe_mxint(x.to(dev), T(ids), T(w), T(gu_p), T(gu_s), T(pd), T(sd))
    ref = MO.moe_layer_a8(x.float().numpy(), ids, w, gu_p, gu_s, pd, sd, swiglu_limit=10.0)
    assert_close(y.float().cpu().numpy(), ref, what="exact_moe_mxint")
    monkeypatch.setenv("MOSAICVM_EXACT_TARGET", "0")
    with pytest.raises(RuntimeError, match="MOSAICVM_EXACT_TARGET"):
        exact_moe_mxint(x.to(dev), T(ids), T(w), T(gu_p), T(gu_s), T(pd), T(sd))
