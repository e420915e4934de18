"""GPU parity of the reference Router's own scoring path and of the MoE layer
at the benchmark geometry (hidden 7168, inter 2048, top-8).

* The reference Router (``model/layers.py:127-150``): sqrtsoftplus scores, an
  ``e_score_correction_bias`` added for selection only, renormalization with
  ``clamp_min(1e-9)`` and ``routed_scaling_factor`` 1.5, 256 experts, with
  planted exact key ties and one-ulp logit neighbours.  ids and weights must
  be bit-exact on every device path: the router kernel, the single-token
  decode kernel (routing fused into gate/up) and both layout kernels.
* M = 4 and 16 at hidden 7168 / inter 2048 on a 32-expert bank (one GPU's
  expert-parallel share), A16 contract.
* BASELINE.json configs[3] at full size: 4096 tokens, 256 experts, Zipf(1.1)
  popularity with 8 experts pinned to zero, A8 contract; sampled tokens,
  including one routed to the most loaded expert, against the oracle.

Float bar: |got - ref| <= 2e-2 * max(1, |ref|) elementwise (the benchmark spec).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import codecs as C
from oracle import moe as MO

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _ops():
    from mosaic_amd import ops
    return ops


def assert_close(got, ref, tol=TOL, what=""):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref) / np.maximum(1.0, np.abs(ref))
    worst = float(err.max()) if err.size else 0.0
    assert worst <= tol, f"{what}: max scaled error {worst:.3e} > {tol} (at {np.unravel_index(err.argmax(), err.shape)})"


def _router_case(m: int, e: int = 256, seed: int = 4):
    """Seeded N(0,1) logits and N(0, 0.1) biases with planted ties on even rows:
    experts 17 and 200 share a logit and a bias (an exact key tie), expert 31
    sits one ulp above them with the same bias."""
    rng = np.random.default_rng(seed)
    logits = rng.standard_normal((m, e)).astype(np.float32)
    bias = (rng.standard_normal(e) * 0.1).astype(np.float32)
    bias[17] = bias[200]
    bias[31] = bias[200]
    for r in range(0, m, 2):
        logits[r, 200] = logits[r, 17] = logits[r].max() + np.float32(0.5)
        logits[r, 31] = np.nextafter(logits[r, 200], np.float32(np.inf))
    return logits, bias


ROUTER = dict(score_func="sqrtsoftplus", route_scale=1.5)


def test_route_kernel_reference_router_bit_exact(dev):
    ops = _ops()
    logits, bias = _router_case(64)
    ids, w = ops.moe_route_topk(torch.from_numpy(logits).to(dev), 8, "sqrtsoftplus", route_scale=1.5,
                                bias=torch.from_numpy(bias).to(dev))
    ids_ref, w_ref = MO.route_topk(logits, 8, "sqrtsoftplus", bias=bias, route_scale=1.5)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy(), w_ref)
    assert list(ids_ref[0]).index(17) < list(ids_ref[0]).index(200)


def _score_tie_case(m: int, func: str, e: int = 256, k: int = 8, seed: int = 8):
    """Seeded logits where, on every row, two experts whose logits are one ulp
    apart share one fp32 score and the LARGER logit belongs to the HIGHER
    index: once inside the picks (experts 40 and 60 near the top) and once at
    the k-th / (k+1)-th boundary (experts 70 and 90), so ranking by logit
    would disagree with ranking by score with ties to the lower index."""
    rng = np.random.default_rng(seed)
    logits = (rng.standard_normal((m, e)) * 0.5).astype(np.float32)
    for r in range(m):
        for lo, hi, base in ((40, 60, 3.0), (70, 90, None)):
            if base is None:  # 40 and 60 lead, so k - 3 others go before 90 (k-th) and 70
                rest = np.sort(np.delete(logits[r], [40, 60, 70, 90]))[::-1]
                base = float(rest[k - 4] + rest[k - 3]) / 2
            t = np.float32(base)
            for _ in range(64):  # walk up until t and its lower neighbour share a score
                tl = np.nextafter(t, np.float32(-np.inf))
                if MO.score_fn(np.array([[tl, t]], dtype=np.float32), func)[0].tolist() == \
                        MO.score_fn(np.array([[t, t]], dtype=np.float32), func)[0].tolist():
                    break
                t = np.nextafter(t, np.float32(np.inf))
            logits[r, hi], logits[r, lo] = t, np.nextafter(t, np.float32(-np.inf))
    return logits


@pytest.mark.parametrize("func", ["sigmoid", "sqrtsoftplus"])
def test_route_score_ties_without_bias(dev, func):
    """No bias: the kernels select on the logit and must fall back to the
    scores when two picks, or the last pick and the next candidate, share an
    fp32 score (ids bit-exact on the router kernel and the decode kernel)."""
    ops = _ops()
    logits = _score_tie_case(32, func)
    ids_ref, w_ref = MO.route_topk(logits, 8, func)
    assert all(40 in row and 70 in row and 90 not in row for row in ids_ref.tolist())
    ids, w = ops.moe_route_topk(torch.from_numpy(logits).to(dev), 8, func)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy(), w_ref)
    e, h, inter = 256, 512, 512
    g, raw = _device_bank(ops, dev, e - 1, h, inter, seed=5)
    gp, gs, dp, ds = raw
    gu_b, d_b = ops.mxt16_prepack(gp, gs), ops.mxt16_prepack(dp, ds)
    for r in range(4):  # M = 1: routing fused into the decode gate/up kernel
        x = torch.randn(1, h, generator=g, device=dev).to(torch.bfloat16)
        _, ids1, w1 = ops.moe_a16_forward(x, gu_b, d_b, logits=torch.from_numpy(logits[r:r + 1]).to(dev), top_k=8,
                                          score_func=func)
        np.testing.assert_array_equal(ids1.cpu().numpy(), ids_ref[r:r + 1])
        np.testing.assert_array_equal(w1.cpu().numpy(), w_ref[r:r + 1])


def _device_bank(ops, dev, e, h, inter, seed):
    """e routed experts + 1 shared, N(0, 0.02) quantized on the device (ceil recipe)."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    gp = torch.empty(e + 1, 2 * inter, h // 2, dtype=torch.uint8, device=dev)
    gs = torch.empty(e + 1, 2 * inter, h // 32, dtype=torch.uint8, device=dev)
    dp = torch.empty(e + 1, h, inter // 2, dtype=torch.uint8, device=dev)
    ds = torch.empty(e + 1, h, inter // 32, dtype=torch.uint8, device=dev)
    for i in range(e + 1):
        p, s = ops.mx_quantize((torch.randn(2 * inter, h, generator=g, device=dev) * 0.02).to(torch.bfloat16))
        gp[i].copy_(p)
        gs[i].copy_(s)
        p, s = ops.mx_quantize((torch.randn(h, inter, generator=g, device=dev) * 0.02).to(torch.bfloat16))
        dp[i].copy_(p)
        ds[i].copy_(s)
    return g, (gp, gs, dp, ds)


def _host_getters(raw, used):
    """Host copies of the used experts only (the oracle streams them by id)."""
    gp, gs, dp, ds = raw
    host = {e: (gp[e].cpu().numpy(), gs[e].cpu().numpy(), dp[e].cpu().numpy(), ds[e].cpu().numpy()) for e in used}
    return tuple((lambda j: (lambda e: host[e][j]))(j) for j in range(4))


@pytest.mark.parametrize("m,a8", [(1, False), (4, False), (40, False), (3, True)])
def test_moe_paths_reference_router_bit_exact(dev, m, a8):
    """Routing fused into the layer (M = 1: the decode gate/up kernel; M = 4: the
    small layout kernel; M = 40: the one-workgroup layout kernel; A8 at M = 3)
    with the reference Router's scoring: ids and weights bit-exact, output
    within the float bar."""
    ops = _ops()
    e, h, inter, k = 256, 512, 512, 8
    g, raw = _device_bank(ops, dev, e - 1, h, inter, seed=100 + m)  # 256 experts (the last one unused as shared)
    gp, gs, dp, ds = raw
    logits, bias = _router_case(m)
    x = torch.randn(m, h, generator=g, device=dev).to(torch.bfloat16)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    fwd = ops.moe_a8_forward if a8 else ops.moe_a16_forward
    y, ids, w = fwd(x, ops.mxt16_prepack(gp, gs), ops.mxt16_prepack(dp, ds), logits=T(logits),
                    top_k=k, route_bias=T(bias), swiglu_limit=10.0, **ROUTER)
    ids_ref, w_ref = MO.route_topk(logits, k, "sqrtsoftplus", bias=bias, route_scale=1.5)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy(), w_ref)
    oracle = MO.moe_layer_a8 if a8 else MO.moe_layer_a16
    get = _host_getters(raw, sorted(set(ids_ref.flatten().tolist())))
    ref = oracle(x.float().cpu().numpy(), ids_ref, w_ref, *get, swiglu_limit=10.0)
    assert_close(y.float().cpu().numpy(), ref, what=f"moe m={m} a8={a8} reference router")


@pytest.mark.parametrize("m", [4, 16, 64])
def test_moe_a16_baseline_geometry_multi_token(dev, m):
    """M = 4 / 16 / 64 at hidden 7168, inter 2048, top-8, shared expert, on a
    32-expert bank: the layout + grouped gate/up + down + combine kernels at the
    shapes the bench times."""
    ops = _ops()
    e, h, inter, k = 32, 7168, 2048, 8
    g, raw = _device_bank(ops, dev, e, h, inter, seed=40 + m)
    gp, gs, dp, ds = raw
    x = torch.randn(m, h, generator=g, device=dev).to(torch.bfloat16)
    logits = torch.randn(m, e, generator=g, device=dev)
    y, ids, w = ops.moe_a16_forward(x, ops.mxt16_prepack(gp[:e], gs[:e]), ops.mxt16_prepack(dp[:e], ds[:e]),
                                    logits=logits, top_k=k,
                                    shared=(ops.mxt16_prepack(gp[e], gs[e]), ops.mxt16_prepack(dp[e], ds[e])))
    ids_ref, w_ref = MO.route_topk(logits.cpu().numpy(), k, "sigmoid")
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    get = _host_getters(raw, sorted(set(ids_ref.flatten().tolist())))
    ref = MO.moe_layer_a16(x.float().cpu().numpy(), ids_ref, w_ref, *get,
                           shared=(gp[e].cpu().numpy(), gs[e].cpu().numpy(), dp[e].cpu().numpy(),
                                   ds[e].cpu().numpy()))
    assert_close(y.float().cpu().numpy(), ref, what=f"moe a16 m={m} baseline geometry")


def test_moe_a8_prefill_config4_full_size(dev):
    """BASELINE.json configs[3] at full size: 4096 tokens, 256 experts + shared,
    hidden 7168, inter 2048, top-8 by Gumbel-top-k over Zipf(1.1) popularity
    on a seeded expert permutation with 8 experts pinned to zero.  Routing,
    layout and the empty experts are checked in full; four sampled tokens (one
    routed to the most loaded expert) are checked against the A8 oracle."""
    ops = _ops()
    m, e, h, inter, k = 4096, 256, 7168, 2048, 8
    g, raw = _device_bank(ops, dev, e, h, inter, seed=77)
    gp, gs, dp, ds = raw
    perm = torch.randperm(e, generator=g, device=dev)
    logp = torch.tensor([-1.1 * math.log(r + 1) for r in range(e)], device=dev)[torch.argsort(perm)]
    logp[perm[-8:]] = -1e4
    u = torch.rand(m, e, generator=g, device=dev).clamp(1e-9, 1 - 1e-9)
    logits = logp[None, :] - torch.log(-torch.log(u))
    x = torch.randn(m, h, generator=g, device=dev).to(torch.bfloat16)
    y, ids, w = ops.moe_a8_forward(x, ops.mxt16_prepack(gp[:e], gs[:e]), ops.mxt16_prepack(dp[:e], ds[:e]),
                                   logits=logits, top_k=k, swiglu_limit=10.0,
                                   shared=(ops.mxt16_prepack(gp[e], gs[e]), ops.mxt16_prepack(dp[e], ds[e])))
    lg = logits.cpu().numpy()
    ids_ref, w_ref = MO.route_topk(lg, k, "sigmoid")
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(w.cpu().numpy(), w_ref)
    counts = np.bincount(ids_ref.flatten(), minlength=e)
    assert np.all(counts[perm[-8:].cpu().numpy()] == 0), "pinned experts must receive no tokens"
    top = int(counts.argmax())
    assert counts[top] > 1000
    rng = np.random.default_rng(3)
    rows = [int(np.nonzero((ids_ref == top).any(axis=1))[0][0])] + rng.choice(m, 3, replace=False).tolist()
    get = _host_getters(raw, sorted(set(ids_ref[rows].flatten().tolist())))
    ref = MO.moe_layer_a8(x[rows].float().cpu().numpy(), ids_ref[rows], w_ref[rows], *get, swiglu_limit=10.0,
                          shared=(gp[e].cpu().numpy(), gs[e].cpu().numpy(), dp[e].cpu().numpy(),
                                  ds[e].cpu().numpy()))
    assert_close(y[rows].float().cpu().numpy(), ref, what="config 4 sampled tokens")
