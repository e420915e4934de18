"""Pins the routing / layout / MoE oracles (CPU)."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import codecs as C
from oracle import moe as MO


@pytest.mark.parametrize("func", ["sigmoid", "softmax", "sqrtsoftplus"])
def test_route_topk_equals_full_sort_of_scores(func):
    """Selecting on the logit equals a stable full sort of the scores
    (.mosaicvm/source/inference_model.py:573-583) on seeded N(0,1) logits."""
    rng = np.random.default_rng(0)
    logits = rng.standard_normal((64, 256)).astype(np.float32)
    ids, w = MO.route_topk(logits, 8, func)
    scores = MO.score_fn(logits, func)
    for r in range(64):
        order = sorted(range(256), key=lambda e: (-float(scores[r, e]), e))[:8]
        assert ids[r].tolist() == order
    picked = np.take_along_axis(scores, ids, 1).astype(np.float64)
    if func != "softmax":
        np.testing.assert_allclose(w.sum(1), 1.0, rtol=1e-6)
        picked = picked / picked.sum(1, keepdims=True)
    np.testing.assert_allclose(w, picked, rtol=1e-6)


def test_route_ties_go_to_lower_index():
    logits = np.zeros((1, 16), dtype=np.float32)
    logits[0, [3, 9, 12]] = 2.0
    ids, _ = MO.route_topk(logits, 5)
    assert ids[0].tolist() == [3, 9, 12, 0, 1]


def test_route_bias_selects_but_does_not_weight():
    """Bias shifts selection only (inference_model.py:579-586)."""
    logits = np.array([[0.0, 0.1, 0.2, 0.3]], dtype=np.float32)
    bias = np.array([5.0, 0, 0, 0], dtype=np.float32)
    ids, w = MO.route_topk(logits, 2, "sigmoid", bias=bias)
    assert ids[0].tolist() == [0, 3]
    s = MO.score_fn(logits, "sigmoid")[0]
    np.testing.assert_allclose(w[0], [s[0] / (s[0] + s[3]), s[3] / (s[0] + s[3])], rtol=1e-6)


def test_layout_reference_kat():
    """tests/test_moe_layout.py:13-24."""
    sorted_ids, perm, offsets, counts = MO.layout_assignments(np.array([3, 0, 3, 1]), 4)
    assert counts.tolist() == [1, 1, 0, 2]
    assert offsets.tolist() == [0, 1, 2, 2, 4]
    assert sorted_ids.tolist() == [0, 1, 3, 3]
    assert perm.tolist() == [1, 3, 0, 2]  # stable: within expert 3, assignment 0 before 2


@pytest.mark.parametrize("block_m", [1, 8, 16])
def test_emit_tiles_closed_form(block_m):
    """tests/test_emit_tiles.py:14-34 without the 32-tile cap."""
    counts = np.array([0, 1, block_m - 1, block_m, block_m + 1, 3 * block_m + 2, 40 * block_m + 3])
    ei, ms, rows = MO.emit_tiles(counts, block_m)
    exp = [(e, t * block_m, min(block_m, c - t * block_m)) for e, c in enumerate(counts.tolist())
           for t in range((c + block_m - 1) // block_m)]
    assert list(zip(ei.tolist(), ms.tolist(), rows.tolist())) == exp
    assert sum(1 for e in ei if e == 6) == (40 * block_m + 3 + block_m - 1) // block_m > 32  # reference cap


def _bank(rng, e, h, inter):
    q = lambda n, k: C.quantize_mxfp4_ceil((rng.standard_normal((n, k)) * 0.05).astype(np.float32))
    gu = [q(2 * inter, h) for _ in range(e)]
    d = [q(h, inter) for _ in range(e)]
    return (np.stack([a[0] for a in gu]), np.stack([a[1] for a in gu]), np.stack([a[0] for a in d]),
            np.stack([a[1] for a in d]))


def _independent(x, ids, w, bank, limit, weight_after_down=False):
    """Per-token float64 loop over dequantized experts (tests/test_exact_expert_semantics.py:38-55 style)."""
    gp, gs, dp, ds = bank
    out = np.zeros(x.shape, dtype=np.float64)
    for t in range(x.shape[0]):
        for s in sorted(range(ids.shape[1]), key=lambda j: int(ids[t, j])):
            e = int(ids[t, s])
            wgu = C.dequant_mxfp4(gp[e], gs[e]).astype(np.float64)
            wd = C.dequant_mxfp4(dp[e], ds[e]).astype(np.float64)
            inter = wgu.shape[0] // 2
            gu = wgu @ x[t].astype(np.float64)
            g, u = gu[:inter], gu[inter:]
            if limit > 0:
                g, u = np.minimum(g, limit), np.clip(u, -limit, limit)
            z = g / (1 + np.exp(-g)) * u
            if weight_after_down:
                out[t] += float(w[t, s]) * (wd @ C.round_bf16(z.astype(np.float32)).astype(np.float64))
            else:
                out[t] += wd @ C.round_bf16((z * float(w[t, s])).astype(np.float32)).astype(np.float64)
    return out


@pytest.mark.parametrize("limit", [0.0, 10.0])
def test_moe_a16_vs_independent_loop(limit):
    rng = np.random.default_rng(7)
    e, h, inter, m, k = 6, 128, 64, 3, 3
    bank = _bank(rng, e, h, inter)
    x = C.round_bf16((rng.standard_normal((m, h)) * 6).astype(np.float32))
    ids, w = MO.route_topk(rng.standard_normal((m, e)).astype(np.float32), k)
    got = MO.moe_layer_a16(x, ids, w, *bank, swiglu_limit=limit, out_bf16=False)
    ref = _independent(x, ids, w, bank, limit)
    np.testing.assert_allclose(got, ref, rtol=2e-3, atol=2e-3)


def test_weight_before_down_is_detectable():
    """A planted mistake (route weight applied after the down projection) must
    move the result beyond the parity tolerance (tests/test_exact_expert_semantics.py:78-107)."""
    rng = np.random.default_rng(8)
    e, h, inter = 4, 128, 64
    bank = _bank(rng, e, h, inter)
    x = C.round_bf16((rng.standard_normal((2, h)) * 6).astype(np.float32))
    ids = np.array([[1, 3], [0, 2]])
    w = np.array([[0.25, 1.5], [0.5, 0.01]], dtype=np.float32)
    good = MO.moe_layer_a16(x, ids, w, *bank, swiglu_limit=10.0, out_bf16=False)
    bad = _independent(x, ids, w, bank, 10.0, weight_after_down=True)
    assert not np.allclose(good, bad, atol=1e-3)


def test_moe_a8_equals_mxint_sequence():
    """fused_moe_mxint contract (kernels/mxint.py:1587-1722): A8 gate/up -> bf16, SwiGLU,
    x weight, bf16, act_quant, A8 down -> bf16 partials, ascending fp32 sum."""
    from oracle import linear as L
    rng = np.random.default_rng(9)
    e, h, inter = 3, 256, 128
    bank = _bank(rng, e, h, inter)
    x = C.round_bf16(rng.standard_normal((2, h)).astype(np.float32))
    ids = np.array([[2, 0], [1, 2]])
    w = np.array([[0.6, 0.4], [0.3, 0.7]], dtype=np.float32)
    got = MO.moe_layer_a8(x, ids, w, *bank, swiglu_limit=10.0)
    gp, gs, dp, ds = bank
    for t in range(2):
        acc = np.zeros(h, dtype=np.float32)
        for s in np.argsort(ids[t], kind="stable"):
            ex = ids[t, s]
            g = L.mx_linear_a8(x[t:t + 1], gp[ex], gs[ex])[0]
            z = MO.swiglu(g[:inter], g[inter:], 10.0)
            z = C.round_bf16((z * w[t, s]).astype(np.float32))
            acc = (acc + L.mx_linear_a8(z[None], dp[ex], ds[ex])[0]).astype(np.float32)
        np.testing.assert_array_equal(got[t], C.round_bf16(acc))
