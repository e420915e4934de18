"""Pins the routing / layout / MoE oracles (CPU)."""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

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


# ---- A8 MoE oracle pinned by an independent torch-CPU restatement ----------
# Written from kernels/mxint.py:1676-1722 (the non-fused epilogue of
# fused_moe_mxint), kernels/fp4_source.py:110-156 (act_quant_ref and the
# source-semantics linear) and kernels/mxfp4.py:20-23 (the E2M1 table), with
# torch's own float8_e4m3fn cast, frexp/ldexp scales, F.silu and explicit
# bfloat16 casts -- nothing from oracle/ except the test data.
_E2M1 = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0])


def _t_act_quant(x):
    m, k = x.shape
    xb = x.float().reshape(m, k // 128, 128)
    val = xb.abs().amax(-1).clamp_min(1e-4) * (1.0 / 448.0)
    mant, ex = torch.frexp(val)  # val = mant * 2^ex, mant in [0.5, 1): power-of-two ceil
    s = torch.ldexp(torch.ones_like(val), torch.where(mant == 0.5, ex - 1, ex))
    return (xb / s[..., None]).clamp(-448.0, 448.0).reshape(m, k).to(torch.float8_e4m3fn), s


def _t_weight(packed, scale):
    p = torch.from_numpy(packed).long()
    b = torch.stack([_E2M1[p & 15], _E2M1[p >> 4]], dim=-1).reshape(p.shape[0], -1)  # low nibble = even K
    return b, torch.ldexp(torch.ones(scale.shape), torch.from_numpy(scale).int() - 127)


def _t_linear_a8(x, packed, scale):
    xq, sa = _t_act_quant(x)
    a = xq.float()
    b, sw = _t_weight(packed, scale)
    acc = torch.zeros(a.shape[0], b.shape[0])
    for g in range(a.shape[1] // 32):
        acc = acc + (a[:, 32 * g:32 * g + 32] @ b[:, 32 * g:32 * g + 32].T) * sa[:, g // 4, None] * sw[:, g][None, :]
    return acc


def _t_moe_a8(x, ids, w, bank, limit, mistake=None, shared=None):
    """mistake: None, "weight_after_down", "no_requant" (down on bf16 z with
    dequantized weights) or "fp32_gateup" (gate/up kept in fp32)."""
    gp, gs, dp, ds = bank
    m, h = x.shape
    k = ids.shape[1]

    def expert(xr, gu_p, gu_s, d_p, d_s, wt):
        gu = _t_linear_a8(xr, gu_p, gu_s)
        if mistake != "fp32_gateup":
            gu = gu.to(torch.bfloat16)
        inter = gu.shape[1] // 2
        gate, up = gu[:, :inter].float(), gu[:, inter:].float()
        if limit > 0:
            gate, up = gate.clamp(max=limit), up.clamp(-limit, limit)
        z = F.silu(gate) * up
        if mistake != "weight_after_down":
            z = z * wt
        zd = z.to(torch.bfloat16)
        if mistake == "no_requant":
            bd, swd = _t_weight(d_p, d_s)
            y = zd.float() @ (bd * swd.repeat_interleave(32, dim=1)).T
        else:
            y = _t_linear_a8(zd, d_p, d_s)
        y = y.to(torch.bfloat16).float()
        return y * wt if mistake == "weight_after_down" else y

    partials = torch.zeros(m, k, h)
    for t in range(m):
        for s in range(k):
            e = int(ids[t, s])
            partials[t, s] = expert(x[t:t + 1], gp[e], gs[e], dp[e], ds[e], float(w[t, s]))[0]
    order = torch.from_numpy(ids).long().argsort(dim=1)  # distinct ids per token in these cases
    out = torch.zeros(m, h)
    for s in range(k):
        out = out + partials[torch.arange(m), order[:, s]]
    if shared is not None:  # upstream MoE.forward: y += shared_experts(x), in fp32
        out = out + torch.cat([expert(x[t:t + 1], *shared, 1.0) for t in range(m)])
    return out.to(torch.bfloat16).float().numpy()


def _a8_case(seed=9):
    rng = np.random.default_rng(seed)
    e, h, inter, m = 4, 512, 256, 3
    q = lambda n, kk: C.quantize_mxfp4_ceil(C.round_bf16((rng.standard_normal((n, kk)) * 0.05).astype(np.float32)))
    gu = [q(2 * inter, h) for _ in range(e + 1)]
    dn = [q(h, inter) for _ in range(e + 1)]
    bank = tuple(np.stack(v) for v in ([a[0] for a in gu[:e]], [a[1] for a in gu[:e]], [a[0] for a in dn[:e]],
                                       [a[1] for a in dn[:e]]))
    shared = (gu[e][0], gu[e][1], dn[e][0], dn[e][1])
    x = C.round_bf16((rng.standard_normal((m, h)) * 2).astype(np.float32))
    ids = np.array([[2, 0], [1, 3], [3, 2]])
    w = np.array([[0.6, 0.4], [0.3, 0.7], [0.55, 0.45]], dtype=np.float32)
    return x, ids, w, bank, shared


@pytest.mark.parametrize("with_shared", [False, True])
def test_moe_a8_oracle_equals_torch_restatement(with_shared):
    """The numpy A8 MoE oracle is bit-identical to the torch restatement of
    kernels/mxint.py:1676-1722 (bf16 gate/up, fp32 SwiGLU, x weight, bf16,
    act_quant_ref, A8 down, bf16 partials, ascending-id fp32 sum)."""
    x, ids, w, bank, shared = _a8_case()
    ref = MO.moe_layer_a8(x, ids, w, *bank, swiglu_limit=10.0, shared=shared if with_shared else None)
    got = _t_moe_a8(torch.from_numpy(x), ids, w, bank, 10.0, shared=shared if with_shared else None)
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("mistake", ["weight_after_down", "no_requant", "fp32_gateup"])
def test_moe_a8_planted_mistakes_are_caught(mistake):
    """Each plausible composition mistake, planted in the restatement, moves
    most outputs off the oracle (the honest restatement matches bit for bit)."""
    x, ids, w, bank, _ = _a8_case()
    ref = MO.moe_layer_a8(x, ids, w, *bank, swiglu_limit=10.0)
    bad = _t_moe_a8(torch.from_numpy(x), ids, w, bank, 10.0, mistake=mistake)
    assert np.mean(bad == ref) < 0.5, f"{mistake} not detected"


# ---- routing: scores correctly rounded, bias, scale, planted ties ----------
def _round_f32(v) -> np.float32:
    """Round an mpmath value to the nearest fp32 (ties to even)."""
    import mpmath
    f = np.float32(float(v))
    best = f
    for cand in (np.nextafter(f, np.float32(-np.inf)), np.nextafter(f, np.float32(np.inf))):
        d_c, d_b = abs(mpmath.mpf(float(cand)) - v), abs(mpmath.mpf(float(best)) - v)
        if d_c < d_b or (d_c == d_b and (int(cand.view(np.uint32)) & 1) == 0):
            best = cand
    return best


@pytest.mark.parametrize("func", ["sigmoid", "sqrtsoftplus"])
def test_route_scores_are_correctly_rounded(func):
    """score_fn = the fp32 rounding of the exact function (50-digit mpmath),
    across the logit range, torch's softplus threshold 20 included."""
    import mpmath
    mpmath.mp.dps = 50
    rng = np.random.default_rng(3)
    xs = np.concatenate([rng.standard_normal(200) * 4, [-30.0, -5.0, 0.0, 19.999998, 20.0, 20.000002, 35.0]])
    xs = xs.astype(np.float32)
    got = MO.score_fn(xs[None, :], func)[0]
    for x, g in zip(xs.tolist(), got.tolist()):
        xm = mpmath.mpf(x)
        if func == "sigmoid":
            v = 1 / (1 + mpmath.exp(-xm))
        else:
            v = mpmath.sqrt(xm if x > 20.0 else mpmath.log(1 + mpmath.exp(xm)))
        assert np.float32(g) == _round_f32(v), (func, x)


def test_route_bias_scale_ties_brute_force():
    """sqrtsoftplus + selection bias + renorm (sum clamped at 1e-9) x 1.5, the
    reference Router (model/layers.py:127-150), against a brute-force stable
    sort; rows hold planted exact key ties (equal logits and biases) and
    one-ulp logit neighbours whose scores round together."""
    rng = np.random.default_rng(4)
    m, e, k = 32, 256, 8
    logits = rng.standard_normal((m, e)).astype(np.float32)
    bias = (rng.standard_normal(e) * 0.1).astype(np.float32)
    bias[17] = bias[200]
    for r in range(0, m, 2):
        logits[r, 200] = logits[r, 17] = logits[r].max() + np.float32(0.5)       # exact tie
        logits[r, 31] = np.nextafter(logits[r, 200], np.float32(np.inf))          # one ulp above
        bias[31] = bias[200]
    ids, w = MO.route_topk(logits, k, "sqrtsoftplus", bias=bias, route_scale=1.5)
    sc = MO.score_fn(logits, "sqrtsoftplus")
    key = (sc + bias).astype(np.float32)
    for r in range(m):
        order = sorted(range(e), key=lambda j: (-float(key[r, j]), j))[:k]
        assert ids[r].tolist() == order
        picked = sc[r, order].astype(np.float32)
        tot = np.float32(0)
        for v in picked:
            tot = np.float32(tot + v)
        np.testing.assert_array_equal(w[r], (picked / max(tot, np.float32(1e-9)) * np.float32(1.5)).astype(np.float32))
    # the planted exact tie went to the lower index
    assert list(ids[0]).index(17) < list(ids[0]).index(200)


def test_route_renorm_clamps_tiny_sums():
    """All picked scores underflow: weights stay finite (clamp_min(1e-9), layers.py:147)."""
    logits = np.full((1, 16), -200.0, dtype=np.float32)
    _, w = MO.route_topk(logits, 4, "sigmoid")
    assert np.all(np.isfinite(w)) and np.all(w == 0)


def test_router_logits_are_exact_dot_rounded_once():
    """router_logits = fp32 rounding of the exact dot (Fraction arithmetic)."""
    from fractions import Fraction
    rng = np.random.default_rng(5)
    x = C.round_bf16(rng.standard_normal((2, 64)).astype(np.float32))
    w = (rng.standard_normal((5, 64)) * 0.02).astype(np.float32)
    w[0] = -w[1]  # a row whose dot cancels against its neighbour's
    got = MO.router_logits(x, w)
    for t in range(2):
        for j in range(5):
            exact = sum(Fraction(float(a)) * Fraction(float(b)) for a, b in zip(x[t], w[j]))
            assert got[t, j] == np.float32(float(exact)), (t, j)


# ---- fused_moe_skinny oracle pinned by a torch restatement ----------------
def _t_kn_linear(x_bf16, packed, scale):
    """x @ W with W [K, N] decoded from KN packed/scale (fp32 math, bf16 out),
    kernels/skinny_fp4.py:50-110 (LUT, low nibble = even n, per-32-N scale)."""
    p = torch.from_numpy(packed).long()
    lut = torch.stack([_E2M1[p & 15], _E2M1[p >> 4]], dim=-1).reshape(p.shape[0], -1)
    sw = torch.ldexp(torch.ones(scale.shape), torch.from_numpy(scale).int() - 127).repeat_interleave(32, dim=1)
    return (x_bf16.double() @ (lut * sw).double()).float().to(torch.bfloat16)


def test_moe_skinny_oracle_equals_torch_restatement():
    """kernels/skinny_fp4.py:267-322 in torch bf16 ops: silu/multiply on bf16
    tensors, y_g * weights (bf16), index_add_ into a bf16 zero tensor (the CPU
    index_add_ adds in index order)."""
    rng = np.random.default_rng(12)
    e, h, inter, m, k = 4, 256, 128, 3, 2
    q = lambda n, kk: C.quantize_mxfp4_ceil(C.round_bf16((rng.standard_normal((n, kk)) * 0.05).astype(np.float32)))
    gu = [q(h, 2 * inter) for _ in range(e)]
    dn = [q(inter, h) for _ in range(e)]
    gp, gs = np.stack([a[0] for a in gu]), np.stack([a[1] for a in gu])
    dp, ds = np.stack([a[0] for a in dn]), np.stack([a[1] for a in dn])
    x = C.round_bf16((rng.standard_normal((m, h)) * 2).astype(np.float32))
    ids = np.array([[2, 0], [1, 3], [3, 2]])
    w = np.array([[0.6, 0.4], [0.3, 0.7], [0.55, 0.45]], dtype=np.float32)
    ref = MO.moe_layer_skinny(x, ids, w, gp, gs, dp, ds)
    xt = torch.from_numpy(x).to(torch.bfloat16)
    flat = ids.reshape(-1)
    token_of = np.repeat(np.arange(m), k)
    order = np.argsort(flat, kind="stable")
    yg = torch.zeros(flat.size, h, dtype=torch.bfloat16)
    for p in order:
        g = _t_kn_linear(xt[token_of[p]:token_of[p] + 1], gp[flat[p]], gs[flat[p]])
        z = F.silu(g[:, :inter]) * g[:, inter:]
        yg[p] = _t_kn_linear(z, dp[flat[p]], ds[flat[p]])[0]
    yg = yg * torch.from_numpy(w.reshape(-1)).to(torch.bfloat16)[:, None]
    y = torch.zeros(m, h, dtype=torch.bfloat16)
    y.index_add_(0, torch.from_numpy(token_of), yg)
    np.testing.assert_array_equal(y.float().numpy(), ref)
