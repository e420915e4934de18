"""Pins the DSA oracles (CPU): exact dot, canonical indexer score, top-k rule,
sparse-attention closed forms."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import codecs as C
from oracle import dsa as D


def _codes(rng, shape):
    """Random finite e4m3 codes covering subnormals, normals and +-448."""
    c = rng.integers(0, 256, size=shape, dtype=np.uint8)
    return np.where((c & 0x7F) == 0x7F, c ^ 0x01, c).astype(np.uint8)  # drop NaN codes


def test_exact_dot_equals_integer_restatement():
    """e4m3 * 512 is an integer (|.| <= 229376): the int64 dot is the exact dot."""
    rng = np.random.default_rng(0)
    q = _codes(rng, (8, 128))
    k = _codes(rng, (300, 128))
    k[0] = 0x7E  # 448 everywhere: the largest products
    q[0] = 0x7E
    k[1] = 0x01  # 2^-9: the smallest
    iq = (C.e4m3_decode(q).astype(np.float64) * 512).astype(np.int64)
    ik = (C.e4m3_decode(k).astype(np.float64) * 512).astype(np.int64)
    assert np.all(iq == C.e4m3_decode(q).astype(np.float64) * 512)
    exact = (ik @ iq.T).astype(np.float64) / 2.0 ** 18  # exact: |int dot| < 2^43
    np.testing.assert_array_equal(D.exact_dots(q, k), exact.astype(np.float32))
    assert D.exact_dots(q, k)[0, 0] == np.float32(128 * 448.0 * 448.0)


def test_indexer_scores_match_float64_formula():
    """score[t] = sum_h w_h ReLU(q_h . k_t qs_h ks_t) (inference_model.py:424-425) within fp32 rounding."""
    rng = np.random.default_rng(1)
    b, h, l = 2, 64, 500
    q, qs = D.quantize_rows_e4m3(rng.standard_normal((b, h, 128)))
    k, ks = D.quantize_rows_e4m3(rng.standard_normal((b, l, 128)))
    w = rng.standard_normal((b, h)).astype(np.float32)
    got = D.indexer_scores(q, qs, k, ks, w)
    qv, kv = C.e4m3_decode(q).astype(np.float64), C.e4m3_decode(k).astype(np.float64)
    dots = np.einsum("bhd,bld->blh", qv, kv) * qs[:, None, :] * ks[:, :, None]
    ref = (np.maximum(dots, 0) * w[:, None, :]).sum(-1)
    scale = (np.abs(np.maximum(dots, 0) * w[:, None, :])).sum(-1)
    assert np.all(np.abs(got - ref) <= 1e-5 * scale + 1e-30)
    # a transposed weight or a missing ReLU moves the result far beyond that
    bad = (dots * w[:, None, :]).sum(-1)
    assert np.abs(bad - ref).max() > 1e-2 * scale.max()


def test_indexer_one_hot_closed_form():
    """One nonzero q element (head 3, dim 17): every score is one rounded product chain."""
    rng = np.random.default_rng(2)
    q = np.zeros((1, 16, 128), dtype=np.uint8)
    q[0, 3, 17] = C.e4m3_encode(np.array([1.75], np.float32))[0]
    qs = rng.random((1, 16)).astype(np.float32) + 0.5
    k, ks = D.quantize_rows_e4m3(rng.standard_normal((1, 64, 128)))
    w = rng.standard_normal((1, 16)).astype(np.float32)
    got = D.indexer_scores(q, qs, k, ks, w)[0]
    d = (np.float32(1.75) * C.e4m3_decode(k[0, :, 17])).astype(np.float32)
    a = (d * qs[0, 3]) * ks[0]
    want = np.where(a > 0, a, np.float32(0)) * w[0, 3]
    np.testing.assert_array_equal(got, want.astype(np.float32) + np.float32(0))


def test_topk_rule_brute_force():
    rng = np.random.default_rng(3)
    s = rng.integers(-3, 4, size=(3, 50)).astype(np.float32)  # many ties
    s[1, 7] = np.nan
    lengths = np.array([50, 20, 5])
    got = D.topk_from_scores(s, 8, lengths, offset=100)
    for b in range(3):
        n = lengths[b]
        vals = [(-np.inf if np.isnan(v) else float(v)) for v in s[b, :n]]
        order = sorted(range(n), key=lambda t: (-vals[t], t))[:8]
        exp = [t + 100 for t in order] + [-1] * (8 - len(order))
        assert got[b].tolist() == exp
    assert got[2, 5:].tolist() == [-1, -1, -1]


def test_order_key_is_monotone():
    v = np.array([-np.inf, -3.5, -1e-30, -0.0, 0.0, 1e-30, 2.0, np.inf], dtype=np.float32)
    k = D.f32_order_key(v).astype(np.int64)
    assert np.all(np.diff(k) >= 0) and k[3] < k[4]
    assert D.f32_order_key(np.array([np.nan], np.float32))[0] == 0


def _mla_inputs(rng, b=1, h=16, n=40, t=12, sb=64):
    q = C.round_bf16(rng.standard_normal((b, h, 576)).astype(np.float32))
    lat, ls = D.quantize_rows_e4m3(rng.standard_normal((b, n, 512 // sb, sb)))
    lat = lat.reshape(b, n, 512)
    rope = C.round_bf16(rng.standard_normal((b, n, 64)).astype(np.float32))
    idx = rng.integers(0, n, size=(b, t)).astype(np.int32)
    return q, lat, ls, rope, idx


def test_mla_single_token_is_its_row():
    rng = np.random.default_rng(4)
    q, lat, ls, rope, idx = _mla_inputs(rng)
    idx[:] = -1
    idx[0, 5] = 9
    o = D.mla_sparse_decode(q, lat, ls, rope, None, idx, 0.05)
    row = D.dequant_kv_latent(lat[0, 9], ls[0, 9], 64)
    np.testing.assert_array_equal(o[0], np.broadcast_to(row, o[0].shape))
    # with a sink s0: o = row / (1 + exp(sink - s))
    sink = rng.standard_normal(16).astype(np.float32)
    o2 = D.mla_sparse_decode(q, lat, ls, rope, sink, idx, 0.05)
    kv = np.concatenate([row, rope[0, 9]])
    s = (q[0].astype(np.float64) @ kv.astype(np.float64)).astype(np.float32) * np.float32(0.05)
    want = row[None, :] / (1.0 + np.exp(sink.astype(np.float64) - s))[:, None]
    np.testing.assert_allclose(o2[0], want, rtol=1e-2, atol=1e-6)


def test_mla_equal_scores_give_mean_and_mask():
    rng = np.random.default_rng(5)
    q, lat, ls, rope, idx = _mla_inputs(rng, t=6)
    q[:] = 0
    idx[0] = [1, 2, -1, 3, 40, 2]  # -1 and >= n are masked; a repeated index counts twice
    o = D.mla_sparse_decode(q, lat, ls, rope, None, idx, 1.0)
    rows = D.dequant_kv_latent(lat[0, [1, 2, 3, 2]], ls[0, [1, 2, 3, 2]], 64)
    np.testing.assert_allclose(o[0], np.broadcast_to(rows.mean(0), o[0].shape), rtol=1e-2, atol=1e-3)


def test_mla_matches_naive_softmax():
    """Within the parity tolerance of a float64 softmax without bf16 probabilities."""
    rng = np.random.default_rng(6)
    q, lat, ls, rope, idx = _mla_inputs(rng, b=2, h=16, n=300, t=128)
    sink = rng.standard_normal(16).astype(np.float32)
    o = D.mla_sparse_decode(q, lat, ls, rope, sink, idx, 576 ** -0.5)
    for b in range(2):
        kv = np.concatenate([D.dequant_kv_latent(lat[b], ls[b], 64), rope[b]], -1)[idx[b]].astype(np.float64)
        s = q[b].astype(np.float64) @ kv.T * 576 ** -0.5
        m = s.max(1, keepdims=True)
        p = np.exp(s - m)
        ref = (p @ kv[:, :512]) / (p.sum(1) + np.exp(sink - m[:, 0]))[:, None]
        assert np.all(np.abs(o[b] - ref) <= 2e-2 * np.maximum(1, np.abs(ref)))


def _kv_rows(rng, rows, dn):
    """bf16 kv rows whose 64-blocks span tiny, zero, ordinary and large
    magnitudes, with blocks whose max is exactly 448 * 2^k."""
    x = rng.standard_normal((rows, dn)).astype(np.float32)
    mags = np.float32(2.0) ** rng.integers(-20, 12, size=(rows, dn // 64)).astype(np.float32)
    x = x * np.repeat(mags, 64, axis=1)
    x[0, :64] = 0.0                 # all-zero block: the 1e-4 floor
    x[0, 64:128] *= 1e-7            # below the floor
    x[1, :64] = np.clip(x[1, :64], -1, 1)
    x[1, 7] = 448.0 * 2.0 ** -3     # max exactly 448 * 2^k
    x[1, 64:128] = np.clip(x[1, 64:128], -1, 1)
    x[1, 70] = -448.0 * 2.0 ** 5
    return C.round_bf16(x)


def test_kv_act_quant_matches_torch_restatement():
    """act_quant_sim as torch writes it (log2 / ceil / pow on fp32 tensors and
    torch's e4m3 cast), an independent restatement of the bit-level oracle."""
    import torch
    rng = np.random.default_rng(12)
    x = _kv_rows(rng, 40, 448)
    codes, s, vals = D.kv_act_quant(x)
    xt = torch.from_numpy(x).view(40, 7, 64)
    amax = xt.abs().amax(-1, keepdim=True).clamp_min(1e-4)
    st = torch.pow(2.0, torch.ceil(torch.log2(amax / 448.0)))
    qt = (xt / st).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    np.testing.assert_array_equal(s, st[..., 0].numpy())
    np.testing.assert_array_equal(codes, qt.view(torch.uint8).reshape(40, 448).numpy())
    np.testing.assert_array_equal(vals, (qt.float() * st).to(torch.bfloat16).float().reshape(40, 448).numpy())
    # the bf16 cache row keeps the rope dims and stores exactly the bf16 values
    kv = np.concatenate([x[:3], C.round_bf16(rng.standard_normal((3, 64)).astype(np.float32))], 1)
    row = D.kv_cache_row(kv)
    np.testing.assert_array_equal(row[:, 448:], kv[:, 448:])
    np.testing.assert_array_equal(row[:, :448], C.round_bf16(row[:, :448]))


def test_window_indices_follow_a_ring_buffer():
    """Simulate the ring (slot = position % window) and read back the slots of
    the last `window` positions, oldest first."""
    w = 8
    for p in range(0, 40):
        ring = {}
        for pos in range(p + 1):
            ring[pos % w] = pos
        got = D.window_indices(p, w)
        listed = [ring[s] for s in got if s >= 0]
        assert listed == list(range(max(0, p - w + 1), p + 1)), (p, got)
        assert (got[len(listed):] == -1).all()


def test_decode_indices_static_and_given():
    out = D.decode_indices([3, 40], 8, nc=12, ratio=4, offset=8)
    np.testing.assert_array_equal(out[0, 8:], [8] + [-1] * 11)           # (3 + 1) // 4 = 1 entry
    np.testing.assert_array_equal(out[1, 8:], list(range(8, 18)) + [-1, -1])  # 41 // 4 = 10
    cidx = np.array([[9, 11, -1], [8, 8, 13]], dtype=np.int32)
    out2 = D.decode_indices([3, 40], 8, cidx=cidx, nc=3)
    np.testing.assert_array_equal(out2[:, 8:], cidx)
    np.testing.assert_array_equal(out2[:, :8], out[:, :8])


# ---- dsa_decode_attention: per-head top-k softmax attention ----------------
def _t_topk_attention(q, k, v, topk, scale, mistake=None):
    """``reference_topk_attention`` (mosaicvm/kernels/dsa_attention.py:155-167)
    restated in torch float64: scores = einsum(q, k) * scale over [ctx, H], the
    top-k per head (here a stable sort by (-score, position): torch.topk leaves
    ties open, the build sends them to the lower position), softmax over the
    picked scores, probabilities times the gathered v rows, summed."""
    import torch
    qt, kt, vt = (torch.from_numpy(np.asarray(a, dtype=np.float64)) for a in (q, k, v))
    scores = torch.einsum("hd,chd->ch", qt, kt)
    if mistake != "no_scale":
        scores = scores * scale
    st = scores.T.contiguous()                                   # [H, ctx]
    if mistake == "ties_to_higher":
        rev = torch.sort(-st.flip(-1), dim=-1, stable=True).indices
        order = (st.shape[1] - 1 - rev)[:, :topk]
    else:
        order = torch.sort(-st, dim=-1, stable=True).indices[:, :topk]
    top = st.gather(1, order)
    gathered = vt.permute(1, 0, 2).gather(1, order.unsqueeze(-1).expand(-1, -1, vt.shape[-1]))
    if mistake == "softmax_whole_context":
        probs = torch.softmax(st, dim=-1).gather(1, order)
    else:
        probs = torch.softmax(top, dim=-1)
    out = (probs.unsqueeze(-1) * gathered).sum(dim=1)
    return out.numpy(), order.numpy()


def _topk_attention_case(tied: bool):
    """tests/test_dsa_parity.py's shape (64 heads, d 128, ctx 4096, top-256) with
    bf16 N(0,1) values; the tied case draws q, k from {-1, 0, 1} at d 8 so that
    many scores are equal across the top-k boundary."""
    rng = np.random.default_rng(21 if tied else 20)
    if tied:
        h, d, ctx, topk = 8, 8, 600, 64
        q = rng.integers(-1, 2, size=(h, d)).astype(np.float32)
        k = rng.integers(-1, 2, size=(ctx, h, d)).astype(np.float32)
    else:
        h, d, ctx, topk = 64, 128, 4096, 256
        q = C.round_bf16(rng.standard_normal((h, d)).astype(np.float32))
        k = C.round_bf16(rng.standard_normal((ctx, h, d)).astype(np.float32))
    v = C.round_bf16(rng.standard_normal((ctx, h, 128)).astype(np.float32))
    return q, k, v, topk, 1.0 / np.sqrt(d)


@pytest.mark.parametrize("tied", [False, True])
def test_head_topk_attention_equals_torch_restatement(tied):
    """The oracle's indices equal the restatement's, and its outputs agree
    within 1e-6 (the oracle rounds each score once to fp32)."""
    q, k, v, topk, scale = _topk_attention_case(tied)
    out, idx = D.head_topk_attention(q, k, v, topk, scale)
    ref_out, ref_idx = _t_topk_attention(q, k, v, topk, scale)
    if tied:
        s = np.einsum("hd,chd->hc", q, k)
        kth = np.sort(s, axis=1)[:, ::-1][:, topk - 1]
        assert all((s[i] == kth[i]).sum() > 1 for i in range(len(kth))), "the case must tie at the boundary"
    np.testing.assert_array_equal(idx, ref_idx)
    np.testing.assert_allclose(out, ref_out, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("mistake", ["no_scale", "softmax_whole_context", "ties_to_higher"])
def test_head_topk_attention_planted_mistakes_are_caught(mistake):
    """Each planted mistake moves the restatement off the oracle: the scale
    dropped (outputs), softmax over the whole context (outputs), ties sent to
    the higher position (indices and outputs on the tied case)."""
    q, k, v, topk, scale = _topk_attention_case(tied=(mistake == "ties_to_higher"))
    out, idx = D.head_topk_attention(q, k, v, topk, scale)
    bad_out, bad_idx = _t_topk_attention(q, k, v, topk, scale, mistake=mistake)
    assert not np.allclose(bad_out, out, rtol=1e-3, atol=1e-3), f"{mistake} not detected in the outputs"
    if mistake == "ties_to_higher":
        assert not np.array_equal(bad_idx, idx), "tie order not detected in the indices"
