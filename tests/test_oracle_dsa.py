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
