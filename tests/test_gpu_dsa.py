"""DSA on the GPU through the C ABI: canonical indexer scores and top-k indices
bit-exact against the oracle, the certified bound stage, full-size properties,
and MLA decode within 2e-2 * max(1, |ref|)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import codecs as C
from oracle import dsa as D

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _close(got, ref, tol=TOL):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref) / np.maximum(1.0, np.abs(ref))
    assert err.max() <= tol, f"max scaled err {err.max():.3e}"


def _indexer_inputs(rng, b, h, l):
    q, qs = D.quantize_rows_e4m3(rng.standard_normal((b, h, 128)))
    k, ks = D.quantize_rows_e4m3(rng.standard_normal((b, l, 128)))
    w = (rng.standard_normal((b, h)) * (128 ** -0.5) * (h ** -0.5)).astype(np.float32)
    return q, qs, k, ks, w


def _t(dev, *arrays):
    return [torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in arrays]


@pytest.mark.parametrize("h", [16, 32, 48, 64])
def test_indexer_scores_bit_exact(dev, h):
    from mosaic_amd import ops
    rng = np.random.default_rng(h)
    q, qs, k, ks, w = _indexer_inputs(rng, 2, h, 3000)
    got = ops.dsa_indexer_scores(*_t(dev, q, qs, k, ks, w)).cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), D.indexer_scores(q, qs, k, ks, w).view(np.uint32))


def _finite_codes(rng, shape):
    c = rng.integers(0, 256, size=shape, dtype=np.uint8)
    return np.where((c & 0x7F) == 0x7F, c ^ 0x01, c).astype(np.uint8)


def test_indexer_scores_bit_exact_full_exponent_range(dev):
    """Uniformly random finite codes (subnormals to +-448 in one dot), the
    extremes, and exact cancellation: the exact-dot stage must stay exact."""
    from mosaic_amd import ops
    rng = np.random.default_rng(99)
    b, h, l = 2, 64, 2000
    q, k = _finite_codes(rng, (b, h, 128)), _finite_codes(rng, (b, l, 128))
    k[0, :32] = 0x7E                     # 448 everywhere
    k[0, 32:64] = 0x01                   # 2^-9 everywhere
    k[1, :64, :64] = k[1, :64, 64:] ^ 0x80  # halves cancel against each other
    q[1, :, 64:] = q[1, :, :64]
    qs = (rng.random((b, h)) + 0.5).astype(np.float32)
    ks = (rng.random((b, l)) + 0.5).astype(np.float32)
    w = rng.standard_normal((b, h)).astype(np.float32)
    got = ops.dsa_indexer_scores(*_t(dev, q, qs, k, ks, w)).cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), D.indexer_scores(q, qs, k, ks, w).view(np.uint32))
    idx = ops.dsa_indexer_topk(*_t(dev, q, qs, k, ks, w), 256).cpu().numpy()
    np.testing.assert_array_equal(idx, D.indexer_topk(q, qs, k, ks, w, 256))


def test_indexer_bounds_enclose_exact(dev):
    """The fp8-MFMA stage's interval contains every canonical score."""
    from mosaic_amd import ops
    rng = np.random.default_rng(7)
    q, qs, k, ks, w = _indexer_inputs(rng, 2, 64, 20000)
    k[0, :64] = 0x7E        # largest products
    k[1, :64, ::2] = 0xFE   # alternating signs: cancellation
    lo, hi = ops.dsa_indexer_bounds(*_t(dev, q, qs, k, ks, w))
    lo, hi = lo.cpu().numpy(), hi.cpu().numpy()
    s = D.indexer_scores(q, qs, k, ks, w)
    assert np.all(lo <= s) and np.all(s <= hi)
    assert np.median(hi - lo) < 0.2 * s.std()  # tight enough to prune


def test_indexer_bounds_enclose_wide_product_spans(dev):
    """Dots whose products span many binades inside every run of 8 K: one
    448 x 448 product next to seven products of 7.875 (0.017578 x 448), so a
    sum kept to ~14 bits below the largest product would drop all seven.  Also
    uniformly random finite codes (products from 2^-18 to 2^17.6).  The
    interval must contain the canonical score for every token."""
    from mosaic_amd import ops
    rng = np.random.default_rng(21)
    b, h, l = 2, 64, 4096
    big, small = C.e4m3_encode(np.array([448.0, 0.017578125], np.float32))
    q = np.full((b, h, 128), small, dtype=np.uint8)
    q[:, :, ::8] = big
    k = np.full((b, l, 128), big, dtype=np.uint8)
    k[1] = _finite_codes(rng, (l, 128))
    q[1, 32:] = _finite_codes(rng, (h - 32, 128))
    k[0, l // 2:, 1::8] ^= 0x80     # negative small products in half the rows
    qs = (rng.random((b, h)) + 0.5).astype(np.float32)
    ks = (rng.random((b, l)) + 0.5).astype(np.float32)
    w = np.abs(rng.standard_normal((b, h))).astype(np.float32)
    lo, hi = ops.dsa_indexer_bounds(*_t(dev, q, qs, k, ks, w))
    lo, hi = lo.cpu().numpy(), hi.cpu().numpy()
    s = D.indexer_scores(q, qs, k, ks, w)
    assert np.all(lo <= s) and np.all(s <= hi), f"{int((lo > s).sum() + (s > hi).sum())} scores outside their interval"
    idx = ops.dsa_indexer_topk(*_t(dev, q, qs, k, ks, w), 512).cpu().numpy()
    np.testing.assert_array_equal(idx, D.indexer_topk(q, qs, k, ks, w, 512))


@pytest.mark.parametrize("b,l,topk", [(2, 32768, 2048), (1, 5000, 512), (3, 1000, 2048), (1, 64, 16),
                                        (2, 70000, 2048)])
def test_indexer_topk_bit_exact(dev, b, l, topk):
    from mosaic_amd import ops
    rng = np.random.default_rng(l + topk)
    q, qs, k, ks, w = _indexer_inputs(rng, b, 64, l)
    got = ops.dsa_indexer_topk(*_t(dev, q, qs, k, ks, w), topk).cpu().numpy()
    np.testing.assert_array_equal(got, D.indexer_topk(q, qs, k, ks, w, topk))


@pytest.mark.parametrize("h,b,l,topk", [(16, 2, 5000, 512), (32, 1, 70000, 2048), (48, 3, 1000, 256)])
def test_indexer_topk_bit_exact_fewer_heads(dev, h, b, l, topk):
    """16/32/48 heads: the rescoring's staged q limbs for fewer head tiles, with the range's k rows
    staged in LDS (short ranges) and read from global memory (l = 70000)."""
    from mosaic_amd import ops
    rng = np.random.default_rng(h * 1000 + l)
    q, qs, k, ks, w = _indexer_inputs(rng, b, h, l)
    got = ops.dsa_indexer_topk(*_t(dev, q, qs, k, ks, w), topk).cpu().numpy()
    np.testing.assert_array_equal(got, D.indexer_topk(q, qs, k, ks, w, topk))


def test_indexer_topk_long_ragged_rows_bit_exact(dev):
    """B = 8 rows of ~98K tokens (every bound-kernel wave walks 16 groups of
    16 tokens, the deepest ring), a ragged last group, and rows of very
    different lengths (98341 down to 3000); indices bit-exact against the oracle."""
    from mosaic_amd import ops
    rng = np.random.default_rng(98)
    b, l, topk = 8, 98341, 2048
    q, qs, k, ks, w = _indexer_inputs(rng, b, 64, l)
    lengths = np.array([l, 98000, 97000, 65537, l, 50001, 98340, 3000], dtype=np.int32)
    got = ops.dsa_indexer_topk(*_t(dev, q, qs, k, ks, w), topk, lengths=torch.from_numpy(lengths).to(dev),
                               offset=5).cpu().numpy()
    np.testing.assert_array_equal(got, D.indexer_topk(q, qs, k, ks, w, topk, lengths, 5))


def test_indexer_lengths_offset_and_ties(dev):
    from mosaic_amd import ops
    rng = np.random.default_rng(11)
    b, l, topk = 3, 6000, 1024
    q, qs, k, ks, w = _indexer_inputs(rng, b, 64, l)
    k[0, 100:3000] = k[0, 50]   # thousands of exact ties
    ks[0, 100:3000] = ks[0, 50]
    lengths = np.array([6000, 4000, 700], dtype=np.int32)
    got = ops.dsa_indexer_topk(*_t(dev, q, qs, k, ks, w), topk, lengths=torch.from_numpy(lengths).to(dev),
                               offset=17).cpu().numpy()
    np.testing.assert_array_equal(got, D.indexer_topk(q, qs, k, ks, w, topk, lengths, 17))
    assert (got[2, 700:] == -1).all()


def test_indexer_all_tied_takes_lowest_indices(dev):
    """q = 0: every score is 0, every token is a candidate (radix-select path)."""
    from mosaic_amd import ops
    rng = np.random.default_rng(12)
    q, qs, k, ks, w = _indexer_inputs(rng, 1, 64, 9000)
    q[:] = 0
    got = ops.dsa_indexer_topk(*_t(dev, q, qs, k, ks, w), 512).cpu().numpy()
    assert got[0].tolist() == list(range(512))


def test_indexer_full_size_properties(dev):
    """BASELINE.json configs[4] at full size (B=8, L=131072, top-2048): indices are
    distinct, ordered by the (bit-exact) canonical scores, and no unselected
    token beats a selected one."""
    from mosaic_amd import ops
    torch.manual_seed(0)
    b, h, l, topk = 8, 64, 131072, 2048
    q = (torch.randn(b, h, 128, device=dev) * 60).clamp(-448, 448).to(torch.float8_e4m3fn)
    k = (torch.randn(b, l, 128, device=dev) * 60).clamp(-448, 448).to(torch.float8_e4m3fn)
    qs = torch.rand(b, h, device=dev) * 0.01 + 1e-3
    ks = torch.rand(b, l, device=dev) * 0.01 + 1e-3
    w = torch.randn(b, h, device=dev) * 0.01
    idx = ops.dsa_indexer_topk(q, qs, k, ks, w, topk)
    s = ops.dsa_indexer_scores(q, qs, k, ks, w)
    idx_l = idx.long()
    assert (idx_l >= 0).all() and (idx_l < l).all()
    srt = torch.sort(idx_l, dim=1).values
    assert (srt[:, 1:] != srt[:, :-1]).all()
    sel = torch.gather(s, 1, idx_l)
    assert (sel[:, 1:] <= sel[:, :-1]).all()
    mask = torch.ones_like(s, dtype=torch.bool)
    mask.scatter_(1, idx_l, False)
    best_out = torch.where(mask, s, torch.full_like(s, -float("inf"))).max(1).values
    assert (sel[:, -1] >= best_out).all()
    # spot check: one row against the oracle
    r = 5
    ref = D.indexer_topk(q[r:r + 1].view(torch.uint8).cpu().numpy(), qs[r:r + 1].cpu().numpy(),
                         k[r:r + 1].view(torch.uint8).cpu().numpy(), ks[r:r + 1].cpu().numpy(),
                         w[r:r + 1].cpu().numpy(), topk)
    np.testing.assert_array_equal(idx[r:r + 1].cpu().numpy(), ref)


def _mla(rng, b, h, n, t, sb, masked=0.0):
    q = C.round_bf16(rng.standard_normal((b, h, 576)).astype(np.float32))
    lat, ls = D.quantize_rows_e4m3(rng.standard_normal((b, n, 512 // sb, sb)) * 2.0)
    lat = lat.reshape(b, n, 512)
    rope = C.round_bf16(rng.standard_normal((b, n, 64)).astype(np.float32))
    idx = np.stack([rng.choice(n, t, replace=False) for _ in range(b)]).astype(np.int32)
    if masked:
        idx[rng.random(idx.shape) < masked] = -1
    return q, lat, ls, rope, idx


@pytest.mark.parametrize("b,h,n,t,sb,sink,masked", [(1, 128, 4096, 2048, 64, True, 0.0),
                                                     (2, 128, 3000, 2048, 512, False, 0.1),
                                                     (3, 64, 500, 300, 64, True, 0.3),
                                                     (1, 16, 100, 64, 128, True, 0.0),
                                                     (2, 32, 80, 20, 64, True, 0.2),
                                                     (2, 48, 300, 100, 64, True, 0.1),
                                                     (1, 128, 5000, 300, 64, False, 0.0),
                                                     # the config-5 timed shape: B = 8, 128 heads, top-2048
                                                     # (16 splits x 8 rows x 2 groups = 256 workgroups: 4 head tiles)
                                                     (8, 128, 8192, 2048, 64, True, 0.0),
                                                     # 48 heads, 16 rows, top-16384 (16 splits x 16 rows x 1 group
                                                     # of 3 head tiles = 256 workgroups: 3 head tiles)
                                                     (16, 48, 16400, 16384, 64, True, 0.05)])
def test_mla_fp8_vs_oracle(dev, b, h, n, t, sb, sink, masked):
    from mosaic_amd import ops
    rng = np.random.default_rng(b * 1000 + t)
    q, lat, ls, rope, idx = _mla(rng, b, h, n, t, sb, masked)
    snk = rng.standard_normal(h).astype(np.float32) if sink else None
    scale = 576 ** -0.5
    qd, latd, lsd, rd, idxd = _t(dev, q, lat, ls, rope, idx)
    out = ops.mla_sparse_decode(qd.to(torch.bfloat16), latd, lsd, rd.to(torch.bfloat16), idxd, scale,
                                None if snk is None else torch.from_numpy(snk).to(dev))
    _close(out.float().cpu().numpy(), D.mla_sparse_decode(q, lat, ls, rope, snk, idx, scale, sb))


def test_mla_wide_score_range(dev):
    """Scores rising by over a hundred nats along the token order (the rope part
    grows 300-fold): every head's running maximum moves past the lazy margin
    about six times, within a split and across splits."""
    from mosaic_amd import ops
    rng = np.random.default_rng(33)
    b, h, n, t = 2, 64, 3000, 1024
    q, lat, ls, rope, idx = _mla(rng, b, h, n, t, 64)
    ramp = np.linspace(0.2, 60.0, n).astype(np.float32)
    rope = C.round_bf16(rope * ramp[None, :, None])
    idx = np.sort(idx, axis=1).astype(np.int32)
    snk = rng.standard_normal(h).astype(np.float32)
    qd, latd, lsd, rd, idxd = _t(dev, q, lat, ls, rope, idx)
    out = ops.mla_sparse_decode(qd.to(torch.bfloat16), latd, lsd, rd.to(torch.bfloat16), idxd, 0.1,
                                torch.from_numpy(snk).to(dev))
    _close(out.float().cpu().numpy(), D.mla_sparse_decode(q, lat, ls, rope, snk, idx, 0.1, 64))


def test_mla_all_masked_row_is_zero(dev):
    from mosaic_amd import ops
    rng = np.random.default_rng(21)
    q, lat, ls, rope, idx = _mla(rng, 2, 16, 200, 64, 64)
    idx[1] = -1
    qd, latd, lsd, rd, idxd = _t(dev, q, lat, ls, rope, idx)
    out = ops.mla_sparse_decode(qd.to(torch.bfloat16), latd, lsd, rd.to(torch.bfloat16), idxd, 0.04,
                                torch.zeros(16, device=dev)).float().cpu().numpy()
    assert (out[1] == 0).all()
    _close(out[0], D.mla_sparse_decode(q, lat, ls, rope, np.zeros(16, np.float32), idx, 0.04)[0])


@pytest.mark.parametrize("d,rows,h,n,t", [(512, 4, 64, 700, 256), (576, 4, 64, 700, 256),
                                         # 4 rows x 128 heads x top-2048: 4 head tiles per workgroup
                                         (576, 4, 128, 3000, 2048)])
def test_mla_bf16_kv_vs_oracle(dev, d, rows, h, n, t):
    from mosaic_amd import ops
    rng = np.random.default_rng(d + h + t)
    nb = 2
    q = C.round_bf16(rng.standard_normal((rows, h, d)).astype(np.float32))
    kv = C.round_bf16(rng.standard_normal((nb, n, d)).astype(np.float32))
    idx = rng.integers(-1, n, size=(rows, t)).astype(np.int32)
    sink = rng.standard_normal(h).astype(np.float32)
    out = ops.mla_sparse_decode_bf16(torch.from_numpy(q).to(dev).to(torch.bfloat16),
                                     torch.from_numpy(kv).to(dev).to(torch.bfloat16),
                                     torch.from_numpy(idx).to(dev), d ** -0.5, torch.from_numpy(sink).to(dev))
    _close(out.float().cpu().numpy(), D.sparse_attn(q, kv, sink, idx, d ** -0.5, 512, rows // nb))


def test_upstream_sparse_attn_signature(dev):
    """sparse_attn(q [b,m,h,d], kv [b,n,d], sink, idx [b,m,t], scale), h < 16 padded (inference_kernel.py:355-368)."""
    from mosaic_amd.kernels.dsa import sparse_attn, sparse_attn_fused
    rng = np.random.default_rng(31)
    b, m, h, n, t, d = 2, 3, 8, 300, 128, 512
    q = C.round_bf16(rng.standard_normal((b, m, h, d)).astype(np.float32))
    kv = C.round_bf16(rng.standard_normal((b, n, d)).astype(np.float32))
    idx = rng.integers(-1, n, size=(b, m, t)).astype(np.int32)
    sink = rng.standard_normal(h).astype(np.float32)
    T = lambda a: torch.from_numpy(a).to(dev)
    o = sparse_attn(T(q).to(torch.bfloat16), T(kv).to(torch.bfloat16), T(sink), T(idx), d ** -0.5)
    assert o.shape == (b, m, h, d) and o.dtype == torch.bfloat16
    ref = D.sparse_attn(q.reshape(b * m, h, d), kv, sink, idx.reshape(b * m, t), d ** -0.5, 512, m)
    _close(o.float().cpu().numpy().reshape(b * m, h, d), ref)
    o2 = sparse_attn_fused(T(q[0]).to(torch.bfloat16), T(kv[0]).to(torch.bfloat16), T(sink), T(idx[0]), d ** -0.5)
    _close(o2.float().cpu().numpy(), D.sparse_attn(q[0], kv[:1], sink, idx[0], d ** -0.5, 512, m))
    with pytest.raises(ValueError, match="512"):
        sparse_attn_fused(T(q[0, :, :, :320]).to(torch.bfloat16).contiguous(),
                          T(kv[0, :, :320]).to(torch.bfloat16).contiguous(), T(sink), T(idx[0]), 0.1)


@pytest.mark.parametrize("s,h,n,t,d,masked", [(3, 16, 300, 128, 64, 0.1), (2, 32, 1000, 512, 128, 0.0),
                                              (4, 64, 700, 640, 256, 0.3), (1, 16, 64, 5, 128, 0.0),
                                              (2, 48, 2000, 2048, 256, 0.05), (5, 20, 90, 33, 64, 0.5)])
def test_sparse_attn_fused_small_head_dims(dev, s, h, n, t, d, masked):
    """sparse_attn_fused at the reference's other head dims (mosaicvm/kernels/dsa_sparse.py:92-110:
    d in {64, 128, 256}; V = K): masked picks, a ragged last block, fewer picks
    than one 32-token block, heads padded to 16 (20 -> 32), every row's sink,
    against the oracle's sparse_attn (bf16 probabilities in the value product)."""
    from mosaic_amd.kernels.dsa import sparse_attn_fused
    rng = np.random.default_rng(s * 100 + d + t)
    q = C.round_bf16(rng.standard_normal((s, h, d)).astype(np.float32))
    kv = C.round_bf16(rng.standard_normal((n, d)).astype(np.float32))
    idx = np.stack([rng.choice(n, t, replace=t > n) for _ in range(s)]).astype(np.int32)
    idx[rng.random(idx.shape) < masked] = -1
    sink = rng.standard_normal(h).astype(np.float32)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    o = sparse_attn_fused(T(q).to(torch.bfloat16), T(kv).to(torch.bfloat16), T(sink), T(idx), d ** -0.5)
    assert o.shape == (s, h, d) and o.dtype == torch.bfloat16
    _close(o.float().cpu().numpy(), D.sparse_attn(q, kv[None], sink, idx, d ** -0.5, d, s))


def test_sparse_attn_small_all_masked_and_no_sink(dev):
    """A row with no valid pick gives 0; without a sink the denominator is the
    picks' sum alone (the oracle with sink None)."""
    from mosaic_amd import ops
    rng = np.random.default_rng(7)
    s, h, n, t, d = 3, 16, 200, 96, 128
    q = C.round_bf16(rng.standard_normal((s, h, d)).astype(np.float32))
    kv = C.round_bf16(rng.standard_normal((1, n, d)).astype(np.float32))
    idx = rng.integers(0, n, size=(s, t)).astype(np.int32)
    idx[1] = -1
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    o = ops.sparse_attn_bf16(T(q).to(torch.bfloat16), T(kv).to(torch.bfloat16), T(idx), 0.09).float().cpu().numpy()
    assert (o[1] == 0).all()
    ref = D.sparse_attn(q, kv, None, idx, 0.09, d, s)
    _close(o[[0, 2]], ref[[0, 2]])


def _indexer_drop_in_case(rng, bsz, seqlen, h, n_cache):
    q, qs = D.quantize_rows_e4m3(rng.standard_normal((bsz * seqlen, h, 128)))
    k, ks = D.quantize_rows_e4m3(rng.standard_normal((bsz, n_cache, 128)))
    w = (rng.standard_normal((bsz * seqlen, h)) * (128 ** -0.5) * (h ** -0.5)).astype(np.float32)
    return q, qs, k, ks, w


def test_indexer_drop_in_decode(dev):
    """Indexer scoring at decode (start_pos > 0, seqlen 1): min(index_topk, end_pos // 4)
    picks over the compressed cache, + offset (.mosaicvm/source/inference_model.py:430-439);
    the cache is longer than end_pos // 4 and is read in place (a strided slice)."""
    from mosaic_amd.kernels.dsa import Indexer
    rng = np.random.default_rng(31)
    bsz, h, start = 2, 64, 4000
    n_c = (start + 1) // 4
    q, qs, k, ks, w = _indexer_drop_in_case(rng, bsz, 1, h, n_c + 50)
    ix = Indexer(index_topk=512)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    got = ix.score_topk(T(q).view(torch.float8_e4m3fn).reshape(bsz, 1, h, 128), T(qs).reshape(bsz, 1, h),
                        T(w).reshape(bsz, 1, h), T(k).view(torch.float8_e4m3fn), T(ks), start, 128).cpu().numpy()
    ref = D.indexer_topk(q, qs, k[:, :n_c], ks[:, :n_c], w, 512, None, 128)
    np.testing.assert_array_equal(got.reshape(bsz, 512), ref)


def test_indexer_drop_in_prefill_causal(dev):
    """Indexer scoring at start_pos 0: position i sees the first (i + 1) // 4
    compressed entries, masked picks are -1, valid ones + offset (the query
    rows of one sequence share its cache)."""
    from mosaic_amd.kernels.dsa import Indexer
    rng = np.random.default_rng(32)
    bsz, seqlen, h = 2, 96, 32
    n_c = seqlen // 4
    q, qs, k, ks, w = _indexer_drop_in_case(rng, bsz, seqlen, h, n_c)
    ix = Indexer(index_topk=2048)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    got = ix.score_topk(T(q).view(torch.float8_e4m3fn).reshape(bsz, seqlen, h, 128), T(qs).reshape(bsz, seqlen, h),
                        T(w).reshape(bsz, seqlen, h), T(k).view(torch.float8_e4m3fn), T(ks), 0, 7).cpu().numpy()
    assert got.shape == (bsz, seqlen, n_c)
    kk = np.repeat(k, seqlen, axis=0)
    kss = np.repeat(ks, seqlen, axis=0)
    lengths = np.tile((np.arange(1, seqlen + 1) // 4).astype(np.int32), bsz)
    ref = D.indexer_topk(q, qs, kk, kss, w, n_c, lengths, 7)
    np.testing.assert_array_equal(got.reshape(bsz * seqlen, n_c), ref)
    assert (got[:, 2, :] == -1).all() and (got[:, 3, 1:] == -1).all() and got[0, 3, 0] == 7


@pytest.mark.parametrize("h,d,ctx,topk,dv", [(64, 128, 4096, 256, 128), (8, 64, 1000, 512, 512), (16, 128, 700, 700, 64)])
def test_dsa_decode_attention_vs_oracle(dev, h, d, ctx, topk, dv):
    """dsa_decode_attention (mosaicvm/kernels/dsa_attention.py:113-154; the
    reference's tests/test_dsa_parity.py shape first): per-head picks
    bit-exact in (score desc, position asc) order, output within 2e-2."""
    from mosaic_amd.kernels.dsa import dsa_decode_attention
    rng = np.random.default_rng(h + ctx)
    bf = lambda *sh: torch.from_numpy(rng.standard_normal(sh).astype(np.float32)).to(torch.bfloat16)
    q, k, v = bf(h, d), bf(ctx, h, d), bf(ctx, h, dv)
    k[10:20] = k[5]  # exact score ties within every head
    out, idx = dsa_decode_attention(q.to(dev), k.to(dev), v.to(dev), topk)
    out_ref, idx_ref = D.head_topk_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), topk, d ** -0.5)
    np.testing.assert_array_equal(idx.cpu().numpy(), idx_ref)
    _close(out.float().cpu().numpy(), out_ref)


def _kv_bf16_rows(rng, rows, d, rope=64):
    x = rng.standard_normal((rows, d)).astype(np.float32)
    mags = np.float32(2.0) ** rng.integers(-20, 12, size=(rows, d // 64)).astype(np.float32)
    x = x * np.repeat(mags, 64, axis=1)[:, :d]
    x[0, :64] = 0.0
    x[1, 5] = 448.0 * 2.0 ** -3
    return C.round_bf16(x)


@pytest.mark.parametrize("d", [512, 576])
def test_kv_write_bf16_cache_bit_exact(dev, d):
    from mosaic_amd import ops
    rng = np.random.default_rng(d + 1)
    rows, n = 37, 50
    kv = _kv_bf16_rows(rng, rows, d)
    slots = rng.permutation(n)[:rows].astype(np.int32)
    slots[3] = -1      # skipped
    slots[4] = n + 7   # out of range: skipped
    cache = torch.full((n, d), 7.0, dtype=torch.bfloat16, device=dev)
    ops.dsa_kv_write(torch.from_numpy(kv).to(dev).to(torch.bfloat16), cache, torch.from_numpy(slots).to(dev))
    got = cache.float().cpu().numpy()
    want = np.full((n, d), 7.0, np.float32)
    rows_ok = [(r, s) for r, s in enumerate(slots) if 0 <= s < n]
    for r, s in rows_ok:
        want[s] = D.kv_cache_row(kv[r:r + 1])[0]
    np.testing.assert_array_equal(got, want)


def test_kv_write_fp8_cache_bit_exact(dev):
    from mosaic_amd import ops
    rng = np.random.default_rng(3)
    rows, n = 20, 24
    kv = _kv_bf16_rows(rng, rows, 576)
    slots = np.arange(rows, dtype=np.int32)[::-1].copy()
    codes = torch.zeros(n, 512, dtype=torch.uint8, device=dev)
    scales = torch.zeros(n, 8, dtype=torch.float32, device=dev)
    rope = torch.zeros(n, 64, dtype=torch.bfloat16, device=dev)
    ops.dsa_kv_write(torch.from_numpy(kv).to(dev).to(torch.bfloat16), (codes, scales, rope),
                     torch.from_numpy(slots).to(dev))
    wc, ws, _ = D.kv_act_quant(kv[:, :512])
    np.testing.assert_array_equal(codes.cpu().numpy()[slots], wc)
    np.testing.assert_array_equal(scales.cpu().numpy()[slots], ws)
    np.testing.assert_array_equal(rope.float().cpu().numpy()[slots], kv[:, 512:])


def test_decode_indices_match_oracle(dev):
    from mosaic_amd import ops
    pos = np.array([0, 1, 5, 126, 127, 128, 129, 1000, 65535], dtype=np.int32)
    got = ops.dsa_decode_indices(torch.from_numpy(pos).to(dev), 128, nc=300, ratio=4).cpu().numpy()
    np.testing.assert_array_equal(got, D.decode_indices(pos, 128, nc=300, ratio=4, offset=128))
    rng = np.random.default_rng(4)
    cidx = rng.integers(-1, 900, size=(len(pos), 512)).astype(np.int32)
    got2 = ops.dsa_decode_indices(torch.from_numpy(pos).to(dev), 128, torch.from_numpy(cidx).to(dev)).cpu().numpy()
    np.testing.assert_array_equal(got2, D.decode_indices(pos, 128, cidx=cidx, nc=512))


@pytest.mark.parametrize("fp8", [False, True])
def test_decode_step_against_oracle(dev, fp8):
    """A decode step of the DSA layer (V4: 64 heads, head_dim 512, window 128,
    top-512 compressed picks; FP8: the 512 + 64 MLA cache): write the position's
    kv into the ring, gather window + picks, attend with the sink."""
    from mosaic_amd.kernels.dsa import DecodeKVCache
    rng = np.random.default_rng(40 + fp8)
    d = 576 if fp8 else 512
    h, win, ncomp, t, p = 64, 128, 1024, 512, 700
    cache = DecodeKVCache(head_dim=d, window=win, n_compressed=ncomp, fp8=fp8, device=dev)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    hist = C.round_bf16(rng.standard_normal((win, d)).astype(np.float32))
    ring_pos = np.arange(p - win + 1, p)                      # positions already in the ring
    cache.write_window(T(hist[:1]).to(torch.bfloat16), 0)      # exercised once, then overwritten
    for j, q_ in enumerate(ring_pos):
        cache.write_window(T(hist[j:j + 1]).to(torch.bfloat16), int(q_))
    comp = C.round_bf16(rng.standard_normal((ncomp, d)).astype(np.float32))
    cache.write_compressed(T(comp).to(torch.bfloat16))
    kv_new = C.round_bf16(rng.standard_normal((1, d)).astype(np.float32))
    q = C.round_bf16(rng.standard_normal((1, h, d)).astype(np.float32))
    sink = rng.standard_normal(h).astype(np.float32)
    picks = rng.choice(ncomp, t, replace=False).astype(np.int32) + win
    picks[::7] = -1
    scale = d ** -0.5
    o = cache.step(T(q).to(torch.bfloat16), T(kv_new).to(torch.bfloat16), p, scale, T(sink), T(picks[None]))
    # oracle cache: ring rows by slot, compressed rows after them
    ref_cache = np.zeros((win + ncomp, d), np.float32)
    for j, q_ in enumerate(ring_pos):
        ref_cache[q_ % win] = D.kv_cache_row(hist[j:j + 1])[0]
    ref_cache[p % win] = D.kv_cache_row(kv_new)[0]
    ref_cache[win:] = D.kv_cache_row(comp)
    idx = D.decode_indices([p], win, cidx=picks[None], nc=t)
    ref = D.sparse_attn(q, ref_cache[None], sink, idx, scale, dv=512)
    _close(o.float().cpu().numpy(), ref)


class _Compressor(torch.nn.Module):
    """A stand-in for the model's compressor (not on this build's path): every
    completed group of `ratio` positions writes one bf16 row, a fixed
    projection of the group's last token (rows depend on x and on the position)."""

    def __init__(self, dim, hd, n_rows, ratio, dev, seed):
        super().__init__()
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        self.wc = (torch.randn(dim, hd, generator=g, device=dev) * dim ** -0.5)
        self.kv_cache = torch.zeros(n_rows, hd, dtype=torch.bfloat16, device=dev)
        self.ratio = ratio
        self.calls = []

    def forward(self, x, start_pos):
        self.calls.append((x.shape[0], start_pos))
        for p in range(start_pos, start_pos + x.shape[0]):
            if (p + 1) % self.ratio == 0:
                self.kv_cache[p // self.ratio] = (x[p - start_pos].float() @ self.wc * 3.0).to(torch.bfloat16)


def test_indexer_forward_reference_signature(dev):
    """Indexer.forward(x, qr, freqs, offset, start_pos) (mosaicvm/model/dsa_layers.py:281-321):
    a 40-token prefill, then four decode steps.  wq_b runs on the FP8 W8A16
    linear and weights_proj on the router GEMV; the caller's rope, Hadamard and
    compressor are applied in the reference's order; the FP8 key cache is
    quantized incrementally.  Indices are bit-exact against the oracle's FP8
    indexer fed the same projected q (the rope / Hadamard functions replayed on
    the GPU's wq_b output), the oracle's act_quant of q and of the compressor's
    rows, and the oracle's exact-rounded weights_proj."""
    from mosaic_amd.kernels.dsa import Indexer
    from mosaic_amd.kernels.fp8 import fp8_linear
    from oracle import linear as L
    from oracle import moe as MO
    import scipy.linalg
    rng = np.random.default_rng(41)
    h, hd, dim, qlr, ratio, max_seq = 64, 128, 512, 256, 4, 256
    wq = (rng.standard_normal((h * hd, qlr)) * 0.05).astype(np.float32)
    wq_codes, wq_s = L.quantize_fp8_weight_128(wq)
    wp = C.round_bf16((rng.standard_normal((h, dim)) * 0.05).astype(np.float32))
    freqs = torch.from_numpy(rng.uniform(0.5, 1.5, size=(max_seq, 64)).astype(np.float32)).to(dev)
    had = torch.from_numpy((scipy.linalg.hadamard(hd) / np.sqrt(hd)).astype(np.float32)).to(dev)
    rotary = lambda qp, f: (qp.float() * f[:, None, :]).to(torch.bfloat16)
    hadamard = lambda q: (q.float() @ had).to(torch.bfloat16)
    comp = _Compressor(dim, hd, max_seq // ratio, ratio, dev, seed=5)
    ix = Indexer(n_heads=h, head_dim=hd, index_topk=6, compress_ratio=ratio, max_seq_len=max_seq, rotary=rotary,
                 hadamard=hadamard, compressor=comp, device=dev)
    ix.wq_b = torch.from_numpy(wq_codes).to(dev).view(torch.float8_e4m3fn)
    ix.wq_b_scale = torch.from_numpy(wq_s).to(dev)
    ix.weights_proj = torch.from_numpy(wp).to(dev).to(torch.bfloat16)
    pos = 0
    for s in (40, 1, 1, 1, 1):
        x = torch.from_numpy(rng.standard_normal((s, dim)).astype(np.float32)).to(dev).to(torch.bfloat16)
        qr = torch.from_numpy(rng.standard_normal((s, qlr)).astype(np.float32)).to(dev).to(torch.bfloat16)
        got = ix(x, qr, freqs, 1000, pos).cpu().numpy()
        end = pos + s
        n_c = end // ratio
        assert comp.calls[-1] == (s, pos) and got.shape == (s, min(6, n_c))
        # the oracle's view of the same call
        q = fp8_linear(qr, ix.wq_b, ix.wq_b_scale).view(s, h, hd)
        q = hadamard(torch.cat([q[..., :-64], rotary(q[..., -64:], freqs[pos:end])], -1))
        qc, qs = C.act_quant(q.float().cpu().numpy().reshape(s * h, hd), hd, "amax")
        kc, ks = C.act_quant(comp.kv_cache[:n_c].float().cpu().numpy(), hd, "amax")
        np.testing.assert_array_equal(ix.k_fp8[:n_c].cpu().numpy(), kc)
        w = (MO.router_logits(x.float().cpu().numpy(), wp) * np.float32(hd ** -0.5 * h ** -0.5)).astype(np.float32)
        if pos == 0 or s > 1:
            lengths = ((np.arange(1, s + 1) + pos) // ratio).astype(np.int32)
        else:
            lengths = np.full(s, n_c, dtype=np.int32)
        ref = D.indexer_topk(qc.reshape(s, h, hd), qs.reshape(s, h), np.repeat(kc[None], s, 0),
                             np.repeat(ks.reshape(1, n_c), s, 0), w, min(6, n_c), lengths, 1000)
        np.testing.assert_array_equal(got, ref)
        pos = end
    assert (got >= 1000).all()
