"""The reference-signature drop-ins (``mosaic_amd.kernels``) against the CPU
oracle, written like the reference's own tests (``tests/test_fp4_source.py``,
``tests/test_mxint_gemm.py``, ``tests/test_moe_layout.py``,
``tests/test_emit_tiles.py``, ``tests/test_skinny_fp4.py``)."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import codecs as C
from oracle import linear as L
from oracle import moe as MO

pytestmark = pytest.mark.gpu


def _close(got, ref, tol=2e-2):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref) / np.maximum(1.0, np.abs(ref))
    assert err.max() <= tol, f"max scaled err {err.max():.3e}"


def test_pack_and_dequant_match_oracle(dev):
    from mosaic_amd.kernels.fp4_source import pack_mxfp4_nk
    from mosaic_amd.kernels.mxfp4 import dequant_mxfp4, pack_mxfp4
    torch.manual_seed(0)
    w = torch.randn(64, 256, dtype=torch.bfloat16)
    p_ref, s_ref = C.quantize_mxfp4_floor(w.float().numpy())
    for fn in (pack_mxfp4, pack_mxfp4_nk):
        p, s = fn(w.to(dev))
        assert p.dtype == torch.uint8 and s.dtype == torch.float8_e8m0fnu
        assert p.shape == (64, 128) and s.shape == (64, 8)
        np.testing.assert_array_equal(p.cpu().numpy(), p_ref)
        np.testing.assert_array_equal(s.view(torch.uint8).cpu().numpy(), s_ref)
    dq = dequant_mxfp4(p, s).float().cpu().numpy()
    np.testing.assert_array_equal(dq, C.dequant_mxfp4(p_ref, s_ref))


def test_act_quant_ref_matches_official_math(dev):
    """tests/test_fp4_source.py:34-41."""
    from mosaic_amd.kernels.fp4_source import act_quant_ref
    torch.manual_seed(0)
    x = torch.randn(8, 4096, dtype=torch.bfloat16)
    y, s = act_quant_ref(x.to(dev), 128)
    y0, s0 = C.act_quant(x.float().numpy(), 128, "pow2")
    np.testing.assert_array_equal(s.cpu().numpy(), s0)
    np.testing.assert_array_equal(y.view(torch.uint8).cpu().numpy(), y0)


def test_act_quant_legacy_phase27_differs_on_straddling_blocks(dev):
    """tests/test_fp4_source.py:45-63: the legacy amax/448 scale differs from the pow2 one on
    straddling blocks; both match the oracle bit for bit, an all-zero block included."""
    from mosaic_amd.kernels.fp4_source import act_quant_legacy_phase27, act_quant_ref
    vals = [0.0, 1e-5, -1e-5, 1e-4, 448.0, -448.0, 1.0, 2.0 ** -60]
    vals += [2.0 ** e * 448.0 for e in (-10, -1, 0, 4)]
    vals += [2.0 ** e * 448.0 * 1.0000001 for e in (-10, -1, 0, 4)]
    x = torch.zeros(1, 128 * len(vals), dtype=torch.float32)
    for i, v in enumerate(vals):
        x[0, 128 * i + 7] = v
    xb = x.to(torch.bfloat16)
    y, s = act_quant_ref(xb.to(dev), 128)
    yl, sl = act_quant_legacy_phase27(xb.to(dev), 128)
    assert not torch.equal(sl, s)
    q_ref, s_ref = C.act_quant(xb.float().numpy(), 128, "legacy")
    np.testing.assert_array_equal(sl.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(yl.view(torch.uint8).cpu().numpy(), q_ref)
    with pytest.raises(ValueError):
        act_quant_legacy_phase27(xb.to(dev)[:, :100], 128)


@pytest.mark.parametrize("m,k,n", [(1, 128, 16), (2, 256, 32), (8, 128, 16), (3, 7168, 256)])
def test_a8_gemvs_vs_source_linear(dev, m, k, n):
    """tests/test_fp4_source.py:76-88 / tests/test_mxint_gemm.py:32-55: every A8 GEMV vs the source oracle."""
    from mosaic_amd import ops
    from mosaic_amd.kernels import fp4_source, mxint, qpa_mma, xsimt
    rng = np.random.default_rng(m + k + n)
    w = (rng.standard_normal((n, k)) / math.sqrt(k)).astype(np.float32)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(torch.bfloat16)
    p, s = C.quantize_mxfp4_floor(torch.from_numpy(w).to(torch.bfloat16).float().numpy())
    ref = L.mx_linear_a8(x.float().numpy(), p, s)
    P, S, X = torch.from_numpy(p).to(dev), torch.from_numpy(s).to(dev), x.to(dev)
    pre = xsimt.prepack_xsimt(P, S)
    outs = [xsimt.xsimt_gemm(X, P, S, n), xsimt.xsimt_gemm(X, P, S, n, prepacked=pre),
            qpa_mma.qpa_mma_gemm(X, P, S, n), mxint.mxint_dp4a_gemm(X, P, S, n), mxint.mxint_imma_gemm(X, P, S, n),
            fp4_source.reference_fp4_linear_source_semantics(X, P, S),
            xsimt.xsimt_gemm(X, P, S, n, prequant=ops.act_quant(X, 128, "pow2"))]
    for o in outs:
        assert o.dtype == torch.bfloat16 and o.shape == (m, n)
        _close(o.float().cpu().numpy(), ref)
    p2, s2 = xsimt.inverse_prepack_xsimt(pre)
    assert torch.equal(p2, P) and torch.equal(s2, S)
    with pytest.raises(ValueError, match="n_out"):
        xsimt.xsimt_gemm(X, P, S, n + 16)


def _bank(rng, e, h, inter):
    q = lambda r, c: C.quantize_mxfp4_ceil((rng.standard_normal((r, c)) * 0.05).astype(np.float32))
    gu = [q(2 * inter, h) for _ in range(e)]
    d = [q(h, inter) for _ in range(e)]
    return (np.stack([a[0] for a in gu]), np.stack([a[1] for a in gu]), np.stack([a[0] for a in d]),
            np.stack([a[1] for a in d]))


@pytest.mark.parametrize("m,k", [(1, 6), (5, 8), (12, 4)])
def test_fused_moe_mxint_vs_oracle(dev, m, k, monkeypatch):
    from mosaic_amd.kernels import exact_moe, mxint, qpa_mma
    rng = np.random.default_rng(m * 10 + k)
    e, h, inter = 16, 256, 128
    gp, gs, dp, ds = _bank(rng, e, h, inter)
    x = torch.from_numpy(rng.standard_normal((m, h)).astype(np.float32)).to(torch.bfloat16)
    ids = np.stack([rng.choice(e, k, replace=False) for _ in range(m)])
    w = rng.random((m, k)).astype(np.float32)
    ref = MO.moe_layer_a8(x.float().numpy(), ids, w, gp, gs, dp, ds, swiglu_limit=10.0)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    bank = mxint.prepack_expert_bank_mxint(T(gp), T(gs), packed_d=T(dp), scale_d=T(ds))
    outs = [mxint.fused_moe_mxint(x.to(dev), T(ids), T(w), bank=bank),
            mxint.fused_moe_mxint(x.to(dev), T(ids), T(w), T(gp), T(gs), T(dp), T(ds)),
            qpa_mma.fused_moe_qpa(x.to(dev), T(ids), T(w), T(gp), T(gs), T(dp), T(ds)),
            exact_moe.exact_moe(x.to(dev), T(ids), T(w), T(gp), T(gs), T(dp), T(ds))]
    for o in outs:
        _close(o.float().cpu().numpy(), ref)
    monkeypatch.setenv("MOSAICVM_EXACT_TARGET", "0")
    with pytest.raises(RuntimeError, match="MOSAICVM_EXACT_TARGET"):
        exact_moe.exact_moe(x.to(dev), T(ids), T(w), T(gp), T(gs), T(dp), T(ds))


def test_layout_assignments_kat(dev):
    """tests/test_moe_layout.py:13-24."""
    from mosaic_amd.kernels.moe_layout import layout_assignments
    expert_ids = torch.tensor([3, 0, 3, 1], device=dev, dtype=torch.int64)
    sorted_ids, perm, offsets, counts = layout_assignments(expert_ids, n_experts=4)
    assert counts.tolist() == [1, 1, 0, 2]
    assert int(offsets[-1].item()) == 4
    for ex in range(4):
        seg = sorted_ids[int(offsets[ex]):int(offsets[ex + 1])]
        assert (seg == ex).all()
    assert perm.tolist() == [1, 3, 0, 2]
    with pytest.raises(ValueError, match="CUDA"):
        layout_assignments(expert_ids.cpu(), 4)


@pytest.mark.parametrize("block_m", [1, 8, 16])
def test_emit_tiles_kat(dev, block_m):
    """tests/test_emit_tiles.py:14-34."""
    from mosaic_amd.kernels.w4a16_grouped import emit_tiles
    counts = torch.tensor([0, 1, block_m - 1, block_m, block_m + 1, 3 * block_m + 2], device=dev, dtype=torch.int32)
    ei, ms, nt, rows = emit_tiles(counts, block_m=block_m, max_tiles=64)
    nt = int(nt.item())
    exp = [(e_, t * block_m, min(block_m, c - t * block_m)) for e_, c in enumerate(counts.tolist())
           for t in range((c + block_m - 1) // block_m)]
    assert nt == len(exp)
    assert list(zip(ei[:nt].tolist(), ms[:nt].tolist(), rows[:nt].tolist())) == exp
    # a cap below the total: n_tiles is still the true total (tile_offsets[-1:] in the
    # reference), and the entries that fit are the first ones of the full list
    cap = len(exp) - 2
    ei, ms, nt, rows = emit_tiles(counts, block_m=block_m, max_tiles=cap)
    assert int(nt.item()) == len(exp) and ei.numel() == cap
    assert list(zip(ei.tolist(), ms.tolist(), rows.tolist())) == exp[:cap]


@pytest.mark.parametrize("m", [1, 3, 8])
def test_skinny_kn_vs_dequant_matmul(dev, m):
    """tests/test_skinny_fp4.py:16-25: x @ dequant_mxfp4 on the KN layout."""
    from mosaic_amd.kernels.mxfp4 import pack_mxfp4
    from mosaic_amd.kernels.skinny_fp4 import skinny_mxfp4_gemm
    torch.manual_seed(m)
    k, n = 512, 384
    w = torch.randn(k, n, dtype=torch.bfloat16)
    p, s = pack_mxfp4(w.to(dev))
    x = torch.randn(m, k, dtype=torch.bfloat16)
    y = skinny_mxfp4_gemm(x.to(dev), p, s, n).float().cpu().numpy()
    ref = C.round_bf16((x.float().numpy().astype(np.float64) @ C.dequant_mxfp4(
        p.cpu().numpy(), s.view(torch.uint8).cpu().numpy()).astype(np.float64)).astype(np.float32))
    _close(y, ref)


def test_upstream_fp8_ops_vs_oracle(dev):
    from mosaic_amd.kernels import fp8
    rng = np.random.default_rng(4)
    m, n, k = 5, 384, 1024
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    xf = rng.standard_normal((m, k)).astype(np.float32)
    bq, bs = L.quantize_fp8_weight_128(w)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    # upstream act_quant without scale_fmt: s = max(amax, 1e-4)/448
    q, s = fp8.act_quant(T(xf))
    q0, s0 = C.act_quant(xf, 128, "amax")
    np.testing.assert_array_equal(s.cpu().numpy(), s0)
    np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), q0)
    ref = L.fp8_block_gemm(q0, s0, bq, bs, out_bf16=False)
    prev = torch.get_default_dtype()
    try:
        torch.set_default_dtype(torch.float32)
        c32 = fp8.fp8_gemm(q, s, T(bq).view(torch.float8_e4m3fn), T(bs))
    finally:
        torch.set_default_dtype(prev)
    _close(c32.cpu().numpy(), ref, 1e-4)
    hf = fp8.w8a8_block_fp8_matmul(q, T(bq).view(torch.float8_e4m3fn), s, T(bs), [128, 128], torch.float32)
    _close(hf.cpu().numpy(), ref, 1e-4)
    # pow2 act scales in e8m0 -> fp4_gemm against the A8 MXFP4 oracle
    qp, sp = fp8.act_quant(T(xf), 128, scale_fmt="ue8m0", scale_dtype=torch.float8_e8m0fnu)
    assert sp.dtype == torch.float8_e8m0fnu
    wp, ws = C.quantize_mxfp4_ceil(w)
    out = fp8.fp4_gemm(qp, sp, T(wp), T(ws))
    _close(out.float().cpu().numpy(), L.mx_linear_a8(xf, wp, ws))
    # a scale that is not a power of two is caught on the device (no host sync):
    # exactly the rows that carry one come out NaN
    sp32 = fp8._scales_f32(sp).clone()
    sp32[2, 1] *= 1.5
    sp32[4, 0] = -sp32[4, 0]
    bad = fp8.fp4_gemm(qp, sp32, T(wp), T(ws)).float().cpu().numpy()
    assert np.isnan(bad[[2, 4]]).all()
    np.testing.assert_array_equal(bad[[0, 1, 3]], out.float().cpu().numpy()[[0, 1, 3]])
    # the MXT16 prepack of (wp, ws) is reused while they live and are unmodified
    from mosaic_amd.kernels import _prepack_cache
    wt, wst = T(wp), T(ws)
    assert _prepack_cache.mxt16(wt, wst) is _prepack_cache.mxt16(wt, wst)
    w1 = _prepack_cache.mxt16(wt, wst)
    wt.view(torch.uint8)[0, 0] ^= 0x11
    assert _prepack_cache.mxt16(wt, wst) is not w1
    # inplace quant-dequant
    xt = T(xf).to(torch.bfloat16)
    x0 = xt.clone()
    fp8.act_quant(xt, 128, scale_fmt="ue8m0", inplace=True)
    cq, cs = C.act_quant(x0.float().cpu().numpy(), 128, "pow2")
    want = C.round_bf16((C.e4m3_decode(cq).reshape(m, -1, 128) * cs[..., None]).reshape(m, k))
    np.testing.assert_array_equal(xt.float().cpu().numpy(), want)


def test_fp8_linear_w8a16_vs_dequant_matmul(dev):
    from mosaic_amd.kernels import fp8
    rng = np.random.default_rng(6)
    m, n, k = 7, 256, 512
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    bq, bs = L.quantize_fp8_weight_128(w)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(torch.bfloat16)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    y = fp8.fp8_linear(x.to(dev), T(bq).view(torch.float8_e4m3fn), T(bs)).float().cpu().numpy()
    wd = C.round_bf16(C.e4m3_decode(bq) * np.repeat(np.repeat(bs, 128, 0), 128, 1)[:n, :k])
    _close(y, C.round_bf16((x.float().numpy().astype(np.float64) @ wd.T.astype(np.float64)).astype(np.float32)))
    np.testing.assert_array_equal(fp8.dequant_fp8(T(bq), T(bs)).float().cpu().numpy(), wd)


def _swiglu_quant_oracle(gu: np.ndarray, w: np.ndarray | None, inter: int, limit: float):
    """oracle z = bf16(swiglu * w) and its act_quant_ref, plus a mask of the values
    whose fp32 z lies within 8 ulp of a bf16 rounding midpoint (there a 1-ulp
    difference between two exp implementations may pick the other bf16 value)."""
    z = MO.swiglu(gu[:, :inter], gu[:, inter:], limit)
    if w is not None:
        z = (z * w[:, None]).astype(np.float32)
    low = z.view(np.uint32) & 0xFFFF
    near = np.abs(low.astype(np.int64) - 0x8000) <= 8
    q, s = C.act_quant(C.round_bf16(z), 128, "pow2")
    return q, s, near


@pytest.mark.parametrize("a,inter,scale,limit,weighted", [
    (24, 256, 3.0, 10.0, True),    # tests/test_mxint_epilogue.py:87-104
    (8, 128, 30.0, 10.0, True),    # clamp engaged, :107-117
    (37, 2048, 2.0, 10.0, True),   # config geometry (inter 2048)
    (5, 384, 4.0, 0.0, False),     # no clamp, no route weight (ops entry)
])
def test_mxint_swiglu_quant_down_vs_oracle(dev, a, inter, scale, limit, weighted):
    from mosaic_amd import ops
    from mosaic_amd.kernels.mxint import mxint_swiglu_quant_down
    rng = np.random.default_rng(a * 7 + inter)
    gu = torch.from_numpy((rng.standard_normal((a, 2 * inter)) * scale).astype(np.float32)).to(torch.bfloat16)
    w = (rng.random(a) * 1.5).astype(np.float32) if weighted else None
    q_ref, s_ref, near = _swiglu_quant_oracle(gu.float().numpy(), w, inter, limit)
    if limit > 0:
        q, s = mxint_swiglu_quant_down(gu.to(dev), torch.from_numpy(w).to(dev), inter, limit)
    else:
        q, s = ops.swiglu_act_quant(gu.to(dev), None, inter, 0.0)
    assert q.dtype == torch.float8_e4m3fn and tuple(s.shape) == (a, inter // 128)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    got = q.view(torch.uint8).cpu().numpy()
    np.testing.assert_array_equal(got[~near], q_ref[~near])
    diff = np.abs(C.e4m3_decode(got[near]) - C.e4m3_decode(q_ref[near]))
    assert (diff <= np.abs(C.e4m3_decode(q_ref[near])) * 2.0 ** -2 + 2.0 ** -9).all()
    with pytest.raises(ValueError):
        mxint_swiglu_quant_down(gu.to(dev), None, inter, 0.0)


@pytest.mark.parametrize("k_tok,top_k,h,e", [(5, 6, 320, 16), (64, 8, 7168, 256), (1, 8, 7168, 256)])
def test_mxint_routed_reduce_bitwise(dev, k_tok, top_k, h, e):
    """tests/test_mxint_epilogue.py:120-148: packed-order partials summed per token in
    ascending expert id, fp32, one bf16 rounding -- bit-exact against the oracle's
    combine over the oracle's stable layout."""
    from mosaic_amd.kernels.mxint import mxint_routed_reduce
    rng = np.random.default_rng(k_tok + h)
    ids = np.stack([rng.permutation(e)[:top_k] for _ in range(k_tok)])
    a = k_tok * top_k
    yd = torch.from_numpy((rng.standard_normal((a, h)) * 2.0).astype(np.float32)).to(torch.bfloat16)
    _, perm, _, _ = MO.layout_assignments(ids.reshape(-1), e)
    row_of_flat = np.empty(a, dtype=np.int64)
    row_of_flat[perm] = np.arange(a)
    slot_rows = row_of_flat.reshape(k_tok, top_k)
    order = np.argsort(ids, axis=1, kind="stable")
    ydf = yd.float().numpy()
    partial = {(t, s): ydf[slot_rows[t, s]] for t in range(k_tok) for s in range(top_k)}
    ref = C.round_bf16(MO._combine(k_tok, h, ids, partial, None))
    T = lambda v: torch.from_numpy(np.ascontiguousarray(v)).to(dev)
    got = mxint_routed_reduce(yd.to(dev), T(slot_rows), T(order), h)
    assert got.dtype == torch.bfloat16 and tuple(got.shape) == (k_tok, h)
    np.testing.assert_array_equal(got.float().cpu().numpy(), ref)


def test_pack_gate_up_mxfp4_matches_packing_the_concatenation(dev):
    """kernels/skinny_fp4.py:231-234: gate|up concatenated along N, then the floor packer;
    the result feeds fused_moe_skinny's KN bank."""
    from mosaic_amd.kernels.skinny_fp4 import pack_gate_up_mxfp4
    rng = np.random.default_rng(41)
    k, inter = 256, 96
    g = (rng.standard_normal((k, inter)) * 0.05).astype(np.float32)
    u = (rng.standard_normal((k, inter)) * 0.05).astype(np.float32)
    gb, ub = (torch.from_numpy(a).to(torch.bfloat16) for a in (g, u))
    p, s = pack_gate_up_mxfp4(gb.to(dev), ub.to(dev))
    p_ref, s_ref = C.quantize_mxfp4_floor(torch.cat([gb, ub], 1).float().numpy())
    assert tuple(p.shape) == (k, inter) and tuple(s.shape) == (k, 2 * inter // 32)
    np.testing.assert_array_equal(p.cpu().numpy(), p_ref)
    np.testing.assert_array_equal(s.view(torch.uint8).cpu().numpy(), s_ref)
    with pytest.raises(ValueError):
        pack_gate_up_mxfp4(gb.to(dev), ub.to(dev)[:, :64])


def test_xsimt_prepack_expert_bank_and_exact_decode(dev):
    """kernels/xsimt.py:380-394 (a stacked bank, cached) and :96-113 (e4m3 -> exact f16)."""
    from mosaic_amd import ops
    from mosaic_amd.kernels import _prepack_cache
    from mosaic_amd.kernels.xsimt import decode_activation_exact, prepack_expert_bank
    rng = np.random.default_rng(43)
    e, n, k = 3, 64, 256
    P = torch.from_numpy(rng.integers(0, 256, (e, n, k // 2), dtype=np.uint8)).to(dev)
    S = torch.from_numpy(rng.integers(100, 140, (e, n, k // 32), dtype=np.uint8)).to(dev)
    bank = prepack_expert_bank(P, S)
    assert prepack_expert_bank(P, S) is bank
    ref = ops.mxt16_prepack(P, S)
    assert torch.equal(bank.packed, ref.packed) and torch.equal(bank.scale, ref.scale)
    p2, s2 = ops.mxt16_unpack(bank)
    assert torch.equal(p2, P) and torch.equal(s2, S)
    del bank, ref
    _prepack_cache.clear()
    codes = np.arange(256, dtype=np.uint8)
    codes = codes[(codes & 0x7F) != 0x7F].reshape(2, 127)  # NaN codes excluded
    x8 = torch.from_numpy(codes).to(dev).view(torch.float8_e4m3fn)
    out = decode_activation_exact((x8, None))
    assert out.dtype == torch.float16
    np.testing.assert_array_equal(out.float().cpu().numpy(), C.e4m3_decode(codes))


def test_qpa_launch_census_counts_library_launches(dev):
    """kernels/qpa_mma.py:833-856: the census of one fused_moe_qpa call has the reference's
    keys and counts at least the MoE's gate/up and down launches as the library's."""
    from mosaic_amd.kernels import qpa_mma
    rng = np.random.default_rng(47)
    e, h, inter, m, k = 8, 256, 128, 3, 2
    gp, gs, dp, ds = _bank(rng, e, h, inter)
    x = torch.from_numpy(rng.standard_normal((m, h)).astype(np.float32)).to(torch.bfloat16).to(dev)
    ids = torch.from_numpy(np.stack([rng.choice(e, k, replace=False) for _ in range(m)])).to(dev)
    w = torch.from_numpy(rng.random((m, k)).astype(np.float32)).to(dev)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    fn = lambda: qpa_mma.fused_moe_qpa(x, ids, w, T(gp), T(gs), T(dp), T(ds))
    fn()
    c = qpa_mma.launch_census(fn)
    if "launch_census" in c:
        assert c["custom_launches"] >= 2
    else:
        assert set(c) == {"total_cuda_launches", "custom_qpa_launches", "custom_xsimt_launches",
                          "custom_mxint_launches", "layout_launches", "epilogue_launches"}
        assert c["custom_qpa_launches"] >= 2
        assert c["total_cuda_launches"] == c["custom_qpa_launches"] + c["layout_launches"] + c["epilogue_launches"]
