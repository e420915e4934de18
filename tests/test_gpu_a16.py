"""GPU parity of the A16 MXFP4 linear, routing, expert sort and A16 MoE layer.

Float bar: |got - ref| <= 2e-2 * max(1, |ref|) elementwise against the CPU
oracle's dequant-then-matmul of identical packed bytes (the benchmark spec's 2e-2 tolerance).
Index bar: routing ids, permutation, tile list bit-exact.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import codecs as C
from oracle import linear as L
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


def _bf16(a):
    return torch.from_numpy(np.asarray(a, dtype=np.float32)).to(torch.bfloat16)


def _quant_weights(rng, n, k, std=0.02):
    w = (rng.standard_normal((n, k)) * std).astype(np.float32)
    w = _bf16(w).float().numpy()
    return C.quantize_mxfp4_ceil(w)


@pytest.mark.parametrize("m,n,k", [(1, 16, 128), (1, 2048, 7168), (3, 40, 256), (16, 64, 1024), (17, 130, 384),
                                   (33, 48, 7168), (5, 7168, 2048)])
def test_linear_a16_vs_oracle(dev, m, n, k):
    ops = _ops()
    rng = np.random.default_rng(m * 1000 + n + k)
    packed, scale = _quant_weights(rng, n, k)
    x = _bf16(rng.standard_normal((m, k)))
    ref = L.mx_linear_a16(x.float().numpy(), packed, scale)
    y = ops.mx_linear_a16(x.to(dev), torch.from_numpy(packed).to(dev), torch.from_numpy(scale).to(dev))
    assert_close(y.float().cpu().numpy(), ref, what=f"linear m={m} n={n} k={k}")


def test_linear_a16_onehot_picks_column(dev):
    """x = e_j selects dequantized column j exactly (closed form)."""
    ops = _ops()
    rng = np.random.default_rng(1)
    n, k = 64, 256
    packed, scale = _quant_weights(rng, n, k, std=1.0)
    x = np.zeros((16, k), dtype=np.float32)
    cols = rng.choice(k, 16, replace=False)
    x[np.arange(16), cols] = 1.0
    y = ops.mx_linear_a16(_bf16(x).to(dev), torch.from_numpy(packed).to(dev),
                          torch.from_numpy(scale).to(dev)).float().cpu().numpy()
    w = C.dequant_mxfp4(packed, scale)
    np.testing.assert_array_equal(y, C.round_bf16(w[:, cols].T))


@pytest.mark.parametrize("n,k", [(16, 128), (48, 384), (2048, 7168), (32, 640)])
def test_mxt16_prepack_bitexact_roundtrip(dev, n, k):
    """The prepack is the documented permutation of 16-byte blocks and scale
    bytes, and unpack inverts it (reference test class: prepacks are bit-exact
    invertible, tests/test_qpa_mma.py:18-52)."""
    ops = _ops()
    rng = np.random.default_rng(n + k)
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    scale = rng.integers(0, 256, (n, k // 32), dtype=np.uint8)
    w = ops.mxt16_prepack(torch.from_numpy(packed).to(dev), torch.from_numpy(scale).to(dev))
    ns, ns4 = k // 128, (k // 128 + 3) // 4
    blocks = packed.reshape(n // 16, 16, ns, 4, 16)              # g, c, S, q, byte
    want_p = blocks.transpose(0, 2, 3, 1, 4).reshape(-1)         # g, S, q, c, byte
    np.testing.assert_array_equal(w.packed.cpu().numpy().reshape(-1), want_p)
    sc = np.zeros((n // 16, 16, ns4 * 4, 4), dtype=np.uint8)     # g, c, S, q
    sc[:, :, :ns, :] = scale.reshape(n // 16, 16, ns, 4)
    want_s = sc.reshape(n // 16, 16, ns4, 4, 4).transpose(0, 2, 4, 1, 3).reshape(-1)  # g, S4, q, c, s
    np.testing.assert_array_equal(w.scale.cpu().numpy().reshape(-1), want_s)
    p2, s2 = ops.mxt16_unpack(w)
    np.testing.assert_array_equal(p2.cpu().numpy(), packed)
    np.testing.assert_array_equal(s2.cpu().numpy(), scale)


@pytest.mark.parametrize("m,n,k", [(1, 16, 128), (1, 2048, 7168), (3, 48, 640), (16, 64, 1024), (20, 7168, 2048),
                                   (1, 528, 3072), (1, 64, 8192), (1, 4096, 1024)])
def test_mxt16_linear_a16_vs_oracle(dev, m, n, k):
    ops = _ops()
    rng = np.random.default_rng(m * 31 + n + k)
    packed, scale = _quant_weights(rng, n, k)
    x = _bf16(rng.standard_normal((m, k)))
    ref = L.mx_linear_a16(x.float().numpy(), packed, scale)
    w = ops.mxt16_prepack(torch.from_numpy(packed).to(dev), torch.from_numpy(scale).to(dev))
    y = ops.mxt16_linear_a16(x.to(dev), w)
    assert_close(y.float().cpu().numpy(), ref, what=f"mxt16 linear m={m} n={n} k={k}")


@pytest.mark.parametrize("m,n,k", [(1, 16, 128), (1, 2048, 7168), (3, 48, 640), (16, 64, 1024), (20, 7168, 2048),
                                   (70, 96, 512),
                                   # one row: the ring kernel's plans (K split 8 / 4 / 2 ways, rings of 4 and 8,
                                   # waves with no steps, a K tail of one step past whole 4-step groups)
                                   (1, 7168, 2048), (1, 4608, 7168), (1, 20480, 640), (1, 1536, 1152)])
def test_mxt16_linear_a8_vs_oracle(dev, m, n, k):
    """A8 "source semantics" linear (kernels/fp4_source.py:132-156) on the scaled MFMA."""
    ops = _ops()
    rng = np.random.default_rng(m * 13 + n + k)
    packed, scale = _quant_weights(rng, n, k)
    x = _bf16(rng.standard_normal((m, k)))
    ref = L.mx_linear_a8(x.float().numpy(), packed, scale)
    w = ops.mxt16_prepack(torch.from_numpy(packed).to(dev), torch.from_numpy(scale).to(dev))
    y = ops.mxt16_linear_a8(x.to(dev), w)
    assert_close(y.float().cpu().numpy(), ref, what=f"mxt16 a8 m={m} n={n} k={k}")
    # and it is the A8 contract, not the A16 one: rounding of x to e4m3 shows
    a16 = L.mx_linear_a16(x.float().numpy(), packed, scale, out_bf16=False)
    assert np.abs(y.float().cpu().numpy() - a16).max() > 1e-3


def test_mxt16_linear_a8_onehot_and_scales_kat(dev):
    """Closed form: one-hot e4m3 x (value 1.0, activation scale 2^a) selects
    2^a * dequantized weight column k exactly, with per-32 weight scales
    2^(b-127) -- pins the MFMA operand order and both e8m0 scale paths."""
    ops = _ops()
    rng = np.random.default_rng(3)
    n, k = 32, 256
    codes = rng.integers(0, 16, (n, k), dtype=np.uint8)
    packed = C.pack_codes(codes)
    scale = (120 + (np.arange(n)[:, None] + np.arange(k // 32)[None, :]) % 9).astype(np.uint8)
    w = ops.mxt16_prepack(torch.from_numpy(packed).to(dev), torch.from_numpy(scale).to(dev))
    W = C.dequant_mxfp4(packed, scale)
    xq = np.zeros((k, k), dtype=np.uint8)
    xq[np.arange(k), np.arange(k)] = 0x38  # e4m3 1.0
    a = (np.arange(k) % 5 - 2).astype(np.float32)
    sa = np.repeat((2.0 ** a)[:, None], k // 128, axis=1).astype(np.float32)
    y = ops.mxt16_linear_a8(None, w, prequant=(torch.from_numpy(xq).to(dev), torch.from_numpy(sa).to(dev)))
    np.testing.assert_array_equal(y.float().cpu().numpy(), C.round_bf16(W.T * (2.0 ** a)[:, None]))


@pytest.mark.parametrize("m,e,k,func", [(1, 256, 8, "sigmoid"), (64, 256, 8, "sigmoid"), (16, 64, 6, "softmax"),
                                        (9, 256, 8, "sqrtsoftplus"), (4, 16, 16, "sigmoid")])
def test_route_topk_vs_oracle(dev, m, e, k, func):
    ops = _ops()
    rng = np.random.default_rng(m + e + k)
    logits = rng.standard_normal((m, e)).astype(np.float32)
    logits[0, 5] = logits[0, 9] = logits[0].max() + 1.0  # exact tie -> lower index first
    ids, w = ops.moe_route_topk(torch.from_numpy(logits).to(dev), k, func)
    ids_ref, w_ref = MO.route_topk(logits, k, func)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(w.cpu().numpy(), w_ref, rtol=1e-5, atol=1e-7)
    assert ids.cpu().numpy()[0, 0] == 5 and ids.cpu().numpy()[0, 1] == 9


@pytest.mark.parametrize("m,k,e,shared", [(1, 8, 256, True), (4, 8, 256, False), (64, 8, 256, True),
                                          (300, 8, 16, True), (2, 1, 4, False), (4096, 8, 256, True),
                                          (700, 8, 16, False), (5000, 1, 4, True), (8000, 8, 512, True)])
def test_layout_vs_oracle(dev, m, k, e, shared):
    ops = _ops()
    rng = np.random.default_rng(m * 7 + e)
    ids = np.stack([rng.choice(e, k, replace=False) for _ in range(m)]).astype(np.int64)
    w = rng.random((m, k)).astype(np.float32)
    out = ops.moe_layout(torch.from_numpy(ids).to(dev), torch.from_numpy(w).to(dev), e, has_shared=shared,
                         block_m=16)
    flat = ids.reshape(-1)
    if shared:
        flat = np.concatenate([flat, np.full(m, e)])
    sorted_ids, perm, offsets, counts = MO.layout_assignments(flat, e + int(shared))
    np.testing.assert_array_equal(out["perm"].cpu().numpy(), perm)
    np.testing.assert_array_equal(out["sorted_ids"].cpu().numpy(), sorted_ids)
    np.testing.assert_array_equal(out["counts"].cpu().numpy(), counts)
    np.testing.assert_array_equal(out["offsets"].cpu().numpy(), offsets)
    inv = np.empty_like(perm)
    inv[perm] = np.arange(perm.size)
    np.testing.assert_array_equal(out["inv_pos"].cpu().numpy(), inv)
    tok = np.where(perm < m * k, perm // k, perm - m * k)
    np.testing.assert_array_equal(out["perm_token"].cpu().numpy(), tok)
    cpos = np.empty((m, k + int(shared)), dtype=np.int64)
    for t in range(m):
        order = np.argsort(ids[t], kind="stable")
        cpos[t, :k] = inv[t * k + order]
        if shared:
            cpos[t, k] = inv[m * k + t]
    np.testing.assert_array_equal(out["combine_pos"].cpu().numpy(), cpos)
    ei, ms, rows = MO.emit_tiles(counts, 16)
    nt = int(out["n_tiles"].cpu().item())
    np.testing.assert_array_equal(out["tile_p0"].cpu().numpy()[:nt], offsets[ei] + ms)
    assert nt == ei.size
    np.testing.assert_array_equal(out["tile_expert"].cpu().numpy()[:nt], ei)
    np.testing.assert_array_equal(out["tile_start"].cpu().numpy()[:nt], ms)
    np.testing.assert_array_equal(out["tile_rows"].cpu().numpy()[:nt], rows)


def test_layout_reference_kat(dev):
    """tests/test_moe_layout.py:13-24: ids [3,0,3,1] -> counts [1,1,0,2]."""
    ops = _ops()
    out = ops.moe_layout(torch.tensor([[3], [0], [3], [1]], device=dev), None, 4)
    assert out["counts"].cpu().tolist() == [1, 1, 0, 2]
    assert out["offsets"].cpu().tolist() == [0, 1, 2, 2, 4]
    assert out["sorted_ids"].cpu().tolist() == [0, 1, 3, 3]
    assert out["perm"].cpu().tolist() == [1, 3, 0, 2]


@pytest.mark.parametrize("block_m", [1, 8, 16])
def test_emit_tiles_reference_kat(dev, block_m):
    """tests/test_emit_tiles.py:14-34 closed form, without the 32-tile cap."""
    ops = _ops()
    counts = [0, 1, block_m - 1, block_m, block_m + 1, 3 * block_m + 2, 40 * block_m + 3]
    exp = []
    for e, c in enumerate(counts):
        for t in range((c + block_m - 1) // block_m):
            exp.append((e, t * block_m, min(block_m, c - t * block_m)))
    ei, ms, nt, rows = ops.emit_tiles(torch.tensor(counts, device=dev), block_m, 128)
    n = int(nt.item())
    assert n == len(exp)
    assert list(zip(ei[:n].tolist(), ms[:n].tolist(), rows[:n].tolist())) == exp
    ei, ms, nt, rows = ops.emit_tiles(torch.zeros(5, dtype=torch.int32, device=dev), block_m, 8)
    assert int(nt.item()) == 0


def _make_bank(rng, e, h, inter):
    gu = [_quant_weights(rng, 2 * inter, h) for _ in range(e)]
    d = [_quant_weights(rng, h, inter) for _ in range(e)]
    return (np.stack([g[0] for g in gu]), np.stack([g[1] for g in gu]), np.stack([x[0] for x in d]),
            np.stack([x[1] for x in d]))


@pytest.mark.parametrize("m,e,h,inter,k,shared,limit", [
    (1, 16, 256, 128, 4, True, 0.0), (3, 16, 256, 128, 4, False, 10.0), (20, 8, 384, 256, 2, True, 0.0),
    (37, 32, 512, 128, 8, True, 10.0), (600, 16, 256, 128, 8, True, 0.0),
    # small-batch layout kernel: up to 16 tokens x (8 + shared) assignments, 256 experts
    (16, 64, 256, 128, 8, True, 0.0), (9, 256, 256, 128, 8, True, 10.0), (16, 256, 256, 128, 15, True, 0.0)])
def test_moe_a16_small_vs_oracle(dev, m, e, h, inter, k, shared, limit):
    ops = _ops()
    rng = np.random.default_rng(m + e + h)
    gp, gs, dp, ds = _make_bank(rng, e, h, inter)
    sh = _make_bank(rng, 1, h, inter) if shared else None
    x = _bf16(rng.standard_normal((m, h)))
    logits = rng.standard_normal((m, e)).astype(np.float32)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    gu_b, d_b = ops.mxt16_prepack(T(gp), T(gs)), ops.mxt16_prepack(T(dp), T(ds))
    shb = None if sh is None else (ops.mxt16_prepack(T(sh[0][0]), T(sh[1][0])),
                                   ops.mxt16_prepack(T(sh[2][0]), T(sh[3][0])))
    y, ids, w = ops.moe_a16_forward(x.to(dev), gu_b, d_b, logits=T(logits), top_k=k, shared=shb,
                                    swiglu_limit=limit)
    ids_ref, w_ref = MO.route_topk(logits, k, "sigmoid")
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    ref = MO.moe_layer_a16(x.float().numpy(), ids_ref, w_ref, gp, gs, dp, ds,
                           shared=None if sh is None else tuple(t[0] for t in sh), swiglu_limit=limit)
    assert_close(y.float().cpu().numpy(), ref, what="moe a16")


def test_moe_a16_given_ids_weight_before_down(dev):
    """ids/weights supplied (fused_moe_* call form); scaling z before down
    differs from scaling the output after (tests/test_exact_expert_semantics.py:78-107)."""
    ops = _ops()
    rng = np.random.default_rng(8)
    e, h, inter, m, k = 4, 256, 128, 2, 2
    gp, gs, dp, ds = _make_bank(rng, e, h, inter)
    x = _bf16(rng.standard_normal((m, h)) * 6.0)
    ids = np.array([[1, 3], [0, 2]])
    w = np.array([[0.25, 1.5], [0.5, 0.01]], dtype=np.float32)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    y, _, _ = ops.moe_a16_forward(x.to(dev), ops.mxt16_prepack(T(gp), T(gs)), ops.mxt16_prepack(T(dp), T(ds)),
                                  ids=T(ids), weights=T(w), swiglu_limit=10.0)
    ref = MO.moe_layer_a16(x.float().numpy(), ids, w, gp, gs, dp, ds, swiglu_limit=10.0)
    assert_close(y.float().cpu().numpy(), ref, what="moe given ids")
    unit = MO.moe_layer_a16(x.float().numpy(), ids, np.ones_like(w), gp, gs, dp, ds, swiglu_limit=10.0)
    assert not np.allclose(y.float().cpu().numpy(), unit, atol=1e-3)


# ---- batch-1 decode path (fused routing + gate/up, fused down + combine) ----
# It is taken for M == 1 when hidden and inter are multiples of 512.
@pytest.mark.parametrize("e,h,inter,k,shared,limit,func", [
    (16, 512, 512, 4, True, 0.0, "sigmoid"), (32, 1024, 512, 8, False, 10.0, "sigmoid"),
    (64, 2048, 1024, 6, True, 10.0, "softmax"), (8, 512, 1024, 8, True, 0.0, "sqrtsoftplus"),
    (16, 1536, 2048, 1, True, 0.0, "sigmoid"), (8, 5120, 512, 4, True, 0.0, "sigmoid"),
    (8, 1024, 4096, 2, True, 10.0, "sigmoid")])
def test_moe_a16_decode1_vs_oracle(dev, e, h, inter, k, shared, limit, func):
    ops = _ops()
    rng = np.random.default_rng(e * 7 + h + inter + k)
    gp, gs, dp, ds = _make_bank(rng, e, h, inter)
    sh = _make_bank(rng, 1, h, inter) if shared else None
    x = _bf16(rng.standard_normal((1, h)))
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    gu_b, d_b = ops.mxt16_prepack(T(gp), T(gs)), ops.mxt16_prepack(T(dp), T(ds))
    shb = None if sh is None else (ops.mxt16_prepack(T(sh[0][0]), T(sh[1][0])),
                                   ops.mxt16_prepack(T(sh[2][0]), T(sh[3][0])))
    for rep in range(2):  # two calls in a row with different routing reuse the workspace
        logits = rng.standard_normal((1, e)).astype(np.float32)
        y, ids, w = ops.moe_a16_forward(x.to(dev), gu_b, d_b, logits=T(logits), top_k=k, shared=shb,
                                        swiglu_limit=limit, score_func=func)
        ids_ref, w_ref = MO.route_topk(logits, k, func)
        np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
        np.testing.assert_allclose(w.cpu().numpy(), w_ref, rtol=1e-6, atol=1e-7)
        ref = MO.moe_layer_a16(x.float().numpy(), ids_ref, w_ref, gp, gs, dp, ds,
                               shared=None if sh is None else tuple(t[0] for t in sh), swiglu_limit=limit)
        assert_close(y.float().cpu().numpy(), ref, what=f"moe a16 decode1 call {rep}")


def test_moe_a16_decode1_given_ids_drop_and_duplicate(dev):
    """ids given: an out-of-range id is dropped, a repeated id counts twice."""
    ops = _ops()
    rng = np.random.default_rng(21)
    e, h, inter, k = 8, 512, 512, 4
    gp, gs, dp, ds = _make_bank(rng, e, h, inter)
    sh = _make_bank(rng, 1, h, inter)
    x = _bf16(rng.standard_normal((1, h)) * 3.0)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    ids = np.array([[5, -1, 2, 5]])
    w = np.array([[0.5, 0.7, 0.25, 0.125]], dtype=np.float32)
    shb = (ops.mxt16_prepack(T(sh[0][0]), T(sh[1][0])), ops.mxt16_prepack(T(sh[2][0]), T(sh[3][0])))
    y, _, _ = ops.moe_a16_forward(x.to(dev), ops.mxt16_prepack(T(gp), T(gs)), ops.mxt16_prepack(T(dp), T(ds)),
                                  ids=T(ids.astype(np.int32)), weights=T(w), shared=shb, swiglu_limit=10.0)
    keep = ids[0] >= 0
    ref = MO.moe_layer_a16(x.float().numpy(), ids[:, keep], w[:, keep], gp, gs, dp, ds,
                           shared=tuple(t[0] for t in sh), swiglu_limit=10.0)
    assert_close(y.float().cpu().numpy(), ref, what="moe decode1 given ids")


# ---- 2..4 tokens with routing on the device: layout, grouped gate/up, then
# one down kernel that walks every tile and combines in registers ----
@pytest.mark.parametrize("m,e,h,inter,k,shared,limit,func", [
    (2, 16, 512, 512, 4, True, 0.0, "sigmoid"),          # 1 super-step per K part, 2-row buffers
    (3, 32, 1024, 1024, 8, False, 10.0, "softmax"),      # 2 super-steps per part, no shared expert
    (4, 64, 2048, 2048, 8, True, 10.0, "sqrtsoftplus"),  # 4 super-steps per part
    (4, 8, 512, 4096, 2, True, 0.0, "sigmoid"),          # 8 K parts
    (2, 8, 4096, 512, 8, True, 0.0, "sigmoid"),          # 16-column workgroups; every token picks every expert
    (4, 8, 1024, 512, 8, True, 10.0, "sigmoid"),         # every tile holds all 4 tokens
    (4, 256, 512, 512, 16, True, 0.0, "sigmoid")])       # the longest tile list (68 tiles)
def test_moe_a16_small_batch_down_vs_oracle(dev, m, e, h, inter, k, shared, limit, func):
    ops = _ops()
    rng = np.random.default_rng(m * 11 + e + h + inter + k)
    gp, gs, dp, ds = _make_bank(rng, e, h, inter)
    sh = _make_bank(rng, 1, h, inter) if shared else None
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    gu_b, d_b = ops.mxt16_prepack(T(gp), T(gs)), ops.mxt16_prepack(T(dp), T(ds))
    shb = None if sh is None else (ops.mxt16_prepack(T(sh[0][0]), T(sh[1][0])),
                                   ops.mxt16_prepack(T(sh[2][0]), T(sh[3][0])))
    ws = ops.MoEWorkspace()
    for rep in range(2):  # two calls in a row with different tokens and routing share the workspace
        x = _bf16(rng.standard_normal((m, h)))
        logits = rng.standard_normal((m, e)).astype(np.float32)
        y, ids, w = ops.moe_a16_forward(x.to(dev), gu_b, d_b, logits=T(logits), top_k=k, shared=shb,
                                        swiglu_limit=limit, score_func=func, workspace=ws)
        ids_ref, w_ref = MO.route_topk(logits, k, func)
        np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
        ref = MO.moe_layer_a16(x.float().numpy(), ids_ref, w_ref, gp, gs, dp, ds,
                               shared=None if sh is None else tuple(t[0] for t in sh), swiglu_limit=limit)
        assert_close(y.float().cpu().numpy(), ref, what=f"moe a16 m={m} small-batch down, call {rep}")


@pytest.mark.parametrize("a8", [False, True])
def test_moe_given_ids_repeated_and_dropped_multi_token(dev, a8):
    """Layout path (M > 1): a repeated expert id in one token counts once per
    slot (slot order inside the expert), an out-of-range id is dropped."""
    ops = _ops()
    rng = np.random.default_rng(33)
    e, h, inter, m, k = 8, 256, 128, 3, 4
    gp, gs, dp, ds = _make_bank(rng, e, h, inter)
    x = _bf16(rng.standard_normal((m, h)) * 2.0)
    ids = np.array([[5, -1, 2, 5], [1, 1, 1, 7], [0, 3, 9, 3]])
    w = rng.uniform(0.1, 1.0, size=(m, k)).astype(np.float32)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    fwd = ops.moe_a8_forward if a8 else ops.moe_a16_forward
    y, _, _ = fwd(x.to(dev), ops.mxt16_prepack(T(gp), T(gs)), ops.mxt16_prepack(T(dp), T(ds)),
                  ids=T(ids.astype(np.int32)), weights=T(w), swiglu_limit=10.0)
    oracle = MO.moe_layer_a8 if a8 else MO.moe_layer_a16
    for t in range(m):
        keep = (ids[t] >= 0) & (ids[t] < e)
        ref = oracle(x[t:t + 1].float().numpy(), ids[t:t + 1, keep], w[t:t + 1, keep], gp, gs, dp, ds,
                     swiglu_limit=10.0)
        assert_close(y[t:t + 1].float().cpu().numpy(), ref, what=f"moe repeated ids token {t}")


def test_moe_empty_batch_returns_empty(dev):
    """An empty batch (M = 0) gives empty outputs without a launch, on both contracts,
    with routing on the device or with given ids, and on the KN (skinny) layout."""
    ops = _ops()
    rng = np.random.default_rng(3)
    e, h, inter = 4, 256, 128
    gp, gs, dp, ds = _make_bank(rng, e, h, inter)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    gu, dn = ops.mxt16_prepack(T(gp), T(gs)), ops.mxt16_prepack(T(dp), T(ds))
    x = torch.empty(0, h, dtype=torch.bfloat16, device=dev)
    for fwd in (ops.moe_a16_forward, ops.moe_a8_forward):
        y, ids, w = fwd(x, gu, dn, logits=torch.empty(0, e, device=dev), top_k=2)
        assert tuple(y.shape) == (0, h) and tuple(ids.shape) == (0, 2) and tuple(w.shape) == (0, 2)
        y, ids, w = fwd(x, gu, dn, ids=torch.empty(0, 2, dtype=torch.int32, device=dev),
                        weights=torch.empty(0, 2, device=dev))
        assert tuple(y.shape) == (0, h) and tuple(ids.shape) == (0, 2)
        with pytest.raises(ValueError):
            fwd(x, gu, dn)
    kn_gu = torch.zeros(e, h, inter, dtype=torch.uint8, device=dev)
    kn_gs = torch.full((e, h, 2 * inter // 32), 127, dtype=torch.uint8, device=dev)
    kn_d = torch.zeros(e, inter, h // 2, dtype=torch.uint8, device=dev)
    kn_ds = torch.full((e, inter, h // 32), 127, dtype=torch.uint8, device=dev)
    y = ops.moe_skinny_forward(x, torch.empty(0, 2, dtype=torch.int32, device=dev), torch.empty(0, 2, device=dev),
                               kn_gu, kn_gs, kn_d, kn_ds)
    assert tuple(y.shape) == (0, h)


def test_moe_a8_prefill_tile_boundaries(dev):
    """Prefill kernels (A8) at the tile-shape boundaries, with given ids: experts
    with 1, 64 (last light tile), 65 (first full-tile path), 128 and 129 (the
    second and third row quarters of a partial tile), 256 (one full tile) and 257
    rows (a full tile plus a one-row light tile), plus the shared expert."""
    ops = _ops()
    rng = np.random.default_rng(61)
    e, h, inter = 7, 512, 512
    rows = [1, 64, 65, 128, 129, 256, 257]
    ids = np.concatenate([np.full(r, i) for i, r in enumerate(rows)])
    rng.shuffle(ids)
    m = ids.size
    ids = ids.reshape(m, 1).astype(np.int32)
    w = rng.uniform(0.1, 1.0, size=(m, 1)).astype(np.float32)
    gp, gs, dp, ds = _make_bank(rng, e, h, inter)
    sh = _make_bank(rng, 1, h, inter)
    x = _bf16(rng.standard_normal((m, h)))
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    shb = (ops.mxt16_prepack(T(sh[0][0]), T(sh[1][0])), ops.mxt16_prepack(T(sh[2][0]), T(sh[3][0])))
    y, _, _ = ops.moe_a8_forward(x.to(dev), ops.mxt16_prepack(T(gp), T(gs)), ops.mxt16_prepack(T(dp), T(ds)),
                                 ids=T(ids), weights=T(w), shared=shb, swiglu_limit=10.0)
    ref = MO.moe_layer_a8(x.float().numpy(), ids, w, gp, gs, dp, ds, swiglu_limit=10.0,
                          shared=tuple(t[0] for t in sh))
    assert_close(y.float().cpu().numpy(), ref, what="moe a8 prefill tile boundaries")


def test_moe_a16_decode1_baseline_geometry(dev):
    """BASELINE.json configs[1] geometry (hidden 7168, inter 2048, top-8, shared) on a
    32-expert bank quantized on the device; oracle over the experts actually used."""
    ops = _ops()
    e, h, inter, k = 32, 7168, 2048, 8
    g = torch.Generator(device=dev)
    g.manual_seed(5)
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
    x = torch.randn(1, h, generator=g, device=dev).to(torch.bfloat16)
    logits = torch.randn(1, e, generator=g, device=dev)
    y, ids, w = ops.moe_a16_forward(x, ops.mxt16_prepack(gp[:e], gs[:e]), ops.mxt16_prepack(dp[:e], ds[:e]),
                                    logits=logits, top_k=k,
                                    shared=(ops.mxt16_prepack(gp[e], gs[e]), ops.mxt16_prepack(dp[e], ds[e])))
    ids_ref, w_ref = MO.route_topk(logits.cpu().numpy(), k, "sigmoid")
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    host = lambda t: (lambda i: t[i].cpu().numpy())
    ref = MO.moe_layer_a16(x.float().cpu().numpy(), ids_ref, w_ref, host(gp), host(gs), host(dp), host(ds),
                           shared=(gp[e].cpu().numpy(), gs[e].cpu().numpy(), dp[e].cpu().numpy(),
                                   ds[e].cpu().numpy()))
    assert_close(y.float().cpu().numpy(), ref, what="moe decode1 baseline geometry")


@pytest.mark.parametrize("m,e,h,inter,k,shared,limit", [
    (1, 16, 256, 128, 4, False, 10.0), (3, 16, 256, 128, 4, True, 10.0), (20, 8, 384, 256, 2, False, 0.0),
    (37, 32, 512, 128, 8, True, 10.0), (520, 8, 256, 128, 8, True, 10.0), (300, 16, 384, 256, 4, False, 0.0),
    (1100, 32, 256, 128, 8, True, 10.0),
    # prefill kernels (H, I multiples of 512): full and partial 256-row tiles, light (<= 64-row) tiles
    (600, 8, 512, 512, 8, True, 10.0), (130, 32, 512, 512, 8, True, 0.0), (300, 16, 1024, 512, 8, False, 10.0),
    (16, 32, 256, 128, 8, True, 10.0)])
def test_moe_a8_small_vs_oracle(dev, m, e, h, inter, k, shared, limit):
    """A8 layer (fused_moe_mxint contract) vs the A8 oracle of identical bytes."""
    ops = _ops()
    rng = np.random.default_rng(m + e + h + 1)
    gp, gs, dp, ds = _make_bank(rng, e, h, inter)
    sh = _make_bank(rng, 1, h, inter) if shared else None
    x = _bf16(rng.standard_normal((m, h)))
    logits = rng.standard_normal((m, e)).astype(np.float32)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    gu_b, d_b = ops.mxt16_prepack(T(gp), T(gs)), ops.mxt16_prepack(T(dp), T(ds))
    shb = None if sh is None else (ops.mxt16_prepack(T(sh[0][0]), T(sh[1][0])),
                                   ops.mxt16_prepack(T(sh[2][0]), T(sh[3][0])))
    y, ids, w = ops.moe_a8_forward(x.to(dev), gu_b, d_b, logits=T(logits), top_k=k, shared=shb, swiglu_limit=limit)
    ids_ref, w_ref = MO.route_topk(logits, k, "sigmoid")
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    ref = MO.moe_layer_a8(x.float().numpy(), ids_ref, w_ref, gp, gs, dp, ds, swiglu_limit=limit,
                          shared=None if sh is None else tuple(t[0] for t in sh))
    assert_close(y.float().cpu().numpy(), ref, what="moe a8")


@pytest.mark.parametrize("m,n,k", [(128, 256, 512), (257, 512, 1024), (1024, 512, 2048), (300, 7168, 512),
                                   (64, 1536, 1536), (100, 320, 1024), (384, 512, 1536), (400, 256, 512),
                                   # staged dense kernel: 64-row tiles (M <= 256), split K over whole 512-K
                                   # chunks (uneven: 7 chunks in 4 slices), N tails (592 = 2 x 256 + 80,
                                   # 576 = 2 x 256 + 64), the 33-row threshold, the 16-row kernel at 32 rows
                                   (33, 256, 1024), (32, 512, 1024), (65, 592, 1536), (200, 576, 2048),
                                   (128, 8192, 3584), (256, 1040, 4096), (520, 592, 3072), (4096, 576, 1024),
                                   # up to 256 rows on one 256-row tile per column, split 3 ways (the 64-row
                                   # plan would leave most CUs idle), with a 16-column N tail
                                   (120, 16400, 1536)])
def test_mxt16_linear_a8_prefill_vs_oracle(dev, m, n, k):
    """Dense A8 MXFP4 GEMM at prefill sizes (fp4_gemm, .mosaicvm/source/inference_kernel.py:441-536):
    above 32 rows with K a multiple of 512 the staged scaled-MFMA kernel runs with
    64-row tiles up to 256 rows (256-row tiles when 64-row ones would leave most
    CUs idle) and 256-row tiles above (the last tile light or a partial full one), 256-column tiles with the N tail masked, and K split into
    512-K chunk slices while the tiles cover at most half of the GPU; the other
    shapes run the 16-row kernel."""
    ops = _ops()
    rng = np.random.default_rng(m + n + k + 7)
    p, s = _quant_weights(rng, n, k)
    x = C.round_bf16(rng.standard_normal((m, k)).astype(np.float32))
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    y = ops.mxt16_linear_a8(T(x).to(torch.bfloat16), ops.mxt16_prepack(T(p), T(s)))
    assert_close(y.float().cpu().numpy(), L.mx_linear_a8(x, p, s), what=f"a8 prefill {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", [(128, 1024, 4096), (4096, 576, 2048)])
def test_mxt16_linear_a8_split_plan_matches_unsplit(dev, m, n, k):
    """A split-K plan without its workspace runs unsplit (mosaic_mxt16_linear_a8);
    both agree with the oracle, and the split reduce sums the slices in order
    (two split calls are bit-identical)."""
    import ctypes
    from mosaic_amd import _lib
    ops = _ops()
    rng = np.random.default_rng(m + n + k)
    p, s = _quant_weights(rng, n, k)
    x = C.round_bf16(rng.standard_normal((m, k)).astype(np.float32))
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    w = ops.mxt16_prepack(T(p), T(s))
    assert _lib.lib().mosaic_mxt16_linear_a8_workspace_bytes(m, n, k) > 0, "the shape must take a split plan"
    xq, sa = ops.act_quant(T(x).to(torch.bfloat16), 128, "pow2")
    y1 = ops.mxt16_linear_a8(None, w, prequant=(xq, sa))
    y2 = ops.mxt16_linear_a8(None, w, prequant=(xq, sa))
    assert torch.equal(y1, y2)
    y0 = torch.empty_like(y1)
    _lib.call("mosaic_mxt16_linear_a8", ctypes.c_void_p(xq.data_ptr()), ctypes.c_void_p(sa.data_ptr()),
              ctypes.c_void_p(w.packed.data_ptr()), ctypes.c_void_p(w.scale.data_ptr()),
              ctypes.c_void_p(y0.data_ptr()), m, n, k, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    ref = L.mx_linear_a8(x, p, s)
    assert_close(y1.float().cpu().numpy(), ref, what="split plan")
    assert_close(y0.float().cpu().numpy(), ref, what="unsplit plan")


@pytest.mark.parametrize("m", [128, 4096])
@pytest.mark.parametrize("n,k", [(7168, 16384), (18432, 7168), (24576, 1536), (1536, 7168), (576, 7168)])
def test_mxt16_linear_a8_config3_shapes(dev, m, n, k):
    """The timed dense A8 MXFP4 GEMMs (config-3 shapes with MXFP4 weights, as
    bench.py times them: ceil-recipe weights N(0, 0.02), 1x128 pow2 e4m3
    activations) at full size: every column of sampled rows against the A8
    oracle of identical bytes."""
    ops = _ops()
    g = torch.Generator(device=dev)
    g.manual_seed(n + k + m)
    p, sc = ops.mx_quantize((torch.randn(n, k, generator=g, device=dev) * 0.02).to(torch.bfloat16), "ceil")
    x = torch.randn(m, k, generator=g, device=dev).to(torch.bfloat16)
    xq, sa = ops.act_quant(x, 128, "pow2")
    y = ops.mxt16_linear_a8(None, ops.mxt16_prepack(p, sc), prequant=(xq, sa))
    rows = sorted({0, m // 2 - 1, m // 2, m - 1} | set(np.random.default_rng(k).choice(m, 4, replace=False).tolist()))
    ref = L.mx_linear_a8(None, p.cpu().numpy(), sc.cpu().numpy(),
                         quant=(xq[rows].view(torch.uint8).cpu().numpy(), sa[rows].cpu().numpy()))
    assert_close(y[rows].float().cpu().numpy(), ref, what=f"a8 dense ({m}, {n}, {k})")
    assert torch.isfinite(y.float()).all()
