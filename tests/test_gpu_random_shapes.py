"""Seeded random shapes through every dispatch of the linears, against the CPU oracle:
the A8 MXFP4 linear (16-row kernel, staged 64- and 256-row plans, split K, N tails),
the A16 MXFP4 linear (NK and KN layouts) and the FP8 block GEMM (skinny, decode ring,
tiled, split K, big tiles, mid; at M <= 64 also over the T16 prepack), the one-row A8 ring
and fp8_w8a16_linear.  Float bar |got - ref| <= 2e-2 * max(1, |ref|).  Sizes keep each
oracle call under ~1e8 multiply-adds (a few 1e8-1e9 for the wide FP8 and W8A16 cases)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import codecs as C
from oracle import linear as L

pytestmark = pytest.mark.gpu

N_CASES = 32


def _close(got, ref, what):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref) / np.maximum(1.0, np.abs(ref))
    assert err.max() <= 2e-2, f"{what}: max scaled err {err.max():.3e}"


def _shape(rng, m_max, n_step, n_max, k_step, k_max, budget=1e8):
    while True:
        m = int(rng.integers(1, m_max + 1))
        n = n_step * int(rng.integers(1, n_max // n_step + 1))
        k = k_step * int(rng.integers(1, k_max // k_step + 1))
        if m * n * k <= budget:
            return m, n, k


def _bf16(a):
    return torch.from_numpy(np.asarray(a, dtype=np.float32)).to(torch.bfloat16)


@pytest.mark.parametrize("seed", range(N_CASES))
def test_a8_linear_random_shapes(dev, seed):
    from mosaic_amd import ops
    rng = np.random.default_rng(9000 + seed)
    # K of whole 512-K chunks half the time (the staged plans), else any multiple of 128
    m, n, k = _shape(rng, 400, 16, 1600, 512 if seed % 2 == 0 else 128, 4096)
    p, s = C.quantize_mxfp4_ceil(_bf16(rng.standard_normal((n, k)) * 0.05).float().numpy())
    x = _bf16(rng.standard_normal((m, k)))
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    y = ops.mxt16_linear_a8(x.to(dev), ops.mxt16_prepack(T(p), T(s)))
    _close(y.float().cpu().numpy(), L.mx_linear_a8(x.float().numpy(), p, s), f"a8 {m}x{n}x{k}")


@pytest.mark.parametrize("seed", range(N_CASES))
def test_a16_linears_random_shapes(dev, seed):
    from mosaic_amd import ops
    rng = np.random.default_rng(9100 + seed)
    m, n, k = _shape(rng, 64, 32, 2048, 128, 4096)
    x = _bf16(rng.standard_normal((m, k)))
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    p, s = C.quantize_mxfp4_ceil(_bf16(rng.standard_normal((n, k)) * 0.05).float().numpy())
    y = ops.mx_linear_a16(x.to(dev), T(p), T(s))
    _close(y.float().cpu().numpy(), L.mx_linear_a16(x.float().numpy(), p, s), f"a16 nk {m}x{n}x{k}")
    w = ops.mxt16_prepack(T(p), T(s))
    _close(ops.mxt16_linear_a16(x.to(dev), w).float().cpu().numpy(), L.mx_linear_a16(x.float().numpy(), p, s),
           f"a16 mxt16 {m}x{n}x{k}")
    pk, sk = C.quantize_mxfp4_ceil(_bf16(rng.standard_normal((k, n)) * 0.05).float().numpy())
    yk = ops.mx_kn_linear_a16(x.to(dev), T(pk), T(sk))
    _close(yk.float().cpu().numpy(), L.mx_linear_kn_a16(x.float().numpy(), pk, sk), f"a16 kn {m}x{n}x{k}")


@pytest.mark.parametrize("seed", range(N_CASES))
def test_fp8_block_gemm_random_shapes(dev, seed):
    from mosaic_amd import ops
    rng = np.random.default_rng(9200 + seed)
    m, n, k = _shape(rng, 600 if seed % 3 else 16, 1, 1500, 128, 3072)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    bq, bs = L.quantize_fp8_weight_128(w)
    aq, a_s = C.act_quant(x, 128, "amax")
    T = lambda v: torch.from_numpy(np.ascontiguousarray(v)).to(dev)
    c = ops.fp8_block_gemm(T(aq), T(a_s), T(bq), T(bs))
    _close(c.float().cpu().numpy(), L.fp8_block_gemm(aq, a_s, bq, bs), f"fp8 {m}x{n}x{k}")
    n16 = n - n % 16  # the T16 prepack of the weight's first whole 16-row groups
    if m <= ops.FP8_T16_MAX_M and n16:
        b16, s16 = bq[:n16], bs[:(n16 + 127) // 128]
        ct = ops.fp8_block_gemm(T(aq), T(a_s), ops.fp8_t16_prepack(T(b16)), T(s16))
        _close(ct.float().cpu().numpy(), L.fp8_block_gemm(aq, a_s, b16, s16), f"fp8 t16 {m}x{n16}x{k}")


@pytest.mark.parametrize("seed", range(9))
def test_a8_linear_one_row_random_shapes(dev, seed):
    """One row through the A8 decode ring: N drawn so that every third case falls in each
    of its plans (up to 256, up to 1152 and more 16-row tiles), K any multiple of 128."""
    from mosaic_amd import ops
    rng = np.random.default_rng(9250 + seed)
    lo, hi = [(1, 256), (257, 1152), (1153, 1600)][seed % 3]
    n = 16 * int(rng.integers(lo, hi + 1))
    k = 128 * int(rng.integers(1, min(64, int(4e7 // (n * 128))) + 1))
    p, s = C.quantize_mxfp4_ceil(_bf16(rng.standard_normal((n, k)) * 0.05).float().numpy())
    x = _bf16(rng.standard_normal((1, k)))
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    y = ops.mxt16_linear_a8(x.to(dev), ops.mxt16_prepack(T(p), T(s)))
    _close(y.float().cpu().numpy(), L.mx_linear_a8(x.float().numpy(), p, s), f"a8 1x{n}x{k}")


@pytest.mark.parametrize("seed", range(12))
def test_fp8_w8a16_random_shapes(dev, seed):
    """fp8_w8a16_linear at 1..80 rows: the decode ring (<= 16 rows), the mid kernel
    (17..80 rows, N >= 4096) and the row-tile grid (narrower N), any N, K a multiple of 128."""
    from mosaic_amd import ops
    rng = np.random.default_rng(9260 + seed)
    m = int(rng.integers(1, 17)) if seed % 3 == 0 else int(rng.integers(17, ops.W8A16_MAX_M + 1))
    n = int(rng.integers(4096, 9001)) if seed % 3 != 2 else int(rng.integers(1, 4096))
    k = 128 * int(rng.integers(1, min(24, int(4e8 // (m * n * 128))) + 1))
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    bq, bs = L.quantize_fp8_weight_128(w)
    x = _bf16(rng.standard_normal((m, k)))
    T = lambda v: torch.from_numpy(np.ascontiguousarray(v)).to(dev)
    y = ops.fp8_w8a16_linear(x.to(dev), T(bq), T(bs))
    _close(y.float().cpu().numpy(), L.fp8_w8a16_linear(x.float().numpy(), bq, bs), f"w8a16 {m}x{n}x{k}")


@pytest.mark.parametrize("seed", range(8))
def test_fp8_mid_random_shapes(dev, seed):
    """17..64 rows with a weight of 8 MB and more (the mid kernel over the checkpoint rows,
    split K when its workgroups are few), and the same weight over the T16 prepack."""
    from mosaic_amd import ops
    rng = np.random.default_rng(9270 + seed)
    m = int(rng.integers(17, ops.FP8_T16_MAX_M + 1))
    n = 16 * int(rng.integers(64, 513))
    kmin = -(-(8 << 20) // (n * 128))
    k = 128 * int(rng.integers(kmin, max(kmin, (24 << 20) // (n * 128)) + 1))
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    bq, bs = L.quantize_fp8_weight_128(w)
    aq, a_s = C.act_quant(x, 128, "amax")
    T = lambda v: torch.from_numpy(np.ascontiguousarray(v)).to(dev)
    ref = L.fp8_block_gemm(aq, a_s, bq, bs)
    c = ops.fp8_block_gemm(T(aq), T(a_s), T(bq), T(bs))
    _close(c.float().cpu().numpy(), ref, f"fp8 mid {m}x{n}x{k}")
    ct = ops.fp8_block_gemm(T(aq), T(a_s), ops.fp8_t16_prepack(T(bq)), T(bs))
    _close(ct.float().cpu().numpy(), ref, f"fp8 mid t16 {m}x{n}x{k}")


def _bank(rng, e, h, inter):
    q = lambda r, c: C.quantize_mxfp4_ceil(_bf16(rng.standard_normal((r, c)) * 0.05).float().numpy())
    gu = [q(2 * inter, h) for _ in range(e)]
    d = [q(h, inter) for _ in range(e)]
    return (np.stack([a[0] for a in gu]), np.stack([a[1] for a in gu]), np.stack([a[0] for a in d]),
            np.stack([a[1] for a in d]))


def _moe_case(rng, a8):
    e = int(rng.choice([4, 8, 16, 32, 64]))
    k = int(rng.integers(1, min(8, e) + 1))
    h = int(rng.choice([512, 1024] if a8 else [256, 384, 512]))
    inter = int(rng.choice([512, 1024] if a8 else [128, 256, 512]))
    m = int(rng.choice([1, 2, 3, 4, 7, 16, 33, 130, 200] if a8 else [1, 2, 3, 4, 7, 16, 33]))
    func = str(rng.choice(["sigmoid", "softmax", "sqrtsoftplus"]))
    return m, e, h, inter, k, bool(rng.integers(0, 2)), float(rng.choice([0.0, 10.0])), func


@pytest.mark.parametrize("a8", [False, True])
@pytest.mark.parametrize("seed", range(10))
def test_moe_random_configs(dev, seed, a8):
    """Routing on the device (sigmoid / softmax / sqrtsoftplus scores, top-k with ties to the
    lower index, renormalized) then the layer: ids bit-exact, y within the float bar, for
    random expert counts, top-k, widths, batch sizes (decode, layout and, for A8, prefill
    paths), shared expert on or off and SwiGLU limit 0 or 10."""
    from oracle import moe as MO
    from mosaic_amd import ops
    rng = np.random.default_rng(9300 + 17 * seed + a8)
    m, e, h, inter, k, shared, limit, func = _moe_case(rng, a8)
    gp, gs, dp, ds = _bank(rng, e, h, inter)
    sh = _bank(rng, 1, h, inter) if shared else None
    x = _bf16(rng.standard_normal((m, h)))
    logits = rng.standard_normal((m, e)).astype(np.float32)
    T = lambda v: torch.from_numpy(np.ascontiguousarray(v)).to(dev)
    gu_b, d_b = ops.mxt16_prepack(T(gp), T(gs)), ops.mxt16_prepack(T(dp), T(ds))
    shb = None if sh is None else (ops.mxt16_prepack(T(sh[0][0]), T(sh[1][0])),
                                   ops.mxt16_prepack(T(sh[2][0]), T(sh[3][0])))
    fwd = ops.moe_a8_forward if a8 else ops.moe_a16_forward
    y, ids, w = fwd(x.to(dev), gu_b, d_b, logits=T(logits), top_k=k, shared=shb, swiglu_limit=limit,
                    score_func=func)
    ids_ref, w_ref = MO.route_topk(logits, k, func)
    what = f"{'a8' if a8 else 'a16'} m={m} e={e} h={h} i={inter} k={k} shared={shared} limit={limit} {func}"
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref, err_msg=what)
    np.testing.assert_array_equal(w.cpu().numpy(), w_ref, err_msg=what)
    layer = MO.moe_layer_a8 if a8 else MO.moe_layer_a16
    ref = layer(x.float().numpy(), ids_ref, w_ref, gp, gs, dp, ds, swiglu_limit=limit,
                shared=None if sh is None else tuple(t[0] for t in sh))
    _close(y.float().cpu().numpy(), ref, what)


@pytest.mark.parametrize("seed", range(16))
def test_indexer_topk_random_configs(dev, seed):
    """Lightning indexer + exact top-k over random batch, head count, length, top-k, per-row
    lengths (0 to L), offsets and planted ties: indices bit-exact against the oracle."""
    from oracle import dsa as D
    from mosaic_amd import ops
    rng = np.random.default_rng(9400 + seed)
    b = int(rng.integers(1, 5))
    h = int(rng.choice([16, 32, 48, 64]))
    l = int(rng.integers(1, 20001))
    topk = int(rng.choice([1, 5, 64, 256, 512, 1024, 2048]))
    q, qs = D.quantize_rows_e4m3(rng.standard_normal((b, h, 128)))
    k, ks = D.quantize_rows_e4m3(rng.standard_normal((b, l, 128)))
    w = (rng.standard_normal((b, h)) * (128 ** -0.5) * (h ** -0.5)).astype(np.float32)
    if seed % 3 == 0 and l > 8:  # exact ties: one key row copied over a run of positions
        a = int(rng.integers(0, l // 2))
        k[:, a:a + l // 3] = k[:, a:a + 1]
        ks[:, a:a + l // 3] = ks[:, a:a + 1]
    lengths = None
    if seed % 2 == 1:
        lengths = rng.integers(0, l + 1, size=b).astype(np.int32)
        lengths[0] = l if b > 1 else lengths[0]
    offset = int(rng.integers(0, 51))
    T = lambda v: torch.from_numpy(np.ascontiguousarray(v)).to(dev)
    got = ops.dsa_indexer_topk(T(q), T(qs), T(k), T(ks), T(w), topk,
                               lengths=None if lengths is None else T(lengths), offset=offset).cpu().numpy()
    want = D.indexer_topk(q, qs, k, ks, w, topk, lengths, offset)
    np.testing.assert_array_equal(got, want, err_msg=f"b={b} h={h} l={l} topk={topk} lengths={lengths}")


@pytest.mark.parametrize("seed", range(12))
def test_mla_decode_random_configs(dev, seed):
    """MLA decode over the FP8 latent cache at random batch, head count, cache length, pick
    count, scale block, sink and masked picks, against the oracle."""
    from oracle import dsa as D
    from mosaic_amd import ops
    rng = np.random.default_rng(9500 + seed)
    b = int(rng.integers(1, 9))
    h = int(rng.choice([16, 32, 48, 64, 128, 192, 256]))
    n = int(rng.integers(16, 6001))
    t = int(rng.integers(1, min(n, 3000) + 1))
    sb = int(rng.choice([64, 128, 512]))
    masked = float(rng.choice([0.0, 0.1, 0.5]))
    q = C.round_bf16(rng.standard_normal((b, h, 576)).astype(np.float32))
    lat, ls = D.quantize_rows_e4m3(rng.standard_normal((b, n, 512 // sb, sb)) * 2.0)
    lat = lat.reshape(b, n, 512)
    rope = C.round_bf16(rng.standard_normal((b, n, 64)).astype(np.float32))
    idx = np.stack([rng.choice(n, t, replace=False) for _ in range(b)]).astype(np.int32)
    idx[rng.random(idx.shape) < masked] = -1
    snk = rng.standard_normal(h).astype(np.float32) if seed % 2 else None
    T = lambda v: torch.from_numpy(np.ascontiguousarray(v)).to(dev)
    out = ops.mla_sparse_decode(T(q).to(torch.bfloat16), T(lat), T(ls), T(rope).to(torch.bfloat16), T(idx),
                                576 ** -0.5, None if snk is None else T(snk))
    _close(out.float().cpu().numpy(), D.mla_sparse_decode(q, lat, ls, rope, snk, idx, 576 ** -0.5, sb),
           f"mla b={b} h={h} n={n} t={t} sb={sb} masked={masked}")


@pytest.mark.parametrize("seed", range(12))
def test_sparse_attn_fused_random_configs(dev, seed):
    """sparse_attn_fused (V = K) at head dims 64, 128, 256 and 512 with random rows, head
    counts (padded to 16), cache lengths, pick counts and masked picks (all masked included)."""
    from oracle import dsa as D
    from mosaic_amd.kernels.dsa import sparse_attn_fused
    rng = np.random.default_rng(9600 + seed)
    d = int(rng.choice([64, 128, 256, 512]))
    s = int(rng.integers(1, 7))
    h = int(rng.integers(1, 81))
    n = int(rng.integers(1, 3001))
    t = int(rng.integers(1, 1201))
    masked = float(rng.choice([0.0, 0.3, 1.0]))
    q = C.round_bf16(rng.standard_normal((s, h, d)).astype(np.float32))
    kv = C.round_bf16(rng.standard_normal((n, d)).astype(np.float32))
    idx = rng.integers(0, n, size=(s, t)).astype(np.int32)
    idx[rng.random(idx.shape) < masked] = -1
    sink = rng.standard_normal(h).astype(np.float32)
    T = lambda v: torch.from_numpy(np.ascontiguousarray(v)).to(dev)
    o = sparse_attn_fused(T(q).to(torch.bfloat16), T(kv).to(torch.bfloat16), T(sink), T(idx), d ** -0.5)
    _close(o.float().cpu().numpy(), D.sparse_attn(q, kv[None], sink, idx, d ** -0.5, d, s),
           f"sparse_attn d={d} s={s} h={h} n={n} t={t} masked={masked}")
