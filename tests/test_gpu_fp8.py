"""GPU parity of the FP8 block-scaled GEMM against the CPU oracle (A18).

Float bar |got - ref| <= 2e-2 * max(1, |ref|) against the oracle's block
GEMM of identical e4m3 codes and fp32 scales (config 3 recipe: W ~ N(0,1)*0.02
quantized per 128x128 with s = amax/448, x ~ N(0,1) per 1x128)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import codecs as C
from oracle import linear as L

pytestmark = pytest.mark.gpu


def _case(rng, m, n, k):
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    bq, bs = L.quantize_fp8_weight_128(w)
    aq, a_s = C.act_quant(x, 128, "amax")
    return aq, a_s, bq, bs


@pytest.mark.parametrize("m,n,k", [(1, 16, 128), (1, 1536, 7168), (16, 576, 7168), (3, 200, 384), (37, 130, 256),
                                   (128, 256, 1536), (1, 24576, 1536), (64, 7168, 512),
                                   (256, 128, 128), (300, 576, 1024), (1024, 1536, 2048), (513, 700, 384),
                                   (129, 8200, 512), (200, 640, 1536), (96, 1536, 7168), (2304, 7200, 384),
                                   (1024, 16384, 384), (1024, 16384, 2304),
                                   # persistent big-tile grid with more tiles than CUs: a tile's last scale
                                   # chunk of 1 / 3 blocks, ragged N, ragged M (the next tile's first stage
                                   # and scale chunk go out during the current tile's last blocks)
                                   (4096, 4608, 1152), (2560, 7000, 1408), (4000, 4352, 640),
                                   # split K (tiles under half the GPU): tiled<128> x 8 / x 4, tiled<256> x 3
                                   (128, 576, 7168), (128, 7168, 4096), (4096, 576, 7168),
                                   # split K whose slices of ceil(K-blocks / S) would leave the last ones
                                   # empty (33 blocks in 8 slices of 5, 25 in 6 of 5): 7 and 5 slices run
                                   (128, 512, 4224), (256, 512, 4224), (128, 768, 3200), (256, 640, 3200),
                                   # decode ring kernel (M <= 16, N >= 4096): full rows, ragged N, uneven K parts;
                                   # tiles x K parts 2x2, 1x4, 1x8 (M > 4), 1x8 (M <= 4), 1x2
                                   (16, 7168, 4096), (3, 4100, 1024), (7, 5000, 2176), (2, 4096, 1152),
                                   # mid kernel (17..64 rows, N % 16 == 0, weights of 8 MB and more): 2 and
                                   # 4 row groups, ragged rows, partial workgroups, K splits of 8 / 7 / none;
                                   # and the tiled kernel at 65..95 rows
                                   (17, 1280, 7168), (33, 1024, 8192), (50, 2064, 4096), (64, 4096, 2048),
                                   (61, 2048, 8192), (24, 18432, 512), (80, 2048, 4096)])
@pytest.mark.parametrize("out", ["bf16", "f32"])
def test_fp8_block_gemm_vs_oracle(dev, m, n, k, out):
    from mosaic_amd import ops
    rng = np.random.default_rng(m * 7 + n + k)
    aq, a_s, bq, bs = _case(rng, m, n, k)
    T = lambda v: torch.from_numpy(np.ascontiguousarray(v)).to(dev)
    c = ops.fp8_block_gemm(T(aq), T(a_s), T(bq), T(bs), out_dtype=torch.bfloat16 if out == "bf16" else torch.float32)
    ref = L.fp8_block_gemm(aq, a_s, bq, bs, out_bf16=(out == "bf16"))
    got = c.float().cpu().numpy()
    err = np.abs(got - ref) / np.maximum(1.0, np.abs(ref))
    assert err.max() <= 2e-2, f"max scaled err {err.max()}"
    if out == "f32":
        # fp32 output: only the order of the fp32 additions differs from the
        # oracle (MFMA inner sums, K slices summed across waves), so
        # |got - ref| <= gamma_n * sum |terms| with n = K/128 block partials +
        # 128 products per block (gamma_n ~ n * 2^-24; factor 2 for the scale products)
        abs_sum = L.fp8_block_gemm(aq & 0x7F, a_s, bq & 0x7F, np.abs(bs), out_bf16=False)
        bound = 2.0 * (k // 128 + 128) * 2.0 ** -24 * abs_sum + 1e-30
        viol = np.abs(got - ref) - bound
        assert viol.max() <= 0, f"f32 reassociation bound exceeded by {viol.max()} (max scaled err {err.max()})"


@pytest.mark.parametrize("m,n,k,e8m0", [(1, 1536, 7168, False), (1, 18432, 7168, True), (16, 576, 7168, False),
                                        (37, 200, 1024, True), (80, 4096, 512, False), (3, 24576, 1536, True),
                                        (5, 16, 128, False),
                                        # 17..80 rows, N >= 4096 (the mid kernel): 2, 4 and 5 row groups, N not a
                                        # multiple of 16 / 128, one K block, K past one ring chunk; and below
                                        (17, 4096, 2048, False), (64, 4112, 1024, True), (50, 4100, 384, False),
                                        (72, 4096, 128, True), (33, 4608, 9216, False), (40, 1536, 1024, False),
                                        # 4..16 rows, K >= 48 blocks, wide N: the mid kernel with one row group
                                        (4, 16384, 6144, False), (12, 16384, 6144, True), (16, 18432, 6144, False),
                                        (1, 18432, 6144, True), (12, 24576, 1536, False), (16, 18432, 2048, True),
                                        # 17..80 rows over few tiles: the mid kernel with K split (2 and 4 slices,
                                        # N % 16 != 0 with 5 row groups)
                                        (32, 7168, 8192, False), (64, 4096, 7168, True), (80, 4100, 3072, False),
                                        # 6 and 7 compute waves (K split 4 ways), and 5 row groups past 256
                                        # workgroups (7 waves)
                                        (64, 24576, 1536, False), (48, 7168, 6144, True), (72, 32768, 512, False),
                                        # 12..16 rows, a weight of >= 40 MB over few tiles: one row group, K split
                                        (16, 7168, 8192, False),
                                        # 33..80 rows over 1536..4095 columns: the mid kernel with a K split
                                        (64, 2048, 4096, True), (80, 1536, 7168, False)])
def test_fp8_w8a16_linear_vs_oracle(dev, m, n, k, e8m0):
    """fp8_linear's fused decode (bench/fp8_core.py:160-194) against the oracle of
    identical codes and scales: bar 2e-2 * max(1, |ref|)."""
    from mosaic_amd.kernels import fp8
    rng = np.random.default_rng(m + n + k)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    bq, bs = L.quantize_fp8_weight_128(w)
    if e8m0:  # power-of-two block scales, passed as float8_e8m0fnu like the reference's checkpoints
        e = np.clip(np.ceil(np.log2(bs)), -127, 127).astype(np.int32)
        bs = np.exp2(e).astype(np.float32)
        bq = C.e4m3_encode(np.clip(w / np.repeat(np.repeat(bs, 128, 0), 128, 1)[:n, :k], -448, 448))
        s_dev = torch.from_numpy((e + 127).astype(np.uint8)).to(dev).view(torch.float8_e8m0fnu)
    else:
        s_dev = torch.from_numpy(bs).to(dev)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(torch.bfloat16)
    y = fp8.fp8_linear(x.to(dev), torch.from_numpy(bq).to(dev).view(torch.float8_e4m3fn), s_dev)
    ref = L.fp8_w8a16_linear(x.float().numpy(), bq, bs)
    err = np.abs(y.float().cpu().numpy() - ref) / np.maximum(1.0, np.abs(ref))
    assert err.max() <= 2e-2, err.max()


@pytest.mark.parametrize("m,n,k", [(32, 7168, 8192), (80, 4100, 3072), (12, 7168, 8192)])
def test_fp8_w8a16_split_matches_unsplit_entry(dev, m, n, k):
    """The workspace entry splits K for these shapes (fp32 partials summed in slice
    order); the plain entry runs the whole K in one pass: both within the float bar
    of the oracle, and within fp32 reassociation of each other."""
    from mosaic_amd import _lib, ops
    assert _lib.lib().mosaic_fp8_w8a16_workspace_bytes(m, n, k) > 0
    rng = np.random.default_rng(m + 7 * n + k)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    bq, bs = L.quantize_fp8_weight_128(w)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(torch.bfloat16).to(dev)
    wd, sd = torch.from_numpy(bq).to(dev), torch.from_numpy(bs).to(dev)
    y_split = ops.fp8_w8a16_linear(x, wd, sd)
    y_one = torch.empty_like(y_split)
    _lib.call("mosaic_fp8_w8a16_linear", x.data_ptr(), wd.data_ptr(), sd.data_ptr(), y_one.data_ptr(), m, n, k,
              torch.cuda.current_stream().cuda_stream)
    ref = L.fp8_w8a16_linear(x.float().cpu().numpy(), bq, bs)
    for y in (y_split, y_one):
        err = np.abs(y.float().cpu().numpy() - ref) / np.maximum(1.0, np.abs(ref))
        assert err.max() <= 2e-2, err.max()
    diff = (y_split.float() - y_one.float()).abs() / y_one.float().abs().clamp_min(1.0)
    assert diff.max().item() <= 2 ** -7  # one bf16 rounding apart at most


def _device_fp8_case(dev, m, n, k, seed):
    """The config-3 recipe on the device (as bench.py generates it): W ~ N(0, 0.02)
    quantized per 128 x 128 with s = amax / 448, x ~ N(0, 1) per 1 x 128 (amax)."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    nb = (n + 127) // 128
    w = torch.zeros(nb * 128, k, device=dev)
    w[:n] = torch.randn(n, k, generator=g, device=dev) * 0.02
    wb = w.view(nb, 128, k // 128, 128)
    bs = (wb.abs().amax(dim=(1, 3)) / 448.0).clamp_min(1e-12)
    bq = (wb / bs[:, None, :, None]).clamp(-448, 448).reshape(-1, k)[:n].to(torch.float8_e4m3fn)
    x = torch.randn(m, k, generator=g, device=dev).view(m, k // 128, 128)
    a_s = (x.abs().amax(dim=2) / 448.0).clamp_min(1e-12)
    aq = (x / a_s[:, :, None]).clamp(-448, 448).reshape(m, k).to(torch.float8_e4m3fn)
    return aq, a_s, bq, bs


@pytest.mark.parametrize("n,k", [(7168, 16384), (18432, 7168), (24576, 1536), (1536, 7168), (576, 7168)])
def test_fp8_block_gemm_config3_m4096(dev, n, k):
    """The timed config-3 GEMMs at M = 4096, full size (the 256 x 256 big-tile
    kernel for the first three: 448, 1152 and 1536 tiles over 56, 128 and 12
    K-blocks; tiled<256> and its split-K for N = 1536 and 576): every column of
    eight sampled rows (the first and last of 256-row tiles among them) against
    the oracle of identical codes and scales."""
    from mosaic_amd import ops
    m = 4096
    aq, a_s, bq, bs = _device_fp8_case(dev, m, n, k, seed=n + k)
    c = ops.fp8_block_gemm(aq, a_s, bq, bs, out_dtype=torch.bfloat16)
    rows = [0, 255, 256, 2047, 2048, 4095] + np.random.default_rng(n).choice(m, 2, replace=False).tolist()
    ref = L.fp8_block_gemm(aq[rows].view(torch.uint8).cpu().numpy(), a_s[rows].cpu().numpy(),
                           bq.view(torch.uint8).cpu().numpy(), bs.cpu().numpy(), out_bf16=True)
    got = c[rows].float().cpu().numpy()
    err = np.abs(got - ref) / np.maximum(1.0, np.abs(ref))
    assert err.max() <= 2e-2, f"({m}, {n}, {k}): max scaled err {err.max()}"
    assert torch.isfinite(c.float()).all()


def _t16_layout(w: np.ndarray) -> np.ndarray:
    """The T16 byte order by axis permutation: W [G*16 (c), nkb*128 (h, q, j)] viewed
    as [G, c, nkb, h, q, j] and laid out as [G, nkb, h, c, q, j]."""
    n, k = w.shape
    return w.reshape(n // 16, 16, k // 128, 2, 4, 16).transpose(0, 2, 3, 1, 4, 5).reshape(n, k)


@pytest.mark.parametrize("n,k", [(16, 128), (48, 384), (576, 7168), (4096, 1536)])
def test_fp8_t16_prepack_layout_and_inverse(dev, n, k):
    from mosaic_amd import ops
    w = np.random.default_rng(n + k).integers(0, 256, (n, k), dtype=np.uint8)
    t = ops.fp8_t16_prepack(torch.from_numpy(w).to(dev))
    assert (t.n, t.k) == (n, k)
    assert np.array_equal(t.codes.cpu().numpy(), _t16_layout(w))
    assert np.array_equal(ops.fp8_t16_unpack(t).cpu().numpy(), w)


def test_fp8_t16_rejects_bad_shapes(dev):
    from mosaic_amd import ops
    for n, k in [(20, 128), (16, 200)]:
        with pytest.raises(ValueError):
            ops.fp8_t16_prepack(torch.zeros(n, k, dtype=torch.uint8, device=dev))
    t = ops.fp8_t16_prepack(torch.zeros(32, 256, dtype=torch.uint8, device=dev))
    a = torch.zeros(65, 256, dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError):
        ops.fp8_block_gemm(a, torch.ones(65, 2, device=dev), t, torch.ones(1, 2, device=dev))


# every ring plan: K parts of 8 / 4 / 2 (one tile) and 2 / 4 (two tiles), ring
# depths 3..8, short K (4 waves of 3 blocks), ragged K parts; N from one tile to
# 24576 columns with N % 128 != 0 among them
@pytest.mark.parametrize("m,n,k", [(1, 16, 128), (1, 576, 7168), (4, 1536, 1536), (1, 4096, 1536),
                                   (2, 24576, 1536), (3, 7168, 2048), (1, 7168, 16384), (4, 18432, 1024),
                                   (5, 2048, 1536), (16, 576, 7168), (16, 7168, 2048), (16, 24576, 1536),
                                   (7, 6160, 1152), (16, 8192, 7168), (9, 4112, 640), (1, 1552, 2304),
                                   # the mid kernel over the prepack (17..64 rows)
                                   (17, 576, 7168), (32, 1536, 1536), (33, 48, 8192), (50, 2064, 1024),
                                   (64, 4096, 2048), (40, 16, 128), (24, 18432, 256),
                                   # 12..16 rows on very wide shapes with K >= 48 blocks: the
                                   # mid kernel with one row group instead of the ring
                                   (12, 16384, 6144), (16, 18432, 6144),
                                   # 6, 7 (K split 4 ways) and 8 compute waves a workgroup
                                   (20, 24576, 1536), (40, 7168, 4096), (24, 32768, 1024)])
@pytest.mark.parametrize("out", ["bf16", "f32"])
def test_fp8_block_gemm_t16_vs_oracle(dev, m, n, k, out):
    """The GEMM over the T16 prepack: against the oracle (the float bar, and the
    fp32 reassociation bound for an f32 output), and bit for bit against the
    checkpoint-layout call wherever that one runs the same ring kernel."""
    from mosaic_amd import ops
    rng = np.random.default_rng(m * 11 + n + 3 * k)
    aq, a_s, bq, bs = _case(rng, m, n, k)
    T = lambda v: torch.from_numpy(np.ascontiguousarray(v)).to(dev)
    od = torch.bfloat16 if out == "bf16" else torch.float32
    c = ops.fp8_block_gemm(T(aq), T(a_s), ops.fp8_t16_prepack(T(bq)), T(bs), out_dtype=od)
    ref = L.fp8_block_gemm(aq, a_s, bq, bs, out_bf16=(out == "bf16"))
    got = c.float().cpu().numpy()
    err = np.abs(got - ref) / np.maximum(1.0, np.abs(ref))
    assert err.max() <= 2e-2, f"max scaled err {err.max()}"
    if out == "f32":
        abs_sum = L.fp8_block_gemm(aq & 0x7F, a_s, bq & 0x7F, np.abs(bs), out_bf16=False)
        bound = 2.0 * (k // 128 + 128) * 2.0 ** -24 * abs_sum + 1e-30
        assert (np.abs(got - ref) - bound).max() <= 0
    nkb = k // 128
    # the checkpoint-layout call runs the same ring plan (K parts included): ring
    # shapes, except short K with two-tile workgroups, split 2 ways there; and
    # the same mid-kernel plan at 17..64 rows for weights of 8 MB and more (and
    # at 12..16 rows where both layouts take the mid kernel)
    two_tile = m > 4 and (n + 31) // 32 >= 192
    ring = m <= 16 and nkb >= 8 and (n >= 4096 or nkb >= 32) and not (nkb <= 16 and two_tile)
    if ring or (m > 16 and n * k >= 8 << 20):
        c_raw = ops.fp8_block_gemm(T(aq), T(a_s), T(bq), T(bs), out_dtype=od)
        assert torch.equal(c, c_raw)


def test_fp8_gemm_dropin_caches_t16(dev):
    """fp8_gemm / w8a8_block_fp8_matmul at M <= 64 read the cached T16 prepack:
    one cache entry per weight, the checkpoint-layout result bit for bit, and a
    new prepack after an in-place update of the weight."""
    from mosaic_amd import ops
    from mosaic_amd.kernels import _prepack_cache, fp8
    m, n, k = 2, 4096, 2048
    aq, a_s, bq, bs = _case(np.random.default_rng(5), m, n, k)
    T = lambda v: torch.from_numpy(np.ascontiguousarray(v)).to(dev)
    a, sa, b, sb = T(aq).view(torch.float8_e4m3fn), T(a_s), T(bq).view(torch.float8_e4m3fn), T(bs)
    _prepack_cache.clear()
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        c1 = fp8.fp8_gemm(a, sa, b, sb)
        assert _prepack_cache.size() == 1
        c2 = fp8.w8a8_block_fp8_matmul(a, b, sa, sb, [128, 128], torch.bfloat16)
        assert _prepack_cache.size() == 1
        raw = ops.fp8_block_gemm(a, sa, b, sb)
        assert torch.equal(c1, raw) and torch.equal(c2, raw)
        b.view(torch.uint8)[:16] = 0  # rows 0..15 now contribute nothing
        c3 = fp8.fp8_gemm(a, sa, b, sb)
        assert torch.equal(c3, ops.fp8_block_gemm(a, sa, b, sb))
        assert (c3[:, :16] == 0).all() and torch.equal(c3[:, 16:], raw[:, 16:])
    finally:
        torch.set_default_dtype(prev)
        _prepack_cache.clear()
