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
                                   # decode ring kernel (M <= 16, N >= 4096): full rows, ragged N, uneven K parts;
                                   # tiles x K parts 2x2, 1x4, 1x8 (M > 4), 1x8 (M <= 4), 1x2
                                   (16, 7168, 4096), (3, 4100, 1024), (7, 5000, 2176), (2, 4096, 1152)])
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
                                        (5, 16, 128, False)])
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
