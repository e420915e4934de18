"""Pins the linear oracles (CPU): brute force, closed forms, the integer-exact
restatement and the reference's own C kernel (oracle/_ref, when built)."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import codecs as C
from oracle import linear as L
from oracle import ref_c


def _rand_mx(rng, n, k, std=0.02):
    return C.quantize_mxfp4_ceil((rng.standard_normal((n, k)) * std).astype(np.float32))


def test_a16_brute_force_tiny():
    rng = np.random.default_rng(0)
    m, n, k = 2, 3, 64
    packed, scale = _rand_mx(rng, n, k, std=1.0)
    x = C.round_bf16(rng.standard_normal((m, k)).astype(np.float32))
    got = L.mx_linear_a16(x, packed, scale, out_bf16=False)
    codes = C.unpack_codes(packed)
    for i in range(m):
        for j in range(n):
            acc = 0.0
            for kk in range(k):
                w = float(C.E2M1_LUT[codes[j, kk]]) * 2.0 ** (int(scale[j, kk // 32]) - 127)
                acc += float(x[i, kk]) * w
            assert got[i, j] == np.float32(acc)


def test_kn_a16_pins():
    """mx_linear_kn_a16 (KN layout of kernels/skinny_fp4.py:50-144: packed [K, N/2], one e8m0 per 32
    consecutive N): a one-hot x selects a dequantized ROW of the KN weight; brute force (a
    double-precision sum per output) on a small case; and a planted reversal of N fails."""
    rng = np.random.default_rng(5)
    k, n = 96, 64
    packed, scale = _rand_mx(rng, k, n, std=1.0)         # KN: rows are K, blocks of 32 along N
    wkn = C.dequant_mxfp4(packed, scale)                   # [K, N]
    x = np.eye(k, dtype=np.float32)[[0, 7, 95]]
    np.testing.assert_array_equal(L.mx_linear_kn_a16(x, packed, scale, out_bf16=False), wkn[[0, 7, 95]])
    xr = C.round_bf16(rng.standard_normal((3, k)).astype(np.float32))
    got = L.mx_linear_kn_a16(xr, packed, scale, out_bf16=False)
    want = np.array([[sum(float(xr[i, kk]) * float(wkn[kk, j]) for kk in range(k)) for j in range(n)]
                     for i in range(3)], dtype=np.float32)
    np.testing.assert_array_equal(got, want)
    assert not np.array_equal(got, (xr.astype(np.float64) @ wkn[:, ::-1].astype(np.float64)).astype(np.float32))


def test_a16_onehot_selects_column():
    rng = np.random.default_rng(1)
    packed, scale = _rand_mx(rng, 16, 128, std=1.0)
    x = np.eye(128, dtype=np.float32)[:5]
    np.testing.assert_array_equal(L.mx_linear_a16(x, packed, scale, out_bf16=False),
                                  C.dequant_mxfp4(packed, scale)[:, :5].T)


def test_a8_equals_integer_exact_restatement():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4, 512)).astype(np.float32)
    packed, scale = _rand_mx(rng, 24, 512)
    codes, sa = C.act_quant(x, 128, "pow2")
    got = L.mx_linear_a8(x, packed, scale, out_bf16=False)
    ref = L.a8_integer_exact(codes, sa, packed, scale)
    np.testing.assert_array_equal(got, ref)


def test_a8_vs_reference_c_kernel():
    """bench/vnni_source_kernel.c compiled from the reference sources (oracle/Makefile)."""
    lib = ref_c.library()
    if lib is None:
        pytest.skip("oracle/_ref not built or CPU lacks VNNI")
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 1024)).astype(np.float32)
    packed, scale = _rand_mx(rng, 40, 1024)
    codes, sa = C.act_quant(x, 128, "pow2")
    y = ref_c.gemm(codes, sa, ref_c.prepare_weights(packed, scale), lib)
    np.testing.assert_array_equal(y, L.a8_integer_exact(codes, sa, packed, scale))
    np.testing.assert_array_equal(y, L.mx_linear_a8(x, packed, scale, out_bf16=False))


def test_a8_is_close_to_a16_but_not_equal():
    """The two numeric contracts differ by activation quantization (about 3% RMS)."""
    rng = np.random.default_rng(4)
    x = C.round_bf16(rng.standard_normal((2, 2048)).astype(np.float32))
    packed, scale = _rand_mx(rng, 64, 2048)
    a16 = L.mx_linear_a16(x, packed, scale, out_bf16=False)
    a8 = L.mx_linear_a8(x, packed, scale, out_bf16=False)
    rel = np.sqrt(np.mean((a8 - a16) ** 2) / np.mean(a16 ** 2))
    assert 0.002 < rel < 0.08


def test_fp8_block_gemm_vs_dequant_matmul():
    rng = np.random.default_rng(5)
    m, n, k = 5, 200, 384
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    bq, bs = L.quantize_fp8_weight_128(w)
    assert bs.shape == (2, 3)
    aq, a_s = C.act_quant(x, 128, "amax")
    got = L.fp8_block_gemm(aq, a_s, bq, bs, out_bf16=False)
    ref = L.fp8_dequant_matmul(aq, a_s, bq, bs)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)
    # quantized weights reproduce w to e4m3 precision, block scale = amax / 448
    deq = C.e4m3_decode(bq) * np.repeat(np.repeat(bs, 128, 0)[:n], 128, 1)
    assert np.max(np.abs(deq - w)) <= np.max(np.abs(w)) * 2 ** -4
    assert np.float32(np.max(np.abs(w[:128, :128])) / 448) == bs[0, 0]


def test_fp8_w8a16_oracle_vs_dequant_matmul_and_onehot():
    """The block-wise W8A16 oracle (acc += dot(x, decode(w)) * s) equals the
    float64 dequant-then-matmul within fp32 reassociation, and a one-hot x picks
    the dequantized column exactly."""
    rng = np.random.default_rng(21)
    n, k = 192, 384
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    bq, bs = L.quantize_fp8_weight_128(w)
    wd = C.e4m3_decode(bq).astype(np.float64) * np.repeat(np.repeat(bs, 128, 0), 128, 1)[:n, :k]
    x = C.round_bf16(rng.standard_normal((3, k)).astype(np.float32))
    got = L.fp8_w8a16_linear(x, bq, bs)
    ref = C.round_bf16((x.astype(np.float64) @ wd.T).astype(np.float32))
    assert np.max(np.abs(got - ref) / np.maximum(1.0, np.abs(ref))) <= 2 ** -7
    onehot = np.zeros((1, k), dtype=np.float32)
    onehot[0, 200] = 1.0
    np.testing.assert_array_equal(L.fp8_w8a16_linear(onehot, bq, bs)[0], C.round_bf16(wd[:, 200].astype(np.float32)))
