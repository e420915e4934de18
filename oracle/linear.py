"""Linear-layer oracles (numpy) -- TEST INFRASTRUCTURE ONLY, see ``oracle/__init__``.

* ``mx_linear_a16`` (A7): the benchmark spec's "dequant-then-matmul": bf16 x against the
  exactly dequantized MXFP4 W, accumulated wide, rounded once to bf16.
  Restates ``x @ dequant_mxfp4(...)`` (``tests/test_skinny_fp4.py:23``,
  ``kernels/mxfp4.py:130-160``) and the per-expert matmuls of
  ``grouped_expert_forward`` (``model/layers.py:353-365``).
* ``mx_linear_kn_a16`` (A8, skinny): ``skinny_mxfp4_gemm``
  (``kernels/skinny_fp4.py:113-144``) on the KN layout: W [K, N] =
  ``dequant_mxfp4`` of packed [K, N/2] + scale [K, N/32] (blocks of 32 along N),
  y = x @ W accumulated wide, one bf16 rounding.
* ``mx_linear_a8`` (A6): ``reference_fp4_linear_source_semantics``
  (``kernels/fp4_source.py:132-156``): act_quant_ref then, for K32 groups in
  ascending order, acc += (A_g . B_g^T) * sA[:, g//4] * sW[:, g] in fp32.
  Upstream ``fp4_gemm`` (``.mosaicvm/source/inference_kernel.py:441-536``) is the
  same contract.
* ``fp8_block_gemm`` (A18): upstream ``fp8_gemm``
  (``.mosaicvm/source/inference_kernel.py:203-273``): per 128-K block the block
  product is scaled by a_s[m, kb] * b_s[n // 128, kb] and added to an fp32
  accumulator.
* ``fp8_w8a16_linear`` (A18, W8A16): the fused decode kernel of ``fp8_linear``
  (``bench/fp8_core.py:160-194``): per 128-K block, acc += dot(x, decode(w)) * s
  in fp32 (x bf16, w e4m3 decoded without its scale), one bf16 rounding.
* ``quantize_fp8_weight_128`` (config 3 weights): per 128x128 block s =
  amax / 448 (``.mosaicvm/source/hubkernel_act_quant.py:27-35`` restated on
  weight blocks), codes = e4m3(w / s).

Pinned by ``tests/test_oracle_linear.py``: the A6 form is checked against the
integer-exact C1 algorithm of ``bench/vnni_source_kernel.c:8-47`` compiled from
the reference sources into ``oracle/_ref`` (when built) and against a pure
Python restatement of the same integer algorithm; A7 against a float64
brute-force dot on tiny shapes and against closed forms (one-hot x picks a
dequantized column, all-ones scales with constant codes); the FP8 block GEMM
against a float64 dequant-then-matmul of the same codes.
"""
from __future__ import annotations

import numpy as np

from . import codecs as C


def mx_linear_a16(x: np.ndarray, packed: np.ndarray, scale: np.ndarray,
                  out_bf16: bool = True) -> np.ndarray:
    """x [M, K] (bf16-valued) , packed [N, K/2], e8m0 [N, K/32] -> y [M, N].

    Products of a bf16 value and a dequantized E2M1*2^k weight are exact; the
    sum is taken in float64 and rounded once (fp32, then bf16 if requested)."""
    x = np.asarray(x, dtype=np.float32)
    w = C.dequant_mxfp4(packed, scale).astype(np.float64)
    y = (x.astype(np.float64) @ w.T).astype(np.float32)
    return C.round_bf16(y) if out_bf16 else y


def mx_linear_kn_a16(x: np.ndarray, packed: np.ndarray, scale: np.ndarray, out_bf16: bool = True) -> np.ndarray:
    """x [M, K] (bf16-valued), KN packed [K, N/2] + e8m0 [K, N/32] -> y [M, N]."""
    w = C.dequant_mxfp4(packed, scale).astype(np.float64)            # [K, N]
    y = (np.asarray(x, dtype=np.float64) @ w).astype(np.float32)
    return C.round_bf16(y) if out_bf16 else y


def mx_linear_a8(x: np.ndarray, packed: np.ndarray, scale: np.ndarray,
                 out_bf16: bool = True, quant: tuple | None = None) -> np.ndarray:
    """A8 "source semantics" linear (``kernels/fp4_source.py:132-156``).

    ``quant`` optionally supplies (codes u8 [M, K], sA fp32 [M, K/128]) already
    quantized; otherwise ``act_quant_ref`` is applied to ``x``."""
    if quant is None:
        codes, sa = C.act_quant(np.asarray(x, dtype=np.float32), C.ACT_BLOCK, "pow2")
    else:
        codes, sa = quant
    a = C.e4m3_decode(codes).astype(np.float64)            # [M, K]
    b = C.decode_e2m1(packed).astype(np.float64)           # [N, K]
    sw = C.e8m0_to_f32(scale)                              # [N, G]
    m, k = a.shape
    n = b.shape[0]
    g = k // C.MX_BLOCK
    # partial[m, n, g] of the K32 group dot; exact in float64 (every term is
    # a multiple of 2^-10 with magnitude < 2^12), then one fp32 rounding, as
    # the reference's fp32 matmul of those 32 exact products gives when the
    # partial fits 24 bits
    acc = np.zeros((m, n), dtype=np.float32)
    ar = a.reshape(m, g, C.MX_BLOCK)
    br = b.reshape(n, g, C.MX_BLOCK)
    for gi in range(g):
        part = (ar[:, gi, :] @ br[:, gi, :].T).astype(np.float32)
        part = (part * sa[:, gi * C.MX_BLOCK // C.ACT_BLOCK][:, None]).astype(np.float32)
        part = (part * sw[None, :, gi]).astype(np.float32)
        acc = (acc + part).astype(np.float32)
    return C.round_bf16(acc) if out_bf16 else acc


def quantize_fp8_weight_128(w: np.ndarray, block: int = 128):
    """w [N, K] -> (codes u8 [N, K], scale fp32 [ceil(N/128), K/128]), s = amax/448
    per 128x128 block (a partial last row-block uses the rows present)."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    if k % block:
        raise ValueError(f"K={k} must be a multiple of {block}")
    nb = (n + block - 1) // block
    kb = k // block
    s = np.zeros((nb, kb), dtype=np.float32)
    codes = np.zeros((n, k), dtype=np.uint8)
    for i in range(nb):
        r0, r1 = i * block, min(n, (i + 1) * block)
        blk = w[r0:r1].reshape(r1 - r0, kb, block)
        amax = np.max(np.abs(blk), axis=(0, 2)).astype(np.float32)
        si = (amax / np.float32(C.FP8_MAX)).astype(np.float32)
        si = np.where(si == 0, np.float32(1.0), si)
        s[i] = si
        q = np.clip(blk / si[None, :, None], -C.FP8_MAX, C.FP8_MAX).astype(np.float32)
        codes[r0:r1] = C.e4m3_encode(q).reshape(r1 - r0, k)
    return codes, s


def fp8_block_gemm(a_codes: np.ndarray, a_s: np.ndarray, b_codes: np.ndarray,
                   b_s: np.ndarray, out_bf16: bool = True, block: int = 128) -> np.ndarray:
    """C[M, N] = sum_kb (A_kb . B_kb^T) * a_s[m, kb] * b_s[n//128, kb]
    (``.mosaicvm/source/inference_kernel.py:237-250``: Scale_C = a_s * b_s, then
    C_accum += C_block * Scale_C, fp32)."""
    a = C.e4m3_decode(a_codes).astype(np.float64)
    b = C.e4m3_decode(b_codes).astype(np.float64)
    m, k = a.shape
    n = b.shape[0]
    kb = k // block
    acc = np.zeros((m, n), dtype=np.float32)
    rowblk = np.arange(n) // block
    for j in range(kb):
        part = (a[:, j * block:(j + 1) * block] @ b[:, j * block:(j + 1) * block].T).astype(np.float32)
        sc = (a_s[:, j][:, None] * b_s[rowblk, j][None, :]).astype(np.float32)
        acc = (acc + (part * sc).astype(np.float32)).astype(np.float32)
    return C.round_bf16(acc) if out_bf16 else acc


def fp8_dequant_matmul(a_codes, a_s, b_codes, b_s, block: int = 128) -> np.ndarray:
    """float64 dequant-then-matmul of the same FP8 operands (pin for
    ``fp8_block_gemm``; ``runtime/fp8.py:52-64`` dequant form)."""
    a = C.e4m3_decode(a_codes).astype(np.float64)
    b = C.e4m3_decode(b_codes).astype(np.float64)
    m, k = a.shape
    n = b.shape[0]
    a = a * np.repeat(a_s.astype(np.float64), block, axis=1)[:, :k]
    bs = np.repeat(np.repeat(b_s.astype(np.float64), block, axis=0)[:n], block, axis=1)[:, :k]
    return a @ (b * bs).T


def a8_integer_exact(codes: np.ndarray, sa: np.ndarray, packed: np.ndarray,
                     scale: np.ndarray) -> np.ndarray:
    """Integer-exact A8 linear, the algorithm of ``bench/vnni_source_kernel.c:8-47``:
    qA = 512*A (int), qW = 2*W (int), per K32 the exact int dot, then
    fp32 partial = dot * (1/1024) * sa * sw accumulated in ascending K32 order."""
    qa = np.rint(C.e4m3_decode(codes).astype(np.float64) * 512).astype(np.int64)
    qw = np.rint(C.decode_e2m1(packed).astype(np.float64) * 2).astype(np.int64)
    sw = C.e8m0_to_f32(scale)
    m, k = qa.shape
    n = qw.shape[0]
    g = k // C.MX_BLOCK
    acc = np.zeros((m, n), dtype=np.float32)
    for gi in range(g):
        sl = slice(gi * 32, gi * 32 + 32)
        dot = qa[:, sl] @ qw[:, sl].T
        part = (dot.astype(np.float32) * np.float32(1.0 / 1024.0)).astype(np.float32)
        part = (part * sa[:, gi // 4][:, None]).astype(np.float32)
        part = (part * sw[None, :, gi]).astype(np.float32)
        acc = (acc + part).astype(np.float32)
    return acc


def fp8_w8a16_linear(x: np.ndarray, w_codes: np.ndarray, s: np.ndarray, block: int = 128) -> np.ndarray:
    """x [M, K] (bf16-valued), e4m3 codes [N, K], fp32 scales [ceil(N/128), K/128] -> bf16 [M, N]."""
    x = np.asarray(x, dtype=np.float64)
    wd = C.e4m3_decode(w_codes).astype(np.float64)
    n, k = wd.shape
    acc = np.zeros((x.shape[0], n), dtype=np.float32)
    rows = np.arange(n) // block
    for kb in range(k // block):
        sl = slice(kb * block, (kb + 1) * block)
        d = (x[:, sl] @ wd[:, sl].T).astype(np.float32)
        acc = (acc + (d * s[rows, kb][None, :]).astype(np.float32)).astype(np.float32)
    return C.round_bf16(acc)
