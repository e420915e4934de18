"""Codec restatements (numpy) -- TEST INFRASTRUCTURE ONLY, see ``oracle/__init__``.

Covers the element formats of the path:

* E2M1 nibbles and their LUT (A1): ``kernels/mxfp4.py:20-23``, ``_pack_uint4``
  ``kernels/mxfp4.py:85-88`` (low nibble = even K), ``decode_e2m1_nk``
  ``kernels/fp4_source.py:78-84``.
* E8M0 scale decode by exponent-field insertion (A2): ``e8m0_to_fp32``
  ``kernels/fp4_source.py:67-75``; byte 0x00 -> 0.0, 0xFF -> +inf
  (torch's ``float8_e8m0fnu`` would give 2^-127 / NaN).
* MXFP4 quantizers (A3): the benchmark spec's "ceil" recipe of the upstream
  ``fp4_quant_kernel`` (``.mosaicvm/source/inference_kernel.py:128-183``,
  ``fast_round_scale`` ``:23-37``) and the reference packer's FLOOR fallback
  (``kernels/mxfp4.py:32-82``, ``kernels/fp4_source.py:35-64``); both round E2M1
  to nearest-even with saturation at 6.
* E4M3 (OCP e4m3fn) decode/encode (A5) and the 1x128 activation quantizer (A4):
  ``act_quant_ref`` ``kernels/fp4_source.py:110-129`` (power-of-two scale from
  IEEE bits), upstream ``act_quant`` ``.mosaicvm/source/inference_kernel.py:40-125``
  (scale = amax * (1/448), amax >= 1e-4) and the HF variant
  ``.mosaicvm/source/hubkernel_act_quant.py:27-35`` (scale = amax / 448).

Pinned by ``tests/test_oracle_codecs.py``: the reference tests' KATs
(``tests/test_mxfp4.py:47-63``, ``tests/test_mxfp4_decode.py:20-63``,
``tests/test_fp4_source.py:23-63``), torch's own e4m3fn / e8m0 casts on every
byte and on a dense value sweep (the reference's e4m3 boundary is torch's
cast, ``tests/test_mxint_epilogue.py:24-58``), and brute-force nearest-value
search for the E2M1 rounding.
"""
from __future__ import annotations

import numpy as np

MX_BLOCK = 32
ACT_BLOCK = 128
FP8_MAX = 448.0
FP4_MAX = 6.0

# kernels/mxfp4.py:20-23 -- locked E2M1 table, codes 0..7 positive, 8..15 negative.
E2M1_LUT = np.array(
    [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
     -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=np.float32)


# ----------------------------------------------------------------- bf16 -----
def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit pattern, round-to-nearest-even (torch's ``.to(bf16)``)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(a)
    if nan.any():
        r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(a: np.ndarray) -> np.ndarray:
    """fp32 value after a round trip through bf16 (RNE)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(a))


# ----------------------------------------------------------------- E2M1 -----
def unpack_codes(packed: np.ndarray) -> np.ndarray:
    """packed u8 [..., K/2] -> 4-bit codes u8 [..., K]; low nibble = even K
    (``kernels/mxfp4.py:85-88``, ``kernels/fp4_source.py:80-83``)."""
    p = np.asarray(packed, dtype=np.uint8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = p & 0x0F
    out[..., 1::2] = p >> 4
    return out


def pack_codes(codes: np.ndarray) -> np.ndarray:
    """4-bit codes [..., K] -> packed u8 [..., K/2] (inverse of ``unpack_codes``)."""
    c = np.asarray(codes, dtype=np.uint8)
    return (c[..., 0::2] & 0x0F) | ((c[..., 1::2] & 0x0F) << 4)


def decode_e2m1(packed: np.ndarray) -> np.ndarray:
    """packed [..., K/2] -> fp32 E2M1 values [..., K] without block scale."""
    return E2M1_LUT[unpack_codes(packed)]


# ----------------------------------------------------------------- E8M0 -----
def e8m0_to_f32(scale_bytes: np.ndarray) -> np.ndarray:
    """e8m0 byte b -> 2^(b-127) by writing b into the fp32 exponent field
    (``kernels/fp4_source.py:67-75``: clamp(b-127, -127, 128) + 127 == b)."""
    b = np.asarray(scale_bytes, dtype=np.uint8).astype(np.uint32)
    return (b << 23).view(np.float32)


def dequant_mxfp4(packed: np.ndarray, scale_bytes: np.ndarray) -> np.ndarray:
    """NK dequant: packed [N, K/2] + e8m0 [N, K/32] -> fp32 [N, K]
    (``kernels/mxfp4.py:130-160`` with blocks along the last dim).  The
    product of an E2M1 value and a power of two is exact in fp32 and bf16."""
    vals = decode_e2m1(packed)
    s = np.repeat(e8m0_to_f32(scale_bytes), MX_BLOCK, axis=-1)
    with np.errstate(invalid="ignore", over="ignore"):
        return vals * s


# ------------------------------------------------------ E2M1 quantizers -----
def f32_to_e2m1_rne(v: np.ndarray) -> np.ndarray:
    """fp32 -> E2M1 code (u8, low 4 bits), round-to-nearest-even, saturating
    at +-6, NaN -> 7 | sign (restates ``_f32_to_e2m1`` ``kernels/mxfp4.py:46-82``
    by value: ties go to the code with an even mantissa bit)."""
    v = np.asarray(v, dtype=np.float32)
    sign = (np.signbit(v)).astype(np.uint8) << 3
    a = np.abs(v).astype(np.float64)
    # thresholds between grid points 0,.5,1,1.5,2,3,4,6; at an exact midpoint
    # the even code wins: .25->0, .75->1.0(c2), 1.25->1.0(c2), 1.75->2(c4),
    # 2.5->2(c4), 3.5->4(c6), 5->4(c6)
    code = np.zeros(a.shape, dtype=np.uint8)
    code = np.where(a > 0.25, 1, code)
    code = np.where(a >= 0.75, 2, code)
    code = np.where(a > 1.25, 3, code)
    code = np.where(a >= 1.75, 4, code)
    code = np.where(a > 2.5, 5, code)
    code = np.where(a >= 3.5, 6, code)
    code = np.where(a > 5.0, 7, code)
    code = np.where(np.isnan(a), 7, code).astype(np.uint8)
    return code | sign


def _f32_exponent_field(a: np.ndarray) -> np.ndarray:
    return ((np.asarray(a, dtype=np.float32).view(np.uint32) >> 23) & 0xFF).astype(np.int32)


def _f32_mantissa_field(a: np.ndarray) -> np.ndarray:
    return (np.asarray(a, dtype=np.float32).view(np.uint32) & 0x7FFFFF).astype(np.int64)


def pow2_ceil_scale(amax: np.ndarray, max_inv: float) -> np.ndarray:
    """``fast_round_scale`` (``.mosaicvm/source/inference_kernel.py:23-37``):
    v = amax * fp32(max_inv); e = exp(v) - 127 + (mantissa(v) != 0); 2^e by bits.
    Returns (scale fp32, biased exponent int32)."""
    v = (np.asarray(amax, dtype=np.float32) * np.float32(max_inv)).astype(np.float32)
    e = _f32_exponent_field(v) - 127 + (_f32_mantissa_field(v) != 0).astype(np.int32)
    biased = (e + 127).astype(np.int32)
    return (biased.astype(np.uint32) << 23).view(np.float32), biased


def quantize_mxfp4_ceil(w: np.ndarray):
    """The benchmark spec's recipe == upstream ``fp4_quant_kernel``
    (``.mosaicvm/source/inference_kernel.py:128-183``): per 32 contiguous
    elements of the last dim, amax = max|w| clamped to >= 6*2^-126, scale =
    2^ceil(log2(amax*(1/6))), codes = RNE-E2M1(clamp(w/scale, +-6)).
    w [N, K] (fp32 or bf16-valued fp32) -> (packed u8 [N, K/2], e8m0 u8 [N, K/32])."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    if k % MX_BLOCK:
        raise ValueError(f"K={k} must be a multiple of {MX_BLOCK}")
    blk = w.reshape(n, k // MX_BLOCK, MX_BLOCK)
    amax = np.max(np.abs(blk), axis=-1)
    amax = np.maximum(amax, np.float32(6.0 * 2.0 ** -126))
    s, biased = pow2_ceil_scale(amax, 1.0 / FP4_MAX)
    q = np.clip(blk / s[..., None], -FP4_MAX, FP4_MAX).astype(np.float32)
    codes = f32_to_e2m1_rne(q).reshape(n, k)
    return pack_codes(codes), biased.astype(np.uint8)


def quantize_mxfp4_floor(w: np.ndarray):
    """Reference packer FLOOR fallback (``kernels/fp4_source.py:35-64`` with
    ``_floor_e8m0_scale`` ``kernels/mxfp4.py:32-43``): scale exponent =
    floor(log2 amax) - 2 clamped to [-127, 128], NaN amax -> 255; data divided
    by max(2^e, 2^-126) then RNE-saturating E2M1."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    if k % MX_BLOCK:
        raise ValueError(f"K={k} must be a multiple of {MX_BLOCK}")
    blk = w.reshape(n, k // MX_BLOCK, MX_BLOCK)
    amax = np.max(np.abs(blk), axis=-1).astype(np.float32)
    e = _f32_exponent_field(amax) - 127 - 2
    e = np.clip(e, -127, 128)
    biased = (e + 127).astype(np.int32)
    biased = np.where(np.isnan(amax), 255, biased)
    s = (biased.astype(np.uint32) << 23).view(np.float32)
    s = np.maximum(s, np.float32(2.0 ** -126))
    q = (blk / s[..., None]).astype(np.float32)
    codes = f32_to_e2m1_rne(q).reshape(n, k)
    return pack_codes(codes), (biased & 0xFF).astype(np.uint8)


# ----------------------------------------------------------------- E4M3 -----
def _e4m3_table() -> np.ndarray:
    t = np.empty(256, dtype=np.float32)
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        e = (b >> 3) & 0xF
        m = b & 0x7
        if e == 0xF and m == 0x7:
            t[b] = np.nan
        elif e == 0:
            t[b] = s * m * 2.0 ** -9
        else:
            t[b] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return t


E4M3_TABLE = _e4m3_table()


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """e4m3fn byte -> fp32 (``kernels/fp4_source.py:87-91``); 0x7F/0xFF NaN."""
    return E4M3_TABLE[np.asarray(codes, dtype=np.uint8)]


def e4m3_encode(v: np.ndarray) -> np.ndarray:
    """fp32 -> e4m3fn byte, round-to-nearest-even; results beyond 448 (after
    rounding) and inf/NaN give NaN (0x7F | sign), as torch's cast does."""
    v = np.asarray(v, dtype=np.float32)
    sign = np.signbit(v).astype(np.uint8) << 7
    a = np.abs(v).astype(np.float64)
    out = np.zeros(a.shape, dtype=np.int64)
    fin = np.isfinite(a)
    af = np.where(fin, a, 0.0)
    # subnormal range: step 2^-9
    sub = af < 2.0 ** -6
    qs = np.rint(af * 2.0 ** 9)  # rint = round half to even
    # normal range
    _, ex = np.frexp(np.where(sub, 1.0, af))  # af = mant * 2^ex, mant in [0.5, 1)
    e = ex - 1  # af = (1.f) * 2^e
    mant = np.where(sub, 0.0, af / np.ldexp(1.0, e) - 1.0)
    qm = np.rint(mant * 8.0)
    carry = qm >= 8
    e = np.where(carry, e + 1, e)
    qm = np.where(carry, 0, qm)
    normal_code = ((e + 7) << 3) + qm.astype(np.int64)
    out = np.where(sub, qs.astype(np.int64), normal_code)
    over = (~sub) & ((e + 7 > 15) | ((e + 7 == 15) & (qm >= 7)))
    out = np.where(over | ~fin, 0x7F, out)
    return (out.astype(np.uint8) & 0x7F) | sign


# --------------------------------------------------------- act quant 1x128 --
def act_quant(x: np.ndarray, block: int = ACT_BLOCK, mode: str = "pow2"):
    """1 x ``block`` activation quantizer -> (e4m3 codes u8 [M, K], scale fp32 [M, K/block]).

    mode "pow2": ``act_quant_ref`` (``kernels/fp4_source.py:110-129``),
      s = 2^ceil(log2(max(amax,1e-4) * fp32(1/448))) from IEEE bits.
    mode "amax": upstream ``act_quant`` without ``scale_fmt``
      (``.mosaicvm/source/inference_kernel.py:75-80``), s = max(amax,1e-4) * fp32(1/448).
    mode "hf": ``_fp8_act_quant_kernel`` (``.mosaicvm/source/hubkernel_act_quant.py:27-35``),
      s = amax / 448 with no floor.
    mode "legacy": ``act_quant_legacy_phase27`` (``kernels/fp4_source.py:94-107``),
      s = amax / 448, replaced by 1 where it is zero (``:104``).
    In every mode y = e4m3(clamp(x / s, +-448)) (the HF kernel has no clamp;
    x/s is within 448 by construction there).
    """
    x = np.asarray(x, dtype=np.float32)
    m, k = x.shape
    if k % block:
        raise ValueError(f"K={k} must be a multiple of act block {block}")
    xb = x.reshape(m, k // block, block)
    amax = np.max(np.abs(xb), axis=-1).astype(np.float32)
    if mode == "pow2":
        s, _ = pow2_ceil_scale(np.maximum(amax, np.float32(1e-4)), 1.0 / FP8_MAX)
    elif mode == "amax":
        s = (np.maximum(amax, np.float32(1e-4)) * np.float32(1.0 / FP8_MAX)).astype(np.float32)
    elif mode == "hf":
        s = (amax / np.float32(FP8_MAX)).astype(np.float32)
    elif mode == "legacy":
        s = (amax / np.float32(FP8_MAX)).astype(np.float32)
        s = np.where(s == 0, np.float32(1.0), s).astype(np.float32)
    else:
        raise ValueError(mode)
    with np.errstate(divide="ignore", invalid="ignore"):
        y = (xb / s[..., None]).astype(np.float32)
    y = np.clip(y, -FP8_MAX, FP8_MAX)
    return e4m3_encode(y.reshape(m, k)), s.astype(np.float32)


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """``RMSNorm.forward`` (``.mosaicvm/source/inference_model.py:197-202``) with
    its reductions pinned: ss = fp64 sum of squares (bf16 inputs square exactly),
    var = fp32(ss / H), r = fp32(1 / sqrt(fp64(var) + fp64(eps))),
    y = bf16(fp32(w * fp32(x * r))).  x [M, H] bf16 values; returns bf16 values."""
    x = np.asarray(x, dtype=np.float32)
    w = np.asarray(w, dtype=np.float32)
    ss = np.sum(x.astype(np.float64) ** 2, axis=-1)
    var = (ss / np.float64(x.shape[-1])).astype(np.float32)
    r = (1.0 / np.sqrt(var.astype(np.float64) + np.float64(np.float32(eps)))).astype(np.float32)
    y = (w[None, :] * (x * r[:, None]).astype(np.float32)).astype(np.float32)
    return round_bf16(y)

