"""Pins the codec oracle (CPU): reference KATs, torch's own casts, brute force."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import codecs as C


def test_e2m1_lut_matches_locked_table():
    """tests/test_mxfp4.py:47-51."""
    assert C.E2M1_LUT.tolist() == [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                                   -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]
    assert np.signbit(C.E2M1_LUT[8])


def test_nibble_order_and_scale127_kat():
    """tests/test_mxfp4.py:54-63: codes 0..15 twice, low nibble = even index, scale byte 127 = 1x."""
    codes = np.tile(np.arange(16, dtype=np.uint8), 2)[:32]
    packed = (codes[0::2] | (codes[1::2] << 4)).reshape(1, 16)
    np.testing.assert_array_equal(C.unpack_codes(packed)[0], codes)
    dq = C.dequant_mxfp4(packed, np.array([[127]], dtype=np.uint8))[0]
    np.testing.assert_array_equal(dq, C.E2M1_LUT[codes])
    np.testing.assert_array_equal(C.pack_codes(C.unpack_codes(packed)), packed)


def test_exhaustive_code_by_e8m0():
    """All 16 x 256 (code, scale byte) pairs (tests/test_mxfp4_decode.py:20-63) against
    the closed form LUT[c] * 2^(b-127); byte 0 -> 0.0 and 255 -> +inf (reference
    exponent-field insertion, kernels/fp4_source.py:67-75)."""
    codes = np.repeat(np.arange(16, dtype=np.uint8), 256)
    e8 = np.tile(np.arange(256, dtype=np.uint8), 16)
    packed = np.repeat((codes | (codes << 4))[:, None], 16, axis=1)
    with np.errstate(invalid="ignore"):
        got = C.dequant_mxfp4(packed, e8[:, None])
    for i in range(4096):
        c, b = int(codes[i]), int(e8[i])
        s = 0.0 if b == 0 else (math.inf if b == 255 else math.ldexp(1.0, b - 127))
        v = float(C.E2M1_LUT[c])
        want = v * s if not (v == 0 and math.isinf(s)) else math.nan
        row = got[i]
        if math.isnan(want):
            assert np.isnan(row).all()
        else:
            with np.errstate(over="ignore"):
                assert (row == np.float32(want)).all(), (c, b, row[0], want)


def test_e8m0_matches_torch_on_normal_bytes():
    b = np.arange(256, dtype=np.uint8)
    t = torch.from_numpy(b).view(torch.float8_e8m0fnu).float().numpy()
    got = C.e8m0_to_f32(b)
    np.testing.assert_array_equal(got[1:255], t[1:255])
    assert got[0] == 0.0 and np.isposinf(got[255])        # documented divergence from torch
    assert t[0] == 2.0 ** -127 and np.isnan(t[255])


def test_e4m3_decode_all_bytes_vs_torch():
    b = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(b).view(torch.float8_e4m3fn).float().numpy()
    got = C.e4m3_decode(b)
    nan = np.isnan(want)
    assert (np.isnan(got) == nan).all()
    np.testing.assert_array_equal(got[~nan], want[~nan])


def test_e4m3_encoder_vs_torch_cast():
    """Every representable value, its +-1 ulp neighbours, midpoints +-1 ulp, a dense
    sweep and overflow (tests/test_mxint_epilogue.py:24-58 restated against the
    oracle encoder)."""
    fin = C.E4M3_TABLE[np.isfinite(C.E4M3_TABLE)]
    vals = [fin, np.nextafter(fin, np.float32(1e30)), np.nextafter(fin, np.float32(-1e30))]
    pos = np.sort(fin[fin >= 0])
    mids = ((pos[:-1].astype(np.float64) + pos[1:]) / 2).astype(np.float32)
    vals += [mids, np.nextafter(mids, np.float32(1e30)), np.nextafter(mids, np.float32(-1e30))]
    rng = np.random.default_rng(0)
    vals += [rng.uniform(-500, 500, 1 << 18).astype(np.float32), (rng.standard_normal(1 << 16) * 1e-2),
             np.array([464, 465, 480, 1e6, np.inf, -np.inf, 0.0, -0.0], dtype=np.float32)]
    x = np.concatenate([np.asarray(v, dtype=np.float32).ravel() for v in vals])
    x = np.concatenate([x, -x])
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(C.e4m3_encode(x), want)


def _brute_e2m1(v: float) -> int:
    """Nearest E2M1 magnitude by exhaustive distance; ties -> even code; >= 6 saturates."""
    a = abs(v)
    grid = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    if a >= 6.0:
        code = 7
    else:
        d = [abs(a - g) for g in grid]
        best = min(d)
        cands = [i for i, x in enumerate(d) if x == best]
        code = cands[0] if len(cands) == 1 else [c for c in cands if c % 2 == 0][0]
    return code | (8 if math.copysign(1.0, v) < 0 else 0)


def test_e2m1_rne_brute_force():
    rng = np.random.default_rng(1)
    grid = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])
    mids = (grid[:-1] + grid[1:]) / 2
    vals = np.concatenate([rng.uniform(-7, 7, 4000), grid, mids, -mids, np.nextafter(mids, 0), [-0.0, 7.5, -100]])
    vals = vals.astype(np.float32)
    got = C.f32_to_e2m1_rne(vals)
    want = np.array([_brute_e2m1(float(v)) for v in vals], dtype=np.uint8)
    np.testing.assert_array_equal(got, want)


def test_quantize_ceil_scale_closed_form():
    """scale = 2^ceil(log2(amax/6)) (fast_round_scale, .mosaicvm/source/inference_kernel.py:23-37)."""
    rows = []
    for j in (-10, -3, 0, 2):
        for amax in (6 * 2.0 ** j, 6 * 2.0 ** j * 1.0001, 6 * 2.0 ** j * 0.9999, 5.0 * 2.0 ** j):
            r = np.zeros(32, dtype=np.float32)
            r[5] = amax
            r[7] = -amax / 3
            rows.append(r)
    w = np.stack(rows)
    _, s = C.quantize_mxfp4_ceil(w)
    for r, b in zip(w, s[:, 0]):
        amax = float(np.max(np.abs(r)))
        t = np.float32(np.float32(amax) * np.float32(1.0 / 6.0))
        want = math.ceil(math.log2(t))
        assert int(b) - 127 == want, (amax, int(b) - 127, want)


def test_quantize_floor_kat():
    """FLOOR recipe (kernels/mxfp4.py:32-43): exponent floor(log2 amax) - 2."""
    w = np.zeros((3, 32), dtype=np.float32)
    w[0, 0] = 1.0        # floor(log2 1) - 2 = -2 -> 125; 1/0.25 = 4 -> code 6
    w[1, 0] = 7.9        # floor(log2 7.9) = 2 -> 0 -> 127; 7.9 saturates to code 7 (6.0)
    w[2, 3] = -0.3       # floor(log2 0.3) = -2 -> -4 -> 123; -0.3*16 = -4.8 -> code 6|8
    p, s = C.quantize_mxfp4_floor(w)
    assert s[:, 0].tolist() == [125, 127, 123]
    codes = C.unpack_codes(p)
    assert codes[0, 0] == 6 and codes[1, 0] == 7 and codes[2, 3] == 14


@pytest.mark.parametrize("recipe", ["ceil", "floor"])
def test_quantize_roundtrip_idempotent(recipe):
    """FLOOR: quantize(dequant(quantize(w))) == quantize(w) byte for byte
    (tests/test_mxfp4.py:36-44).  CEIL: a block whose amax lands on the code 3*s
    re-quantizes with scale s/2 and code 6, so only the VALUES are idempotent."""
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((64, 256)) * 0.02).astype(np.float32)
    q = C.quantize_mxfp4_ceil if recipe == "ceil" else C.quantize_mxfp4_floor
    p0, s0 = q(w)
    d0 = C.dequant_mxfp4(p0, s0)
    p1, s1 = q(d0)
    np.testing.assert_array_equal(C.dequant_mxfp4(p1, s1), d0)
    if recipe == "floor":
        np.testing.assert_array_equal(p0, p1)
        np.testing.assert_array_equal(s0, s1)


def test_act_quant_pow2_boundaries():
    """tests/test_fp4_source.py:45-63: the pow2 scale is an exact power of two, round-trips
    through e8m0, and differs from the legacy amax/448 scale on straddling blocks."""
    vals = [0.0, 1e-5, -1e-5, 1e-4, 448.0, -448.0, 1.0, 2.0 ** -60]
    vals += [2.0 ** e * 448.0 for e in (-10, -1, 0, 4)]
    vals += [2.0 ** e * 448.0 * 1.0000001 for e in (-10, -1, 0, 4)]
    x = np.zeros((1, 128 * len(vals)), dtype=np.float32)
    for i, v in enumerate(vals):
        x[0, 128 * i + 7] = v
    xb = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    _, s = C.act_quant(xb, 128, "pow2")
    bits = s.view(np.uint32)
    assert (bits & 0x7FFFFF == 0).all()
    np.testing.assert_array_equal(torch.from_numpy(s).to(torch.float8_e8m0fnu).float().numpy(), s)
    _, sl = C.act_quant(xb, 128, "hf")
    assert not np.array_equal(sl, s)
    # closed form: s = 2^ceil(log2(max(amax, 1e-4) / 448))
    for i in range(len(vals)):
        amax = max(abs(float(xb[0, 128 * i + 7])), 1e-4)
        t = float(np.float32(np.float32(amax) * np.float32(1.0 / 448.0)))
        assert s[0, i] == 2.0 ** math.ceil(math.log2(t))


def test_act_quant_legacy_pins():
    """act_quant_legacy_phase27 (kernels/fp4_source.py:94-107): differs from the pow2 scale on
    the straddling blocks of tests/test_fp4_source.py:45-63; an all-zero block gets s = 1 and
    zero codes; amax = 448 gives s = 1 and codes equal to the e4m3 encoding of x; scaling x by
    2^j scales s by 2^j and keeps the codes; s = fl(amax / 448) lies within half an ulp."""
    vals = [0.0, 1e-5, -1e-5, 1e-4, 448.0, -448.0, 1.0, 2.0 ** -60]
    vals += [2.0 ** e * 448.0 for e in (-10, -1, 0, 4)]
    vals += [2.0 ** e * 448.0 * 1.0000001 for e in (-10, -1, 0, 4)]
    x = np.zeros((1, 128 * len(vals)), dtype=np.float32)
    for i, v in enumerate(vals):
        x[0, 128 * i + 7] = v
    xb = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    _, sp = C.act_quant(xb, 128, "pow2")
    ql, sl = C.act_quant(xb, 128, "legacy")
    assert not np.array_equal(sl, sp)
    assert sl[0, 0] == 1.0 and (ql[0, :128] == 0).all()
    rng = np.random.default_rng(11)
    y = C.round_bf16(rng.uniform(-448, 448, (3, 256)).astype(np.float32))
    y[:, 0] = 448.0
    y[:, 128] = -448.0
    qy, sy = C.act_quant(y, 128, "legacy")
    assert (sy == 1.0).all()
    np.testing.assert_array_equal(qy, C.e4m3_encode(y))
    z = C.round_bf16(rng.standard_normal((4, 512)).astype(np.float32))
    qz, sz = C.act_quant(z, 128, "legacy")
    for j in (-20, -3, 5):
        q2, s2 = C.act_quant(z * np.float32(2.0 ** j), 128, "legacy")
        np.testing.assert_array_equal(q2, qz)
        np.testing.assert_array_equal(s2, sz * np.float32(2.0 ** j))
    amax = np.abs(z.reshape(4, 4, 128)).max(-1).astype(np.float64)
    assert (np.abs(sz.astype(np.float64) - amax / 448.0) <= np.spacing(sz) / 2).all()


def test_act_quant_matches_torch_cast_path():
    """y = e4m3(clamp(x / s)) with torch's cast (kernels/fp4_source.py:126-128)."""
    rng = np.random.default_rng(3)
    x = torch.from_numpy(rng.standard_normal((8, 512)).astype(np.float32)).to(torch.bfloat16).float()
    q, s = C.act_quant(x.numpy(), 128, "pow2")
    xs = (x.view(8, 4, 128) / torch.from_numpy(s)[..., None]).clamp(-448, 448).reshape(8, 512)
    want = xs.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(q, want)


def test_rmsnorm_pins():
    """Against torch's RMSNorm.forward (fp32 mean, rsqrt) within one bf16 ulp,
    exactly invariant to power-of-two scaling of x, and the constant-row closed
    form y = sign(a) * w."""
    import torch
    rng = np.random.default_rng(17)
    x = C.round_bf16(rng.standard_normal((9, 1024)).astype(np.float32) * 3)
    w = rng.uniform(0.5, 1.5, 1024).astype(np.float32)
    y = C.rmsnorm(x, w, 1e-6)
    xt = torch.from_numpy(x)
    ref = (torch.from_numpy(w) * (xt * torch.rsqrt(xt.square().mean(-1, keepdim=True) + 1e-6))).to(torch.bfloat16)
    diff = np.abs(y - ref.float().numpy())
    assert (diff <= np.abs(ref.float().numpy()) * 2.0 ** -7).all()
    np.testing.assert_array_equal(C.rmsnorm(x * 4.0, w, 0.0), C.rmsnorm(x, w, 0.0))
    a = np.full((2, 256), -0.375, np.float32)
    np.testing.assert_array_equal(C.rmsnorm(a, w[:256], 0.0), C.round_bf16(-w[:256])[None].repeat(2, 0))
