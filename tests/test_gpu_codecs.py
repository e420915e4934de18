"""GPU parity of the element-format kernels against the CPU oracle (bit-exact).

Reference KATs restated: exhaustive code x e8m0 decode
(``tests/test_mxfp4_decode.py:20-63``), e4m3 all-256 decode (``:36-43``),
e4m3 encoder vs torch's cast on the clamped domain
(``tests/test_mxint_epilogue.py:24-58``), act-quant scale boundaries
(``tests/test_fp4_source.py:45-63``).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import codecs as C

pytestmark = pytest.mark.gpu


def _ops():
    from mosaic_amd import ops
    return ops


def test_dequant_exhaustive_code_by_scale(dev):
    ops = _ops()
    codes = np.repeat(np.arange(16, dtype=np.uint8), 256)
    e8 = np.tile(np.arange(256, dtype=np.uint8), 16)
    packed = np.repeat((codes | (codes << 4))[:, None], 16, axis=1)  # [4096, 16] -> K = 32
    scale = e8[:, None]
    want = C.dequant_mxfp4(packed, scale)
    got32 = ops.mx_dequant(torch.from_numpy(packed).to(dev), torch.from_numpy(scale).to(dev),
                           dtype=torch.float32).cpu().numpy()
    gotbf = ops.mx_dequant(torch.from_numpy(packed).to(dev), torch.from_numpy(scale).to(dev),
                           dtype=torch.bfloat16).float().cpu().numpy()
    inner = (e8 >= 1) & (e8 <= 254)
    # every finite value for scale bytes 1..254 is exact in f32 and bf16
    np.testing.assert_array_equal(got32[inner], want[inner])
    np.testing.assert_array_equal(gotbf[inner], want[inner])
    # the LUT at scale 127 (reference KAT tests/test_mxfp4.py:54-63)
    row = (np.arange(4096) // 256 == 3) & (e8 == 127)
    assert np.all(got32[row] == C.E2M1_LUT[3])


def test_dequant_edge_scale_bytes(dev):
    """e8m0 0x00 / 0xFF: the reference decodes 0.0 / +inf; the hardware
    converts must agree wherever the oracle is finite."""
    ops = _ops()
    codes = np.arange(16, dtype=np.uint8)
    for b in (0, 255):
        packed = np.repeat((codes | (codes << 4))[:, None], 16, axis=1)
        scale = np.full((16, 1), b, dtype=np.uint8)
        want = C.dequant_mxfp4(packed, scale)
        got = ops.mx_dequant(torch.from_numpy(packed).to(dev), torch.from_numpy(scale).to(dev),
                             dtype=torch.float32).cpu().numpy()
        fin = np.isfinite(want)
        np.testing.assert_allclose(got[fin], want[fin], atol=1e-30, rtol=0)


@pytest.mark.parametrize("recipe", ["ceil", "floor"])
def test_mx_quantize_bitexact(dev, recipe):
    ops = _ops()
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((96, 1024)) * 0.02).astype(np.float32)
    w[0] = 0.0                                   # all-zero block -> clamp path
    w[1, :32] = 6.0 * 2.0 ** -126                # tiny
    w[2, :32] = np.float32(3e37)                 # huge
    ties = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0], dtype=np.float32)
    w[3, :32] = np.tile(np.concatenate([ties, -ties]), 2)
    w[4, :32] = np.tile(np.concatenate([ties, -ties]), 2) * 0.75  # mantissa > 1.5 amax
    wb = torch.from_numpy(w).to(torch.bfloat16)
    wf = wb.float().numpy()
    p_ref, s_ref = (C.quantize_mxfp4_ceil if recipe == "ceil" else C.quantize_mxfp4_floor)(wf)
    for src in (wb, torch.from_numpy(wf)):
        p, s = ops.mx_quantize(src.to(dev), recipe)
        np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
        np.testing.assert_array_equal(p.cpu().numpy(), p_ref)


@pytest.mark.parametrize("mode", ["pow2", "amax", "hf", "legacy"])
def test_act_quant_bitexact(dev, mode):
    ops = _ops()
    rng = np.random.default_rng(5)
    x = rng.standard_normal((8, 4096)).astype(np.float32)
    vals = [1e-5, -1e-5, 1e-4, 448.0, -448.0, 1.0, 2.0 ** -60]
    vals += [2.0 ** e * 448.0 for e in (-10, -1, 0, 4)]
    vals += [2.0 ** e * 448.0 * 1.0000001 for e in (-10, -1, 0, 4)]
    xb = np.zeros((1, 128 * 16), dtype=np.float32)
    for i, v in enumerate(vals):
        xb[0, 128 * i + 7] = v
    for arr in (x, xb):
        xt = torch.from_numpy(arr).to(torch.bfloat16)
        xf = xt.float().numpy()
        q_ref, s_ref = C.act_quant(xf, 128, mode)
        if mode == "hf":
            live = np.repeat(s_ref > 0, 128, axis=1)  # all-zero blocks divide 0/0
        else:
            live = np.ones(xf.shape, dtype=bool)
        q, s = ops.act_quant(xt.to(dev), 128, mode)
        np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
        np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy()[live], q_ref[live])


def test_e4m3_decode_all_bytes(dev):
    ops = _ops()
    b = np.arange(256, dtype=np.uint8)
    got = ops.e4m3_decode(torch.from_numpy(b).to(dev)).cpu().numpy()
    want = C.e4m3_decode(b)
    nan = np.isnan(want)
    np.testing.assert_array_equal(got[~nan], want[~nan])
    assert np.isnan(got[nan]).all()


def test_hardware_converters_equal_software_roundings(dev):
    """The fused prefill epilogues round to bf16 and encode e4m3 with gfx950's
    converters; over every fp32 bit pattern they equal the software roundings
    (f32_bf16 on every non-NaN input; e4m3_rne, pinned to torch's cast by the
    test below, on every input after the epilogue's clamp to [-448, 448])."""
    assert _ops().selfcheck_converters(dev) == [0, 0]


def test_e4m3_encode_dense(dev):
    ops = _ops()
    fin = C.E4M3_TABLE[np.isfinite(C.E4M3_TABLE)]
    pos = np.sort(fin[fin >= 0])
    mids = (pos[:-1] + pos[1:]) / 2
    vals = [fin, mids, np.nextafter(mids, np.float32(1e30)), np.nextafter(mids, np.float32(-1e30))]
    rng = np.random.default_rng(3)
    vals += [rng.uniform(-448, 448, 1 << 18), rng.standard_normal(1 << 16) * 1e-2,
             np.array([464.0, 465.0, 470.0, -464.0, 0.0, -0.0], dtype=np.float32)]
    x = np.concatenate([np.asarray(v, dtype=np.float32).ravel() for v in vals] + [-np.concatenate(
        [np.asarray(v, dtype=np.float32).ravel() for v in vals[:4]])])
    got = ops.e4m3_encode(torch.from_numpy(x).to(dev)).cpu().numpy()
    np.testing.assert_array_equal(got, C.e4m3_encode(x))
