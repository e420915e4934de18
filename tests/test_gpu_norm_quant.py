"""RMSNorm with the fused 1x128 act_quant (the A8 linear's producer) against
the oracle: bf16 y, e4m3 codes and scales bit-exact, and an A8 linear fed from
the fused output equal to the unfused path."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import codecs as C

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,h", [(1, 7168), (33, 4096), (5, 128), (3, 16384)])
@pytest.mark.parametrize("mode", ["pow2", "amax", "hf"])
def test_rmsnorm_act_quant_bit_exact(dev, m, h, mode):
    from mosaic_amd import ops
    rng = np.random.default_rng(m * 7 + h)
    x = C.round_bf16((rng.standard_normal((m, h)) * rng.uniform(0.01, 30, (m, 1))).astype(np.float32))
    if mode != "hf":  # (hf divides an all-zero block by a zero scale: NaN codes whose sign is platform-defined)
        x[0, :128] = 0.0  # an all-zero block after the norm
    w = rng.uniform(-2, 2, h).astype(np.float32)
    q, s, y = ops.rmsnorm_act_quant(torch.from_numpy(x).to(dev).to(torch.bfloat16), torch.from_numpy(w).to(dev),
                                    1e-6, mode=mode, return_y=True)
    yr = C.rmsnorm(x, w, 1e-6)
    np.testing.assert_array_equal(y.float().cpu().numpy(), yr)
    qr, sr = C.act_quant(yr, 128, mode)
    np.testing.assert_array_equal(s.cpu().numpy(), sr)
    np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), qr)


def test_fused_output_feeds_the_a8_linear(dev):
    from mosaic_amd import ops
    rng = np.random.default_rng(2)
    m, h, n = 6, 1024, 512
    x = torch.from_numpy(C.round_bf16(rng.standard_normal((m, h)).astype(np.float32))).to(dev).to(torch.bfloat16)
    w = torch.from_numpy(rng.uniform(0.5, 1.5, h).astype(np.float32)).to(dev)
    wp, ws = C.quantize_mxfp4_ceil(C.round_bf16((rng.standard_normal((n, h)) * 0.05).astype(np.float32)))
    wt = ops.mxt16_prepack(torch.from_numpy(wp).to(dev), torch.from_numpy(ws).to(dev))
    q, s, y = ops.rmsnorm_act_quant(x, w, 1e-6, return_y=True)
    fused = ops.mxt16_linear_a8(None, wt, prequant=(q, s))
    unfused = ops.mxt16_linear_a8(y, wt)
    assert torch.equal(fused, unfused)
