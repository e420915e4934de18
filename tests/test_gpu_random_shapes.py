"""Seeded random shapes through every dispatch of the linears, against the CPU oracle:
the A8 MXFP4 linear (16-row kernel, staged 64- and 256-row plans, split K, N tails),
the A16 MXFP4 linear (NK and KN layouts) and the FP8 block GEMM (skinny, decode ring,
tiled, split K, big tiles).  Float bar |got - ref| <= 2e-2 * max(1, |ref|).  Sizes keep
each oracle call under ~1e8 multiply-adds."""
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
