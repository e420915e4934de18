"""GPU parity of the KN-layout A16 kernels: ``skinny_mxfp4_gemm``
(kernels/skinny_fp4.py:113-144) and ``fused_moe_skinny`` (:267-322).

Float bar: |got - ref| <= 2e-2 * max(1, |ref|) elementwise against the oracle
(dequant-then-matmul of identical KN bytes; the skinny MoE with its bf16
epilogue and bf16 combine)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import codecs as C
from oracle import linear as L
from oracle import moe as MO

pytestmark = pytest.mark.gpu

TOL = 2e-2


def assert_close(got, ref, tol=TOL, what=""):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref) / np.maximum(1.0, np.abs(ref))
    worst = float(err.max()) if err.size else 0.0
    assert worst <= tol, f"{what}: max scaled error {worst:.3e} > {tol}"


def _kn(rng, k, n, std=0.02):
    return C.quantize_mxfp4_ceil(C.round_bf16((rng.standard_normal((k, n)) * std).astype(np.float32)))


@pytest.mark.parametrize("m,n,k", [(1, 2048, 7168), (3, 4096, 4096), (8, 64, 128), (17, 96, 256), (5, 32, 32),
                                   (16, 7168, 2048), (40, 512, 1024)])
def test_kn_linear_vs_oracle(dev, m, n, k):
    from mosaic_amd.kernels.skinny_fp4 import skinny_mxfp4_gemm
    rng = np.random.default_rng(m * 3 + n + k)
    p, s = _kn(rng, k, n)
    x = C.round_bf16(rng.standard_normal((m, k)).astype(np.float32))
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    y = skinny_mxfp4_gemm(T(x).to(torch.bfloat16), T(p), T(s).view(torch.float8_e8m0fnu), n)
    assert_close(y.float().cpu().numpy(), L.mx_linear_kn_a16(x, p, s), what=f"kn linear {m}x{n}x{k}")


def test_kn_linear_onehot_picks_row(dev):
    """x = e_j picks row j of W exactly (scale and nibble order of the KN layout)."""
    from mosaic_amd import ops
    rng = np.random.default_rng(2)
    k, n = 256, 128
    p, s = _kn(rng, k, n, std=1.0)
    W = C.dequant_mxfp4(p, s)
    x = np.zeros((4, k), dtype=np.float32)
    for i, j in enumerate([0, 31, 32, 255]):
        x[i, j] = 1.0
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    y = ops.mx_kn_linear_a16(T(x).to(torch.bfloat16), T(p), T(s)).float().cpu().numpy()
    np.testing.assert_array_equal(y, C.round_bf16(W[[0, 31, 32, 255]]))


@pytest.mark.parametrize("m,k,none_w", [(1, 6, False), (5, 2, False), (12, 4, True)])
def test_fused_moe_skinny_vs_oracle(dev, m, k, none_w):
    from mosaic_amd.kernels.skinny_fp4 import fused_moe_skinny
    rng = np.random.default_rng(m + k)
    e, h, inter = 8, 512, 256
    gu = [_kn(rng, h, 2 * inter) for _ in range(e)]
    dn = [_kn(rng, inter, h) for _ in range(e)]
    gp, gs = np.stack([a[0] for a in gu]), np.stack([a[1] for a in gu])
    dp, ds = np.stack([a[0] for a in dn]), np.stack([a[1] for a in dn])
    x = C.round_bf16(rng.standard_normal((m, h)).astype(np.float32))
    ids = np.stack([rng.choice(e, k, replace=False) for _ in range(m)])
    w = np.ones((m, k), dtype=np.float32) if none_w else rng.uniform(0.1, 1.0, size=(m, k)).astype(np.float32)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    y = fused_moe_skinny(T(x).to(torch.bfloat16), T(ids), None if none_w else T(w), T(gp), T(gs).view(
        torch.float8_e8m0fnu), T(dp), T(ds))
    ref = MO.moe_layer_skinny(x, ids, w, gp, gs, dp, ds)
    assert_close(y.float().cpu().numpy(), ref, what=f"fused_moe_skinny m={m} k={k}")


def test_last_launch_count_counts_library_launches(dev):
    """skinny_fp4.last_launch_count (kernels/skinny_fp4.py:17-22): fused_moe_skinny
    resets it and counts its own launches (layout, gate/up, SwiGLU, down,
    combine, plus split-K sums); each skinny_mxfp4_gemm adds its GEMM (and its
    split-K sum).  Every figure equals the library's own launch counter."""
    from mosaic_amd import _lib
    from mosaic_amd.kernels import skinny_fp4 as S
    rng = np.random.default_rng(4)
    e, h, inter, m, k = 4, 256, 128, 2, 2
    gp, gs = (np.stack(a) for a in zip(*[_kn(rng, h, 2 * inter) for _ in range(e)]))
    dp, ds = (np.stack(a) for a in zip(*[_kn(rng, inter, h) for _ in range(e)]))
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    x = T(C.round_bf16(rng.standard_normal((m, h)).astype(np.float32))).to(torch.bfloat16)
    ids = T(np.array([[0, 2], [3, 1]]))
    lib = _lib.lib()
    before = lib.mosaic_launch_count()
    S.fused_moe_skinny(x, ids, None, T(gp), T(gs), T(dp), T(ds))
    n_moe = S.last_launch_count()
    assert n_moe == lib.mosaic_launch_count() - before and n_moe >= 5
    for kk, nn in ((64, 64), (7168, 2048)):
        p, s = _kn(rng, kk, nn)
        xl = T(C.round_bf16(rng.standard_normal((1, kk)).astype(np.float32))).to(torch.bfloat16)
        c0, l0 = S.last_launch_count(), lib.mosaic_launch_count()
        S.skinny_mxfp4_gemm(xl, T(p), T(s), nn)
        assert S.last_launch_count() - c0 == lib.mosaic_launch_count() - l0 in (1, 2)
    S.fused_moe_skinny(x, ids, None, T(gp), T(gs), T(dp), T(ds))
    assert S.last_launch_count() == n_moe
