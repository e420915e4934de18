"""The allocation-free MoE entry point (mosaic_moe_a16_forward_noalloc),
called through the C ABI, against mosaic_moe_a16_forward with a workspace:
bit-identical outputs, ids and weights on two calls in a row, the second with
a smaller input, and a clear rejection of a shape beyond the static scratch."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _bank(ops, dev, e, h, inter, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    def q(n, k):
        return ops.mx_quantize((torch.randn(n, k, generator=g, device=dev) * 0.02).to(torch.bfloat16))
    gu = [q(2 * inter, h) for _ in range(e + 1)]
    dn = [q(h, inter) for _ in range(e + 1)]
    gp = torch.stack([a[0] for a in gu])
    gs = torch.stack([a[1] for a in gu])
    dp = torch.stack([a[0] for a in dn])
    ds = torch.stack([a[1] for a in dn])
    return g, ops.mxt16_prepack(gp[:e], gs[:e]), ops.mxt16_prepack(dp[:e], ds[:e]), (
        ops.mxt16_prepack(gp[e], gs[e]), ops.mxt16_prepack(dp[e], ds[e]))


def _noalloc(ops, x, gu, dn, shared, logits, top_k, limit):
    from mosaic_amd import _lib
    m, h = x.shape
    e = logits.shape[1]
    ids = torch.empty(m, top_k, dtype=torch.int32, device=x.device)
    w = torch.empty(m, top_k, dtype=torch.float32, device=x.device)
    y = torch.empty(m, h, dtype=torch.bfloat16, device=x.device)
    P = ops._ptr
    _lib.call("mosaic_moe_a16_forward_noalloc", P(x), P(logits), P(ids), P(w), P(gu.packed), P(gu.scale),
              P(dn.packed), P(dn.scale), P(shared[0].packed), P(shared[0].scale), P(shared[1].packed),
              P(shared[1].scale), P(y), m, h, gu.n // 2, e, top_k, 0, 1, ctypes.c_float(1.0), None,
              ctypes.c_float(limit), ops._stream())
    return y, ids, w


@pytest.mark.parametrize("h,inter,e", [(7168, 2048, 32), (1024, 512, 16)])
def test_noalloc_matches_workspace_entry(h, inter, e):
    from mosaic_amd import ops
    dev = torch.device("cuda:0")
    g, gu, dn, shared = _bank(ops, dev, e, h, inter, seed=h + e)
    for m in (16, 3) if h == 7168 else (9, 1):  # second call smaller; m = 1 takes the fused decode kernels
        x = torch.randn(m, h, generator=g, device=dev).to(torch.bfloat16)
        logits = torch.randn(m, e, generator=g, device=dev)
        y0, ids0, w0 = ops.moe_a16_forward(x, gu, dn, logits=logits, top_k=8, shared=shared, swiglu_limit=10.0)
        y1, ids1, w1 = _noalloc(ops, x, gu, dn, shared, logits, 8, 10.0)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(ids1.cpu().numpy(), ids0.cpu().numpy())
        np.testing.assert_array_equal(w1.cpu().numpy(), w0.cpu().numpy())
        np.testing.assert_array_equal(y1.view(torch.int16).cpu().numpy(), y0.view(torch.int16).cpu().numpy())


def test_noalloc_rejects_shapes_beyond_scratch():
    from mosaic_amd import _lib, ops
    dev = torch.device("cuda:0")
    lib = _lib.lib()
    cap = lib.mosaic_moe_a16_noalloc_max_bytes()
    assert cap == 8 << 20
    m = 64  # 18 MiB of workspace at hidden 7168, inter 2048, 256 experts, top-8 + shared
    assert lib.mosaic_moe_a16_workspace_bytes(m, 7168, 2048, 256, 8, 1) > cap
    x = torch.zeros(m, 7168, dtype=torch.bfloat16, device=dev)
    # the shape check comes before any pointer is read, so placeholder banks suffice
    gu = ops.MXT16(torch.zeros(256, 1, dtype=torch.uint8, device=dev), torch.zeros(1, dtype=torch.uint8, device=dev),
                   4096, 7168)
    dn = ops.MXT16(gu.packed, gu.scale, 7168, 2048)
    logits = torch.zeros(m, 256, device=dev)
    with pytest.raises(ValueError, match="static scratch"):
        _noalloc(ops, x, gu, dn, (gu, dn), logits, 8, 0.0)
