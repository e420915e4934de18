"""Safetensors MXFP4 experts -> MXT16 banks on the GPU: bit-exact round trip
to the file's bytes and a routed MoE layer over the loaded bank against the
oracle (``runtime/streaming_model.py:247-292`` reads the same tensors)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import write_mxfp4_checkpoint
from oracle import moe as MO

pytestmark = pytest.mark.gpu

LAYER, H, I, E = 5, 512, 256, 6


def _bank(truth, experts):
    gu = np.stack([np.concatenate([truth[(e, "w1")][0], truth[(e, "w3")][0]]) for e in experts])
    gus = np.stack([np.concatenate([truth[(e, "w1")][1], truth[(e, "w3")][1]]) for e in experts])
    d = np.stack([truth[(e, "w2")][0] for e in experts])
    ds = np.stack([truth[(e, "w2")][1] for e in experts])
    return gu, gus, d, ds


@pytest.mark.parametrize("experts", [None, [4, 0, 5]])
def test_load_bank_round_trips_file_bytes(dev, tmp_path, experts):
    from mosaic_amd import loader as LD
    truth = write_mxfp4_checkpoint(tmp_path, LAYER, H, I, E, seed=9)
    gu, dn = LD.load_expert_bank(tmp_path, LAYER, H, I, experts=experts, device=dev)
    ids = list(range(E)) if experts is None else experts
    assert gu.lead == (len(ids),) and (gu.n, gu.k) == (2 * I, H) and (dn.n, dn.k) == (H, I)
    back = LD.unload_expert_bank(gu, dn)
    for j, e in enumerate(ids):
        for w in ("w1", "w3", "w2"):
            np.testing.assert_array_equal(back[j][w].numpy(), truth[(e, w)][0])
            np.testing.assert_array_equal(back[j][w + "_scale"].numpy(), truth[(e, w)][1])


def test_moe_over_loaded_bank_matches_oracle(dev, tmp_path):
    from mosaic_amd import loader as LD
    from mosaic_amd import ops
    truth = write_mxfp4_checkpoint(tmp_path, LAYER, H, I, E, seed=10)
    gu, dn = LD.load_expert_bank(tmp_path, LAYER, H, I, device=dev)
    rng = np.random.default_rng(3)
    m, k = 5, 2
    x = torch.from_numpy(rng.standard_normal((m, H)).astype(np.float32) * 0.1).to(torch.bfloat16)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(m)]).astype(np.int32)
    w = rng.uniform(0.1, 1.0, size=(m, k)).astype(np.float32)
    y, _, _ = ops.moe_a16_forward(x.to(dev), gu, dn, ids=torch.from_numpy(ids).to(dev),
                                  weights=torch.from_numpy(w).to(dev))
    ref = MO.moe_layer_a16(x.float().numpy(), ids, w, *_bank(truth, range(E)))
    got = y.float().cpu().numpy()
    err = np.abs(got - ref) / np.maximum(1.0, np.abs(ref))
    assert err.max() <= 2e-2, f"max scaled err {err.max():.3e}"
