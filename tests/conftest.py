"""Shared test configuration: the ``gpu`` marker and device helpers."""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")


def write_mxfp4_checkpoint(root, layer: int, hidden: int, inter: int, n_experts: int, seed: int = 0,
                           shards: int = 2, packed_dtypes=("I8", "U8"), extra=None):
    """A small V3-style checkpoint of MXFP4 experts under ``root``: per expert
    ``layers.{layer}.ffn.experts.{e}.w{1,3,2}.{weight,scale}``, packed FP4 bytes
    [N, K/2] stored as int8 or uint8 (alternating by expert, per
    ``packed_dtypes``) and E8M0 scales [N, K/32] with exponents near 1.0, split
    over ``shards`` files with a ``model.safetensors.index.json``.  Returns
    {(e, w): (packed uint8 numpy, scale uint8 numpy)} with the bytes written.
    ``extra`` maps more tensor names to torch tensors (written to shard 0)."""
    import json
    from pathlib import Path

    import numpy as np
    import torch
    from safetensors.torch import save_file

    rng = np.random.default_rng(seed)
    root = Path(root)
    root.mkdir(parents=True, exist_ok=True)
    files = [dict() for _ in range(shards)]
    truth = {}
    dims = {"w1": (inter, hidden), "w3": (inter, hidden), "w2": (hidden, inter)}
    for e in range(n_experts):
        pdt = torch.int8 if packed_dtypes[e % len(packed_dtypes)] == "I8" else torch.uint8
        for w, (n, k) in dims.items():
            packed = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
            scale = rng.integers(118, 130, size=(n, k // 32), dtype=np.uint8)
            truth[(e, w)] = (packed, scale)
            name = f"layers.{layer}.ffn.experts.{e}.{w}."
            f = files[(e + len(w)) % shards]
            f[name + "weight"] = torch.from_numpy(packed.copy()).view(pdt)
            f[name + "scale"] = torch.from_numpy(scale.copy()).view(torch.float8_e8m0fnu)
    for k, v in (extra or {}).items():
        files[0][k] = v
    weight_map = {}
    for i, f in enumerate(files):
        fname = f"model-{i:05d}-of-{shards:05d}.safetensors"
        save_file(f, str(root / fname))
        weight_map.update({k: fname for k in f})
    (root / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))
    return truth
