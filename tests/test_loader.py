"""Safetensors MXFP4 expert loader on the host: shard index, cast-free reads,
the no-dtype-cast rule and the expert layout contract
(``runtime/loader.py:20-45,131-138``, ``runtime/streaming_model.py:30-101``)."""
from __future__ import annotations

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from conftest import write_mxfp4_checkpoint
from mosaic_amd import loader as LD

LAYER, H, I, E = 3, 256, 128, 3


@pytest.fixture()
def ckpt(tmp_path):
    truth = write_mxfp4_checkpoint(tmp_path, LAYER, H, I, E, seed=5,
                                   extra={"layers.3.ffn.gate.weight": torch.randn(E, H).to(torch.bfloat16)})
    return tmp_path, truth


def test_index_meta_and_raw_reads_keep_bytes(ckpt):
    root, truth = ckpt
    idx = LD.ShardIndex(root)
    assert len(idx.keys()) == E * 6 + 1
    assert idx.meta("layers.3.ffn.experts.0.w1.weight") == ("I8", (I, H // 2))
    assert idx.meta("layers.3.ffn.experts.1.w1.weight") == ("U8", (I, H // 2))
    assert idx.meta("layers.3.ffn.experts.2.w2.scale") == ("F8_E8M0", (H, I // 32))
    for e in range(E):
        r = LD.read_expert(idx, LAYER, e)
        for w in ("w1", "w3", "w2"):
            assert r[w].dtype == torch.uint8 and r[w + "_scale"].dtype == torch.uint8
            np.testing.assert_array_equal(r[w].numpy(), truth[(e, w)][0])
            np.testing.assert_array_equal(r[w + "_scale"].numpy(), truth[(e, w)][1])
    raw = idx.load_raw_tensor("layers.3.ffn.experts.0.w3.weight")
    assert raw.dtype == torch.int8  # stored dtype, no cast
    np.testing.assert_array_equal(raw.view(torch.uint8).numpy(), truth[(0, "w3")][0])


def test_no_dtype_cast_of_packed_or_e8m0(ckpt):
    root, _ = ckpt
    idx = LD.ShardIndex(root)
    with pytest.raises(ValueError, match="load_raw_tensor"):
        idx.load_tensor("layers.3.ffn.experts.0.w1.weight")
    with pytest.raises(ValueError, match="E8M0"):
        idx.load_tensor("layers.3.ffn.experts.1.w2.scale")
    g = idx.load_tensor("layers.3.ffn.gate.weight", dtype=torch.float32)
    assert g.dtype == torch.float32 and tuple(g.shape) == (E, H)


def test_contract_accepts_the_layout(ckpt):
    root, _ = ckpt
    assert LD.validate_expert_tensors(LD.ShardIndex(root), LAYER, H, I) == E
    assert LD.count_experts(LD.ShardIndex(root), LAYER + 1) == 0


def test_single_file_checkpoint(tmp_path):
    packed = np.arange(64 * 8, dtype=np.uint8).reshape(64, 8)
    scale = np.full((64, 1), 127, np.uint8)
    t = {}
    for w, (n, k) in {"w1": (64, 16), "w3": (64, 16), "w2": (16, 64)}.items():
        t[f"layers.0.ffn.experts.0.{w}.weight"] = torch.from_numpy(
            np.resize(packed, (n, k // 2)).copy())
        t[f"layers.0.ffn.experts.0.{w}.scale"] = torch.from_numpy(
            np.resize(scale, (n, k // 32)).copy()).view(torch.float8_e8m0fnu)
    save_file(t, str(tmp_path / "model.safetensors"))
    idx = LD.ShardIndex(tmp_path)
    assert LD.validate_expert_tensors(idx, 0, 16, 64) == 1


@pytest.mark.parametrize("breakage,match", [
    ("bf16_weight", "expected packed uint8"),
    ("bad_shape", "expected shape"),
    ("missing_scale", "missing layers.3.ffn.experts.1.w3.scale"),
    ("float_scale", "expected E8M0"),
])
def test_contract_reports_layout_problems(tmp_path, breakage, match):
    write_mxfp4_checkpoint(tmp_path, LAYER, H, I, 2, seed=1, shards=1)
    from safetensors.torch import load_file
    f = tmp_path / "model-00000-of-00001.safetensors"
    t = load_file(str(f))
    if breakage == "bf16_weight":
        t["layers.3.ffn.experts.0.w2.weight"] = torch.zeros(H, I // 2, dtype=torch.bfloat16)
    elif breakage == "bad_shape":
        t["layers.3.ffn.experts.1.w1.weight"] = torch.zeros(I, H // 4, dtype=torch.uint8)
    elif breakage == "missing_scale":
        del t["layers.3.ffn.experts.1.w3.scale"]
    else:
        t["layers.3.ffn.experts.0.w1.scale"] = torch.zeros(I, H // 32, dtype=torch.float32)
    save_file(t, str(f))
    import json
    (tmp_path / "model.safetensors.index.json").write_text(
        json.dumps({"metadata": {}, "weight_map": {k: f.name for k in t}}))
    with pytest.raises(LD.ExpertLayoutError, match=match):
        LD.validate_expert_tensors(LD.ShardIndex(tmp_path), LAYER, H, I)


def test_missing_checkpoint(tmp_path):
    with pytest.raises(FileNotFoundError):
        LD.ShardIndex(tmp_path)
