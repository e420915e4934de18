"""Safetensors MXFP4 expert loader into MXT16 banks.

The expert path of the reference's streaming runtime: ``ShardIndex`` and the
raw (cast-free) tensor read of ``mosaicvm/runtime/loader.py:20-45,131-138``,
the on-disk expert contract of ``validate_exact_v4_tensors``
(``mosaicvm/runtime/streaming_model.py:30-101``: packed FP4 E2M1 weights
[N, K/2] stored as I8 or U8, E8M0 scales [N, K/32], per-expert V3-style names
``layers.{i}.ffn.experts.{e}.w{1,3,2}.{weight,scale}``), and the per-expert
read of ``_make_streaming_moe_forward`` (``streaming_model.py:247-292``).

Where the reference unpacks every selected expert to bf16 on each forward, this
loader keeps the checkpoint bytes: one read per expert, a host->device copy of
the raw bytes, and a bit-exact permutation into the MXT16 tile order
(``ops.mxt16_prepack``) that the MoE kernels stream.  ``unload_expert_bank``
inverts it back to the file's bytes.

The no-dtype-cast rule (``loader.py:131-135``): a packed FP4 container must
never be cast (a bf16 cast of an I8/U8 tensor turns byte pairs into numbers).
``ShardIndex.load_tensor`` therefore refuses packed and E8M0 tensors, and the
expert path reads through ``load_raw_tensor`` only.
"""
from __future__ import annotations

import json
from pathlib import Path

import torch
from safetensors import safe_open

from . import ops

_PACKED = ("I8", "U8")
_E8M0 = ("F8_E8M0",)
_NO_CAST = _PACKED + _E8M0


class ExpertLayoutError(ValueError):
    """The checkpoint's expert tensors do not have the MXFP4 layout."""


class ShardIndex:
    """Maps parameter name -> shard file (``model.safetensors.index.json`` or a
    single ``model.safetensors``), as ``runtime/loader.py:20-45``."""

    def __init__(self, model_root: str | Path):
        self.root = Path(model_root)
        self.index_path = self.root / "model.safetensors.index.json"
        self.shards: dict[str, str] = {}
        if self.index_path.exists():
            for param, shard in json.loads(self.index_path.read_text())["weight_map"].items():
                self.shards[param] = shard
        else:
            single = self.root / "model.safetensors"
            if not single.exists():
                raise FileNotFoundError(f"no safetensors under {self.root}")
            with safe_open(single, framework="pt", device="cpu") as f:
                for k in f.keys():
                    self.shards[k] = "model.safetensors"

    def keys(self) -> list[str]:
        return list(self.shards.keys())

    def __contains__(self, param: str) -> bool:
        return param in self.shards

    def _file(self, param: str) -> Path:
        if param not in self.shards:
            raise KeyError(f"{param} is not in the checkpoint under {self.root}")
        return self.root / self.shards[param]

    def meta(self, param: str) -> tuple[str, tuple[int, ...]]:
        """(safetensors dtype string, shape) without reading the data."""
        with safe_open(self._file(param), framework="pt", device="cpu") as f:
            sl = f.get_slice(param)
            return str(sl.get_dtype()), tuple(int(s) for s in sl.get_shape())

    def load_raw_tensor(self, param: str, device: str | torch.device = "cpu") -> torch.Tensor:
        """The stored tensor with its stored dtype (no cast): packed FP4 bytes and
        E8M0 scales keep their bit patterns."""
        with safe_open(self._file(param), framework="pt", device="cpu") as f:
            t = f.get_tensor(param)
        return t.to(device=device)

    def load_tensor(self, param: str, device: str | torch.device = "cpu",
                    dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
        """A float tensor cast to ``dtype``.  Packed FP4 containers and E8M0 scales
        are refused: casting them destroys their bit patterns."""
        dt, _ = self.meta(param)
        if dt in _NO_CAST:
            raise ValueError(f"{param} is a packed/E8M0 container ({dt}); read it with load_raw_tensor, "
                             "a dtype cast would destroy its bit patterns")
        return self.load_raw_tensor(param, device).to(dtype)


def _expert_names(layer: int, e: int, w: str) -> tuple[str, str]:
    p = f"layers.{layer}.ffn.experts.{e}.{w}."
    return p + "weight", p + "scale"


def count_experts(index: ShardIndex, layer: int) -> int:
    """Routed experts of a layer: consecutive ids from 0 with a w1 weight."""
    n = 0
    while _expert_names(layer, n, "w1")[0] in index:
        n += 1
    return n


def validate_expert_tensors(index: ShardIndex, layer: int, hidden: int, inter: int,
                            experts: list[int] | None = None) -> int:
    """Check the MXFP4 expert contract (``streaming_model.py:61-85``) for the given
    experts (default: every expert of the layer): w1/w3 packed [inter, hidden/2],
    w2 packed [hidden, inter/2], stored as I8 or U8, with E8M0 scales of shape
    [N, K/32].  Returns the layer's expert count; raises ExpertLayoutError with
    every problem found."""
    n_exp = count_experts(index, layer)
    problems = []
    if n_exp == 0:
        problems.append(f"no per-expert tensors under layers.{layer}.ffn.experts.*")
    expected = {"w1": (inter, hidden), "w3": (inter, hidden), "w2": (hidden, inter)}
    for e in (range(n_exp) if experts is None else experts):
        if not 0 <= e < max(n_exp, 1):
            problems.append(f"expert {e} out of range (layer {layer} has {n_exp})")
            continue
        for w, (n, k) in expected.items():
            wname, sname = _expert_names(layer, e, w)
            if wname not in index:
                problems.append(f"missing {wname}")
                continue
            dt, shape = index.meta(wname)
            if dt not in _PACKED:
                problems.append(f"{wname}: expected packed uint8 (FP4 E2M1), got {dt}")
            if shape != (n, k // 2):
                problems.append(f"{wname}: expected shape ({n}, {k // 2}), got {shape}")
            if sname not in index:
                problems.append(f"missing {sname}")
                continue
            sdt, sshape = index.meta(sname)
            if sdt not in _E8M0:
                problems.append(f"{sname}: expected E8M0, got {sdt}")
            if sshape != (n, k // 32):
                problems.append(f"{sname}: expected shape ({n}, {k // 32}), got {sshape}")
    if problems:
        raise ExpertLayoutError(f"MXFP4 expert layout violated at layer {layer}: " + "; ".join(problems))
    return n_exp


def _bytes(t: torch.Tensor) -> torch.Tensor:
    """Reinterpret (never cast) a stored byte container as uint8."""
    if t.dtype in (torch.uint8, torch.int8, torch.float8_e8m0fnu):
        return t.view(torch.uint8)
    raise ExpertLayoutError(f"expected a byte container, got {t.dtype}")


def read_expert(index: ShardIndex, layer: int, e: int) -> dict[str, torch.Tensor]:
    """One expert's raw bytes on the host: w1/w3/w2 packed and scale, uint8 views
    of the stored tensors."""
    out = {}
    for w in ("w1", "w3", "w2"):
        wname, sname = _expert_names(layer, e, w)
        out[w] = _bytes(index.load_raw_tensor(wname))
        out[w + "_scale"] = _bytes(index.load_raw_tensor(sname))
    return out


def load_expert_bank(source: str | Path | ShardIndex, layer: int, hidden: int, inter: int,
                     experts: list[int] | None = None,
                     device: str | torch.device = "cuda") -> tuple[ops.MXT16, ops.MXT16]:
    """Read a layer's routed experts (all, or the ids in ``experts``, in that
    order) into MXT16 banks on ``device``: gate/up [E, 2*inter, hidden/2] (w1
    rows, then w3 rows) and down [E, hidden, inter/2] (w2), the layout
    ``ops.moe_a16_forward`` / ``ops.moe_a8_forward`` stream.  The bytes travel
    uncast; the tile permutation runs on the device."""
    index = source if isinstance(source, ShardIndex) else ShardIndex(source)
    n_exp = validate_expert_tensors(index, layer, hidden, inter, experts)
    ids = list(range(n_exp)) if experts is None else list(experts)
    e_n = len(ids)
    gu = torch.empty(e_n, 2 * inter, hidden // 2, dtype=torch.uint8, pin_memory=torch.cuda.is_available())
    gus = torch.empty(e_n, 2 * inter, hidden // 32, dtype=torch.uint8, pin_memory=torch.cuda.is_available())
    dn = torch.empty(e_n, hidden, inter // 2, dtype=torch.uint8, pin_memory=torch.cuda.is_available())
    dns = torch.empty(e_n, hidden, inter // 32, dtype=torch.uint8, pin_memory=torch.cuda.is_available())
    for j, e in enumerate(ids):
        r = read_expert(index, layer, e)
        gu[j, :inter] = r["w1"]
        gu[j, inter:] = r["w3"]
        gus[j, :inter] = r["w1_scale"]
        gus[j, inter:] = r["w3_scale"]
        dn[j] = r["w2"]
        dns[j] = r["w2_scale"]
    dev = torch.device(device)
    to = lambda t: t.to(dev, non_blocking=True)
    return ops.mxt16_prepack(to(gu), to(gus)), ops.mxt16_prepack(to(dn), to(dns))


def unload_expert_bank(gate_up: ops.MXT16, down: ops.MXT16) -> list[dict[str, torch.Tensor]]:
    """Inverse of ``load_expert_bank``: per expert (bank order) the w1/w3/w2
    packed bytes and E8M0 scale bytes, uint8 on the host, equal to the file's."""
    gu, gus = ops.mxt16_unpack(gate_up)
    dn, dns = ops.mxt16_unpack(down)
    inter = gate_up.n // 2
    gu, gus, dn, dns = gu.cpu(), gus.cpu(), dn.cpu(), dns.cpu()
    return [{"w1": gu[j, :inter], "w3": gu[j, inter:], "w1_scale": gus[j, :inter], "w3_scale": gus[j, inter:],
             "w2": dn[j], "w2_scale": dns[j]} for j in range(gu.shape[0])]
