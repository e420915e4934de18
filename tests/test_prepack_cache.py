"""Host logic of the prepacked-weight cache (CPU): entries live exactly as long
as their source tensors, fresh views of a live weight hit, in-place updates and
reused memory miss."""
from __future__ import annotations

import gc

import torch

from mosaic_amd.kernels import _prepack_cache as PC


def _counter():
    n = {"made": 0}

    def make():
        n["made"] += 1
        return object()
    return n, make


def test_entry_dropped_when_source_dies():
    PC.clear()
    n, make = _counter()
    p = torch.zeros(64, 32, dtype=torch.uint8)
    s = torch.zeros(64, 2, dtype=torch.uint8)
    PC.cached((p, s), make)
    assert PC.size() == 1
    del p
    gc.collect()
    assert PC.size() == 0, "the prepacked copy must not outlive its weight"
    del s


def test_fresh_views_hit_and_in_place_updates_miss():
    PC.clear()
    n, make = _counter()
    p = torch.zeros(64, 32, dtype=torch.int8)
    s = torch.zeros(64, 2, dtype=torch.uint8)
    a = PC.cached((p.view(torch.uint8), s.view(torch.uint8)), make)
    b = PC.cached((p.view(torch.uint8), s.view(torch.uint8)), make)
    assert a is b and n["made"] == 1
    p[0, 0] = 3                       # in-place update: version counter moves
    c = PC.cached((p.view(torch.uint8), s.view(torch.uint8)), make)
    assert c is not a and n["made"] == 2
    assert PC.size() == 1
    del p, s, a, b, c
    gc.collect()
    assert PC.size() == 0


def test_four_tensor_key_hits_across_calls():
    """grouped_expert_forward's (gate, up) tuple: keyed on the caller's four
    tensors, so repeated calls reuse one prepacked bank."""
    PC.clear()
    n, make = _counter()
    t = [torch.zeros(2, 32, 16, dtype=torch.uint8) for _ in range(4)]
    for _ in range(5):
        PC.cached(tuple(t), make)
    assert n["made"] == 1 and PC.size() == 1
    t[2] = torch.zeros(2, 32, 16, dtype=torch.uint8)   # a different up tensor
    PC.cached(tuple(t), make)
    assert n["made"] == 2
    del t
    gc.collect()
    assert PC.size() == 0


def test_many_layers_are_not_evicted():
    """More layers than any fixed cap: every weight keeps its entry while alive."""
    PC.clear()
    n, make = _counter()
    ws = [(torch.zeros(16, 8, dtype=torch.uint8), torch.zeros(16, 1, dtype=torch.uint8)) for _ in range(100)]
    for w in ws:
        PC.cached(w, make)
    for w in ws:
        PC.cached(w, make)
    assert n["made"] == 100 and PC.size() == 100
    del ws, w
    gc.collect()
    assert PC.size() == 0
