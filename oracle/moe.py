"""Routed-expert MoE oracles (numpy) -- TEST INFRASTRUCTURE ONLY, see ``oracle/__init__``.

* ``route_topk`` (A10): ``Gate.forward`` (``.mosaicvm/source/inference_model.py:569-589``)
  and ``Router.forward`` (``model/layers.py:118-150``): scores = f(logits)
  (sigmoid | softmax | sqrtsoftplus; each the fp32 rounding of the exact value),
  optional selection bias, top-k, weights = unbiased scores gathered at the
  picks, renormalized (non-softmax, sum clamped at 1e-9) and scaled.  Order and
  ties (the reference leaves them to ``torch.topk``): picks are listed by
  descending selection key (score, or score + bias), equal keys go to the lower
  expert index.
* ``router_logits``: the router projection ``F.linear(x.float(), W.float())`` of
  ``Router.forward`` / ``Gate.forward``, defined as the exact dot product
  rounded once to fp32.
* ``layout_assignments`` (A11): ``kernels/moe_layout.py:8-27`` with a STABLE
  order (inside one expert, ascending flat assignment index).
* ``emit_tiles`` (A12): ``kernels/w4a16_grouped.py:151-169`` without the
  ``MAX_TILES=32`` per-expert cap (``:55-60``).
* ``moe_layer_a16`` (A13-A17, A16 contract): ``grouped_expert_forward``
  (``model/layers.py:329-373``) over MXFP4 experts plus the shared expert
  (``model/layers.py:284-297``; upstream ``MoE.forward`` adds the shared expert
  to the fp32 routed sum, ``inference_model.py:638-649``): fp32 gate/up,
  clamps (gate max-only, up both sides) when limit > 0, SiLU*up, route weight
  BEFORE the down projection, bf16 cast, fp32 down, per-token sum in
  ascending expert id, shared expert added last, one bf16 rounding.
* ``moe_layer_skinny`` (``fused_moe_skinny``, ``kernels/skinny_fp4.py:267-322``):
  KN gate|up into bf16, z = bf16(bf16(silu(gate)) * up), KN down into bf16,
  each row times bf16(weight) rounded to bf16, summed per token in bf16 in
  assignment order from zero (its bf16 ``index_add_``; the reference leaves
  the order of that sum to the device's atomics, so that order is parity
  unpinned and covered by the float tolerance).
* ``moe_layer_a8`` (A8 contract of ``fused_moe_mxint``, ``kernels/mxint.py:1435-1739``):
  A8 gate/up to a bf16 [A, 2*inter] tensor, fp32 SwiGLU, x route weight, bf16,
  act_quant_ref, A8 down to bf16 partials, fp32 ascending-expert-id sum, bf16.

Pinned by ``tests/test_oracle_moe.py``: the reference tests' KATs (counts
[1,1,0,2] of ``tests/test_moe_layout.py:13-24``; the tile-list closed form of
``tests/test_emit_tiles.py:14-34``), brute-force top-k by full sort, an
independent per-token loop (``tests/test_exact_expert_semantics.py:38-55``
style), and the weight-before-down guard (``:78-107``).
"""
from __future__ import annotations

import numpy as np

from . import codecs as C
from . import linear as L


# --------------------------------------------------------------- routing ----
def score_fn(logits: np.ndarray, func: str) -> np.ndarray:
    """Router scores of ``Gate.forward`` (``.mosaicvm/source/inference_model.py:571-577``)
    and ``_router_scores`` (``model/layers.py:110-115``), each defined as the fp32
    rounding of the exact value: evaluated in float64 and rounded once.
    sqrtsoftplus keeps torch's softplus threshold (x > 20 -> x)."""
    lg = np.asarray(logits, dtype=np.float32)
    x = lg.astype(np.float64)
    if func == "sigmoid":
        with np.errstate(over="ignore"):
            return (1.0 / (1.0 + np.exp(-x))).astype(np.float32)
    if func == "softmax":
        e = np.exp(x - x.max(axis=-1, keepdims=True))
        return (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)
    if func == "sqrtsoftplus":
        with np.errstate(over="ignore"):
            sp = np.where(lg > np.float32(20.0), x, np.log1p(np.exp(x)))
        return np.sqrt(sp).astype(np.float32)
    raise ValueError(func)


def topk_lower_index(keys: np.ndarray, k: int) -> np.ndarray:
    """Row-wise top-k of fp32 keys: descending key, equal keys -> lower index.
    NaN keys are never picked before a number."""
    keys = np.asarray(keys, dtype=np.float32)
    m, n = keys.shape
    out = np.empty((m, k), dtype=np.int64)
    idx = np.arange(n)
    for r in range(m):
        kr = np.where(np.isnan(keys[r]), -np.inf, keys[r]).astype(np.float64)
        order = np.lexsort((idx, -kr))
        out[r] = order[:k]
    return out


def route_topk(logits: np.ndarray, top_k: int = 8, score_func: str = "sigmoid",
               bias: np.ndarray | None = None, renorm: bool = True,
               route_scale: float = 1.0):
    """logits [M, E] fp32 -> (ids int64 [M, k], weights fp32 [M, k]).

    ``Gate.forward`` (``inference_model.py:569-589``) / ``Router.forward``
    (``model/layers.py:127-150``): selection key = score (+ bias, one fp32 add),
    picks listed by descending key with ties to the lower expert index; weight =
    unbiased score at the pick, divided by the fp32 sum of the k picked scores
    (in pick order) clamped below at 1e-9 (``layers.py:147``) unless softmax,
    then times ``route_scale``."""
    logits = np.asarray(logits, dtype=np.float32)
    scores = score_fn(logits, score_func)
    key = scores if bias is None else (scores + np.asarray(bias, dtype=np.float32)).astype(np.float32)
    ids = topk_lower_index(key, top_k)
    w = np.take_along_axis(scores, ids, axis=1).astype(np.float32)
    if renorm and score_func != "softmax":
        ssum = np.zeros(w.shape[0], dtype=np.float32)
        for j in range(top_k):  # fp32 sum in pick order
            ssum = (ssum + w[:, j]).astype(np.float32)
        ssum = np.where(ssum < np.float32(1e-9), np.float32(1e-9), ssum).astype(np.float32)
        w = (w / ssum[:, None]).astype(np.float32)
    w = (w * np.float32(route_scale)).astype(np.float32)
    return ids, w


def router_logits(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """logits [M, E] fp32 = x [M, H] . W [E, H]^T, the projection of
    ``Router.forward`` (``model/layers.py:128``) and ``Gate.forward``
    (``.mosaicvm/source/inference_model.py:570``), both ``F.linear(x.float(),
    W.float())``.  Each logit is defined as the exact dot product rounded once
    to fp32: the products of fp32 (or bf16) values are exact in float64 and
    ``math.fsum`` returns the correctly rounded float64 of their exact sum."""
    import math
    x64 = np.asarray(x, dtype=np.float32).astype(np.float64)
    w64 = np.asarray(w, dtype=np.float32).astype(np.float64)
    out = np.empty((x64.shape[0], w64.shape[0]), dtype=np.float32)
    for t in range(x64.shape[0]):
        prod = w64 * x64[t][None, :]
        out[t] = [math.fsum(row) for row in prod]
    return out


# ---------------------------------------------------------------- layout ----
def layout_assignments(expert_ids: np.ndarray, n_experts: int):
    """flat ids [A] -> (sorted_ids [A], perm [A], offsets [E+1], counts [E]).
    perm[p] = flat assignment index placed at sorted position p; stable."""
    ids = np.asarray(expert_ids).reshape(-1).astype(np.int64)
    perm = np.argsort(ids, kind="stable")
    counts = np.bincount(ids, minlength=n_experts).astype(np.int32)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    return ids[perm], perm.astype(np.int64), offsets, counts


def emit_tiles(counts: np.ndarray, block_m: int):
    """counts [E] -> (expert_index, m_start, tile_rows) lists, one entry per
    block_m rows of each expert in ascending expert order (uncapped)."""
    ei, ms, rows = [], [], []
    for e, c in enumerate(np.asarray(counts).tolist()):
        nt = (c + block_m - 1) // block_m
        for t in range(nt):
            ei.append(e)
            ms.append(t * block_m)
            rows.append(min(block_m, c - t * block_m))
    return (np.array(ei, dtype=np.int32), np.array(ms, dtype=np.int32),
            np.array(rows, dtype=np.int32))


# ------------------------------------------------------------ MoE (A16) -----
def _silu32(g):
    g = np.asarray(g, dtype=np.float32)
    with np.errstate(over="ignore"):  # exp(-g) = inf for g < -88.7: g / inf = -0, as in fp32 torch
        return (g / (np.float32(1.0) + np.exp(-g).astype(np.float32))).astype(np.float32)


def swiglu(gate: np.ndarray, up: np.ndarray, limit: float) -> np.ndarray:
    """fp32 SwiGLU with the optional clamps of ``model/layers.py:358-362``."""
    gate = np.asarray(gate, dtype=np.float32)
    up = np.asarray(up, dtype=np.float32)
    if limit > 0:
        gate = np.minimum(gate, np.float32(limit))
        up = np.clip(up, -np.float32(limit), np.float32(limit))
    return (_silu32(gate) * up).astype(np.float32)


def expert_a16(xrow: np.ndarray, wgu: np.ndarray, wd: np.ndarray, weight: float,
               limit: float) -> np.ndarray:
    """One token through one expert given DEQUANTIZED fp32 weights
    wgu [2*inter, H] (gate rows then up rows) and wd [H, inter] -> fp32 [H]."""
    inter = wgu.shape[0] // 2
    gu = (wgu.astype(np.float64) @ np.asarray(xrow, dtype=np.float64)).astype(np.float32)
    z = swiglu(gu[:inter], gu[inter:], limit)
    z = (z * np.float32(weight)).astype(np.float32)
    zd = C.round_bf16(z)
    return (wd.astype(np.float64) @ zd.astype(np.float64)).astype(np.float32)


def _expert_rows(ids: np.ndarray):
    """{expert id: [(token, slot), ...]} over ids [M, k], in token then slot order."""
    rows: dict[int, list] = {}
    for t in range(ids.shape[0]):
        for s in range(ids.shape[1]):
            rows.setdefault(int(ids[t, s]), []).append((t, s))
    return rows


def _combine(m: int, h: int, ids: np.ndarray, partial: dict, shared_part):
    """Per token: fp32 sum of the slot partials in ascending expert id (equal
    ids in slot order), the shared expert's partial added last."""
    out = np.zeros((m, h), dtype=np.float32)
    for t in range(m):
        acc = np.zeros(h, dtype=np.float32)
        for s in np.argsort(ids[t], kind="stable"):
            acc = (acc + partial[(t, int(s))]).astype(np.float32)
        if shared_part is not None:
            acc = (acc + shared_part[t]).astype(np.float32)
        out[t] = acc
    return out


def moe_layer_a16(x, ids, weights, bank_gu, bank_gu_s, bank_d, bank_d_s,
                  shared=None, swiglu_limit: float = 0.0, out_bf16: bool = True):
    """A16 MoE layer over MXFP4 NK banks.

    x [M, H] (bf16-valued fp32); ids [M, k]; weights [M, k] fp32;
    bank_gu [E, 2*inter, H/2] u8, bank_gu_s [E, 2*inter, H/32] u8,
    bank_d [E, H, inter/2] u8, bank_d_s [E, H, inter/32] u8 (numpy arrays or
    callables e -> array, so a test can stream experts from the device);
    shared = (gu, gu_s, d, d_s) or None.  Returns [M, H].  The tokens routed
    to one expert are multiplied together (each row is computed as
    ``expert_a16`` computes it, a float64 product rounded once to fp32).
    """
    get = (lambda b, e: b(e)) if callable(bank_gu) else (lambda b, e: b[e])
    x = np.asarray(x, dtype=np.float32)
    ids = np.asarray(ids)
    weights = np.asarray(weights, dtype=np.float32)
    m, h = x.shape

    def run(wgu, wd, rows_x, rows_w):
        inter = wgu.shape[0] // 2
        gu = (rows_x.astype(np.float64) @ wgu.astype(np.float64).T).astype(np.float32)
        z = swiglu(gu[:, :inter], gu[:, inter:], swiglu_limit)
        z = C.round_bf16((z * rows_w[:, None]).astype(np.float32))
        return (z.astype(np.float64) @ wd.astype(np.float64).T).astype(np.float32)

    partial = {}
    for e, rows in _expert_rows(ids).items():
        wgu = C.dequant_mxfp4(get(bank_gu, e), get(bank_gu_s, e))
        wd = C.dequant_mxfp4(get(bank_d, e), get(bank_d_s, e))
        ts = [t for t, _ in rows]
        ys = run(wgu, wd, x[ts], np.array([weights[t, s] for t, s in rows], dtype=np.float32))
        for i, ts_ in enumerate(rows):
            partial[ts_] = ys[i]
    shared_part = None
    if shared is not None:
        shared_part = run(C.dequant_mxfp4(shared[0], shared[1]), C.dequant_mxfp4(shared[2], shared[3]), x,
                          np.ones(m, dtype=np.float32))
    out = _combine(m, h, ids, partial, shared_part)
    return C.round_bf16(out) if out_bf16 else out


# ------------------------------------------------------------- MoE (A8) -----
def moe_layer_a8(x, ids, weights, bank_gu, bank_gu_s, bank_d, bank_d_s,
                 swiglu_limit: float = 10.0, shared=None):
    """``fused_moe_mxint`` contract (``kernels/mxint.py:1587-1722``): gate/up A8
    into bf16, SwiGLU fp32, x route weight, bf16, act_quant_ref, A8 down into
    bf16 partials, fp32 sum in ascending expert id, bf16.  ``shared`` (optional)
    is run through the same A8 expert with weight 1 and added last.  The tokens
    routed to one expert go through ``mx_linear_a8`` together (its rows are
    independent: per-row activation scales and accumulators)."""
    get = (lambda b, e: b(e)) if callable(bank_gu) else (lambda b, e: b[e])
    x = np.asarray(x, dtype=np.float32)
    ids = np.asarray(ids)
    weights = np.asarray(weights, dtype=np.float32)
    m, h = x.shape

    def run(gu, gus, d, ds, rows_x, rows_w):
        inter = gu.shape[0] // 2
        g = L.mx_linear_a8(rows_x, gu, gus, out_bf16=True)
        z = swiglu(g[:, :inter], g[:, inter:], swiglu_limit)
        z = C.round_bf16((z * rows_w[:, None]).astype(np.float32))
        return L.mx_linear_a8(z, d, ds, out_bf16=True)

    partial = {}
    for e, rows in _expert_rows(ids).items():
        ts = [t for t, _ in rows]
        ys = run(get(bank_gu, e), get(bank_gu_s, e), get(bank_d, e), get(bank_d_s, e), x[ts],
                 np.array([weights[t, s] for t, s in rows], dtype=np.float32))
        for i, ts_ in enumerate(rows):
            partial[ts_] = ys[i]
    shared_part = None
    if shared is not None:
        shared_part = run(shared[0], shared[1], shared[2], shared[3], x, np.ones(m, dtype=np.float32))
    return C.round_bf16(_combine(m, h, ids, partial, shared_part))


# --------------------------------------------------------- MoE (skinny) -----
def _bf(a):
    return C.round_bf16(np.asarray(a, dtype=np.float32))


def moe_layer_skinny(x, ids, weights, gu_p, gu_s, d_p, d_s):
    """``fused_moe_skinny`` over KN banks: gu_p [E, H, I] + gu_s [E, H, 2I/32]
    (gate columns then up columns), d_p [E, I, H/2] + d_s [E, I, H/32]
    (numpy arrays or callables e -> array).  Returns bf16-valued [M, H]."""
    get = (lambda b, e: b(e)) if callable(gu_p) else (lambda b, e: b[e])
    x = np.asarray(x, dtype=np.float32)
    ids = np.asarray(ids).reshape(x.shape[0], -1)
    weights = np.asarray(weights, dtype=np.float32).reshape(ids.shape)
    m, h = x.shape
    contrib = {}
    for e, rows in _expert_rows(ids).items():
        ts = [t for t, _ in rows]
        gu = L.mx_linear_kn_a16(x[ts], get(gu_p, e), get(gu_s, e))           # bf16 [r, 2I]
        inter = gu.shape[1] // 2
        gate, up = gu[:, :inter], gu[:, inter:]
        sg = _bf(gate / (np.float32(1.0) + np.exp(-gate).astype(np.float32)))
        z = _bf(sg * up)
        yg = L.mx_linear_kn_a16(z, get(d_p, e), get(d_s, e))                 # bf16 [r, H]
        for i, (t, s) in enumerate(rows):
            contrib[(t, s)] = _bf(yg[i] * _bf(weights[t, s]))
    out = np.zeros((m, h), dtype=np.float32)
    for t in range(m):
        acc = np.zeros(h, dtype=np.float32)
        for s in range(ids.shape[1]):
            acc = _bf(acc + contrib[(t, s)])
        out[t] = acc
    return out
