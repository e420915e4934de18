"""DSA drop-ins: the lightning indexer with top-k and sparse (MLA) attention.

* ``sparse_attn(q, kv, attn_sink, topk_idxs, softmax_scale)`` -- upstream
  signature (``.mosaicvm/source/inference_kernel.py:355-368``): q [b, m, h, d]
  bf16, kv [b, n, d] bf16, topk_idxs [b, m, topk] int32 -> o [b, m, h, d].
  V = K (d = 512, the V4 geometry); heads are padded to the kernel's head
  groups and stripped, as upstream pads to 16.
* ``sparse_attn_fused(q, kv, sink, topk_idxs, scale)`` and ``sparse_attn_ref``
  -- ``mosaicvm/kernels/dsa_sparse.py:92-110`` / ``mosaicvm/model/dsa.py:214-242``:
  q [s, h, d], kv [n, d], topk_idxs [s, t] -> o [s, h, d] (bf16 only; d = 512).
* ``indexer_topk`` / ``indexer_scores`` -- the FP8 indexer of ``Indexer.forward``
  (``.mosaicvm/source/inference_model.py:408-439``) from quantized q/k.
* ``mla_decode_fp8`` -- MLA decode over an FP8 latent cache (BASELINE format).
* ``dsa_decode_attention(q, k_index, v_full, topk, scale)`` --
  ``mosaicvm/kernels/dsa_attention.py:113-154``: per-head top-k positions and
  softmax attention over them for one token (q [H, d], k_index [ctx, H, d],
  v_full [ctx, H, dv] bf16) -> (out [H, dv], idx [H, topk]); picks listed by
  descending score, ties to the lower position.
* ``Indexer`` -- the scoring and top-k of ``Indexer.forward``
  (``.mosaicvm/source/inference_model.py:408-439``, ``mosaicvm/model/dsa_layers.py:281-321``)
  from already projected FP8 q and the FP8 compressed key cache: the causal
  prefill mask at ``start_pos == 0``, ``min(index_topk, end_pos // ratio)``
  picks, ``-1`` for masked picks, ``+ offset`` otherwise.
* ``DecodeKVCache`` -- the decode-step state of one DSA attention layer
  (``kv_cache`` of ``ExactAttention``, ``mosaicvm/model/dsa_layers.py:393-400``,
  and the ``s == 1`` branch of ``_core_body``, ``:469-481,517-521``): a ring of
  ``window`` kv rows followed by the compressed rows; ``step`` writes the new
  kv row (act_quant_sim of the non-rope dims) into its ring slot, builds the
  window + compressed gather indices and attends with the sink.
"""
from __future__ import annotations

import torch

from .. import ops

_HEAD_STEPS = (16, 32, 48, 64)


def _padded_heads(h: int) -> int:
    for v in _HEAD_STEPS:
        if h <= v:
            return v
    return -(-h // 64) * 64


def _attend(q3: torch.Tensor, kv3: torch.Tensor, sink, idx2: torch.Tensor, scale: float) -> torch.Tensor:
    rows, h, d = q3.shape
    if d != 512:
        raise ValueError(f"sparse attention drop-in supports head dim 512 (V = K), got {d}; "
                         "use ops.mla_sparse_decode_bf16 for the 576 = 512 + 64 MLA layout")
    hp = _padded_heads(h)
    if hp != h:
        q3 = torch.cat([q3, q3.new_zeros(rows, hp - h, d)], dim=1)
        if sink is not None:
            sink = torch.cat([sink.float(), sink.new_zeros(hp - h, dtype=torch.float32)])
    o = ops.mla_sparse_decode_bf16(q3, kv3, idx2, scale, None if sink is None else sink.float().contiguous())
    return o[:, :h] if hp != h else o


def sparse_attn(q: torch.Tensor, kv: torch.Tensor, attn_sink: torch.Tensor, topk_idxs: torch.Tensor,
                softmax_scale: float) -> torch.Tensor:
    b, s, h, d = q.size()
    o = _attend(q.reshape(b * s, h, d).contiguous(), kv.contiguous(), attn_sink,
                topk_idxs.reshape(b * s, -1), softmax_scale)
    return o.reshape(b, s, h, d)


def sparse_attn_fused(q: torch.Tensor, kv: torch.Tensor, sink: torch.Tensor, topk_idxs: torch.Tensor,
                      scale: float) -> torch.Tensor:
    if q.dtype != torch.bfloat16 or kv.dtype != torch.bfloat16:
        raise ValueError("sparse_attn_fused: bf16 q and kv required")
    s, h, d = q.shape
    return _attend(q.contiguous(), kv.contiguous().unsqueeze(0), sink, topk_idxs, scale)


sparse_attn_ref = sparse_attn_fused


def indexer_topk(q_fp8, q_scale, k_fp8, k_scale, weights, topk: int, lengths=None, offset: int = 0):
    """q [B, H, 128] e4m3 + [B, H] f32, k [B, L, 128] e4m3 + [B, L] f32,
    weights [B, H] f32 -> topk_idxs [B, topk] int32."""
    return ops.dsa_indexer_topk(q_fp8, q_scale, k_fp8, k_scale, weights, topk, lengths, offset)


def indexer_scores(q_fp8, q_scale, k_fp8, k_scale, weights):
    return ops.dsa_indexer_scores(q_fp8, q_scale, k_fp8, k_scale, weights)


def mla_decode_fp8(q, kv_latent, kv_scale, kv_rope, topk_idxs, softmax_scale, attn_sink=None):
    return ops.mla_sparse_decode(q, kv_latent, kv_scale, kv_rope, topk_idxs, softmax_scale, attn_sink)


class Indexer(torch.nn.Module):
    """Scoring + top-k stage of ``Indexer.forward`` on FP8 operands.

    ``forward(q_fp8, q_scale, weights, k_cache, k_scale, start_pos, offset)``:
    q_fp8 [bsz, seqlen, H, 128] e4m3 with q_scale [bsz, seqlen, H] f32 (the
    rotated, projected queries), weights [bsz, seqlen, H] f32 (weights_proj(x)
    * softmax_scale * H^-0.5), k_cache [bsz, >= end_pos // ratio, 128] e4m3 with
    k_scale [bsz, ...] f32 -> topk_idxs [bsz, seqlen, min(index_topk, end_pos //
    ratio)] int32.  Score = sum over heads of w_h ReLU(q_h . k_t * q_s * k_s) in
    the canonical order; ties go to the lower index (the reference leaves them
    to torch.topk)."""

    def __init__(self, index_topk: int = 2048, compress_ratio: int = 4):
        super().__init__()
        self.index_topk = index_topk
        self.compress_ratio = compress_ratio

    def forward(self, q_fp8, q_scale, weights, k_cache, k_scale, start_pos: int, offset: int):
        bsz, seqlen, h, d = q_fp8.shape
        ratio = self.compress_ratio
        end_pos = start_pos + seqlen
        n_c = end_pos // ratio
        k = min(self.index_topk, n_c)
        if k == 0:
            return torch.empty(bsz, seqlen, 0, dtype=torch.int32, device=q_fp8.device)
        kc, ks = k_cache[:, :n_c], k_scale[:, :n_c]
        q2 = q_fp8.reshape(bsz * seqlen, h, d)
        qs2, w2 = q_scale.reshape(bsz * seqlen, h).float(), weights.reshape(bsz * seqlen, h).float()
        if start_pos == 0:  # causal: position i scores the first (i + 1) // ratio compressed entries
            bounds = (torch.arange(1, seqlen + 1, device=q_fp8.device) // ratio).to(torch.int32)
            lengths = bounds.repeat(bsz)
        else:
            lengths = torch.full((bsz * seqlen,), n_c, dtype=torch.int32, device=q_fp8.device)
        idx = ops.dsa_indexer_topk_shared(q2, qs2, kc.contiguous(), ks.float().contiguous(), w2, k, lengths, offset)
        return idx.reshape(bsz, seqlen, k)


HEAD_GROUP = 8
CANDIDATES = 512


def dsa_decode_attention(q, k_index, v_full, topk: int = CANDIDATES, scale: float | None = None):
    """``mosaicvm/kernels/dsa_attention.py:113-154`` on the HIP per-head kernels."""
    if q.dim() != 2:
        raise ValueError("batch=1 decode path: q must be [H, index_dim]")
    h, index_dim = q.shape
    ctx = k_index.shape[0]
    if h % HEAD_GROUP:
        raise ValueError(f"heads {h} must be a multiple of {HEAD_GROUP}")
    if ctx < topk:
        raise ValueError("context must cover candidate set")
    if scale is None:
        scale = 1.0 / (index_dim ** 0.5)
    return ops.dsa_head_attention(q.contiguous(), k_index.contiguous(), v_full.contiguous(), topk, scale)


class DecodeKVCache:
    """One sequence's DSA decode cache: rows 0 .. window-1 are the kv ring (slot
    = position % window), rows window .. window + n_compressed - 1 the
    compressed entries (the compressor writes them; ``write_compressed``).

    ``fp8=False``: a bf16 [window + n_compressed, head_dim] cache, the
    reference's own (V4 geometry: head_dim 512 with the rope in the last 64,
    V = the whole row).  ``fp8=True``: e4m3 codes + fp32 scales per 64 + bf16
    rope for the 512 + 64 MLA layout (head_dim 576, V = the 512 latent dims),
    the cache ``ops.mla_sparse_decode`` reads; the attended values are the same
    bf16 numbers either way."""

    def __init__(self, head_dim: int = 512, window: int = 128, n_compressed: int = 0, rope: int = 64,
                 fp8: bool = False, device="cuda"):
        if fp8 and (head_dim - rope != 512 or rope != 64):
            raise ValueError("the FP8 cache holds the 512 + 64 MLA layout")
        self.head_dim, self.window, self.n_compressed, self.rope, self.fp8 = head_dim, window, n_compressed, rope, fp8
        n = window + n_compressed
        dev = torch.device(device)
        if fp8:
            self.cache = (torch.zeros(n, head_dim - rope, dtype=torch.uint8, device=dev),
                          torch.zeros(n, (head_dim - rope) // 64, dtype=torch.float32, device=dev),
                          torch.zeros(n, rope, dtype=torch.bfloat16, device=dev))
        else:
            self.cache = torch.zeros(n, head_dim, dtype=torch.bfloat16, device=dev)

    def write_window(self, kv: torch.Tensor, start_pos: int) -> None:
        """kv [1, head_dim] bf16 of position ``start_pos`` -> ring slot start_pos % window."""
        slots = torch.full((kv.shape[0],), start_pos % self.window, dtype=torch.int32, device=kv.device)
        ops.dsa_kv_write(kv, self.cache, slots, self.rope)

    def write_compressed(self, ckv: torch.Tensor, first: int = 0) -> None:
        """Compressed kv rows [c, head_dim] -> compressed entries first .. first + c - 1."""
        if first < 0 or first + ckv.shape[0] > self.n_compressed:
            raise ValueError(f"compressed rows {first}..{first + ckv.shape[0]} beyond {self.n_compressed}")
        slots = torch.arange(self.window + first, self.window + first + ckv.shape[0], dtype=torch.int32,
                             device=ckv.device)
        ops.dsa_kv_write(ckv, self.cache, slots, self.rope)

    def attend(self, q: torch.Tensor, start_pos: int, softmax_scale: float, sink: torch.Tensor | None = None,
               cidx: torch.Tensor | None = None, ratio: int = 4) -> torch.Tensor:
        """q [1, H, head_dim] bf16 at position start_pos over the window and the
        compressed entries: the indexer picks ``cidx`` [1, t] (already offset by
        window) or, without them, every compressed entry up to (p + 1) // ratio."""
        pos = torch.full((q.shape[0],), start_pos, dtype=torch.int32, device=q.device)
        idx = ops.dsa_decode_indices(pos, self.window, cidx, nc=None if cidx is not None else self.n_compressed,
                                     ratio=ratio, offset=self.window)
        n = self.window + self.n_compressed
        if self.fp8:
            codes, scales, rope = self.cache
            return ops.mla_sparse_decode(q, codes.view(1, n, -1), scales.view(1, n, -1), rope.view(1, n, -1), idx,
                                         softmax_scale, sink)
        return _attend(q, self.cache.view(1, n, -1), sink, idx, softmax_scale)

    def step(self, q: torch.Tensor, kv: torch.Tensor, start_pos: int, softmax_scale: float,
             sink: torch.Tensor | None = None, cidx: torch.Tensor | None = None, ratio: int = 4) -> torch.Tensor:
        """One decode step: write kv into the ring, then attend (the order of
        ``_core_body``'s ``s == 1`` branch)."""
        self.write_window(kv, start_pos)
        return self.attend(q, start_pos, softmax_scale, sink, cidx, ratio)

