"""DSA drop-ins: the lightning indexer with top-k and sparse (MLA) attention.

* ``sparse_attn(q, kv, attn_sink, topk_idxs, softmax_scale)`` -- upstream
  signature (``.mosaicvm/source/inference_kernel.py:355-368``): q [b, m, h, d]
  bf16, kv [b, n, d] bf16, topk_idxs [b, m, topk] int32 -> o [b, m, h, d].
  V = K (d = 512, the V4 geometry, on the MLA kernels; d = 64, 128, 256 on
  the small-head-dim kernel); heads are padded to the kernel's head groups and
  stripped, as upstream pads to 16.
* ``sparse_attn_fused(q, kv, sink, topk_idxs, scale)`` and ``sparse_attn_ref``
  -- ``mosaicvm/kernels/dsa_sparse.py:92-110`` / ``mosaicvm/model/dsa.py:214-242``:
  q [s, h, d], kv [n, d], topk_idxs [s, t] -> o [s, h, d] (bf16 only;
  d in {64, 128, 256, 512}, the reference's set).
* ``indexer_topk`` / ``indexer_scores`` -- the FP8 indexer of ``Indexer.forward``
  (``.mosaicvm/source/inference_model.py:408-439``) from quantized q/k.
* ``mla_decode_fp8`` -- MLA decode over an FP8 latent cache (the benchmark spec's format).
* ``dsa_decode_attention(q, k_index, v_full, topk, scale)`` --
  ``mosaicvm/kernels/dsa_attention.py:113-154``: per-head top-k positions and
  softmax attention over them for one token (q [H, d], k_index [ctx, H, d],
  v_full [ctx, H, dv] bf16) -> (out [H, dv], idx [H, topk]); picks listed by
  descending score, ties to the lower position.
* ``Indexer`` -- ``Indexer.forward(x, qr, freqs, offset, start_pos)``
  (``mosaicvm/model/dsa_layers.py:281-321``, upstream
  ``.mosaicvm/source/inference_model.py:408-439``): the wq_b and weights_proj
  projections on this build's kernels, the caller's rope / Hadamard / fp4
  simulation / compressor, an FP8 key cache and the FP8 indexer + top-k;
  ``score_topk`` is the scoring stage alone over FP8 operands.
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
    if d not in (64, 128, 256, 512):
        raise ValueError(f"sparse attention drop-in supports head dims 64, 128, 256 and 512 (V = K), got {d}; "
                         "use ops.mla_sparse_decode_bf16 for the 576 = 512 + 64 MLA layout")
    hp = _padded_heads(h) if d == 512 else -(-h // 16) * 16
    if hp != h:
        q3 = torch.cat([q3, q3.new_zeros(rows, hp - h, d)], dim=1)
        if sink is not None:
            sink = torch.cat([sink.float(), sink.new_zeros(hp - h, dtype=torch.float32)])
    sink = None if sink is None else sink.float().contiguous()
    if d == 512:
        o = ops.mla_sparse_decode_bf16(q3, kv3, idx2, scale, sink)
    else:
        o = ops.sparse_attn_bf16(q3, kv3, idx2, scale, sink)
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
    """The DSA lightning indexer with the reference's module interface.

    ``forward(x, qr, freqs, offset, start_pos=0)`` -- ``mosaicvm/model/dsa_layers.py:281-321``
    (upstream ``forward(x, qr, start_pos, offset)``,
    ``.mosaicvm/source/inference_model.py:408-439``): x [s, dim] and qr
    [s, q_lora_rank] bf16 of one sequence -> topk_idxs [s, min(index_topk,
    end_pos // ratio)] int32.  In order:

    * q = wq_b(qr) on this build's FP8 W8A16 linear (``wq_b`` e4m3 [H * hd,
      q_lora_rank] with fp32 128 x 128 block scales ``wq_b_scale``, the V4
      checkpoint format), viewed [s, H, hd];
    * the caller's ``rotary(q[..., -rope_dim:], freqs[start_pos:end_pos])``,
      ``hadamard(q)`` and ``q_quant(q)`` (the fp4 simulation), each skipped when
      None: they are the model's, not on the quantized matrix path;
    * the caller's ``compressor(x, start_pos)``, which writes its bf16
      ``kv_cache`` rows; the rows this call can have written (start_pos //
      ratio .. end_pos // ratio - 1) are quantized into the indexer's FP8 key
      cache (e4m3 with one fp32 scale per token, amax / 448), rows before them
      were quantized by earlier calls;
    * weights = weights_proj(x) (bf16 [H, dim], the exact-rounded router GEMV)
      * hd^-0.5 * H^-0.5;
    * q quantized to e4m3 with one fp32 scale per (row, head) (amax / 448), and
      the FP8 indexer + top-k over the cache: score = sum over heads of w_h
      ReLU(q_h . k_t q_s k_s) in the canonical order, ties to the lower index
      (the reference leaves them to torch.topk); when start_pos == 0 or s > 1
      row t sees the first (start_pos + t + 1) // ratio entries and its picks
      past them are -1, valid picks get ``+ offset``.

    The scoring runs in the FP8 format of the build's indexer (q and k e4m3
    with fp32 scales), where the reference scores bf16 q against the bf16
    cache.

    ``score_topk(q_fp8, q_scale, weights, k_cache, k_scale, start_pos, offset)``
    is the scoring and top-k stage alone over already projected FP8 q
    [bsz, seqlen, H, 128] (+ [bsz, seqlen, H] scales and weights) and a batched
    FP8 key cache [bsz, >= end_pos // ratio, 128] (+ [bsz, ...] f32 scales),
    read in place; the causal mask applies at start_pos == 0 (upstream)."""

    def __init__(self, n_heads: int = 64, head_dim: int = 128, index_topk: int = 2048, compress_ratio: int = 4,
                 rope_dim: int = 64, max_seq_len: int = 4096, rotary=None, hadamard=None, q_quant=None,
                 compressor=None, device=None):
        super().__init__()
        self.n_heads, self.head_dim, self.rope_dim = n_heads, head_dim, rope_dim
        self.index_topk = index_topk
        self.compress_ratio = compress_ratio
        self.softmax_scale = head_dim ** -0.5
        self.rotary, self.hadamard, self.q_quant, self.compressor = rotary, hadamard, q_quant, compressor
        self.wq_b: torch.Tensor | None = None        # e4m3 [H * hd, q_lora_rank]
        self.wq_b_scale: torch.Tensor | None = None  # f32 [ceil(H * hd / 128), q_lora_rank / 128]
        self.weights_proj: torch.Tensor | None = None  # bf16 [H, dim]
        n_c = max_seq_len // compress_ratio
        self.register_buffer("k_fp8", torch.zeros(n_c, head_dim, dtype=torch.uint8, device=device), persistent=False)
        self.register_buffer("k_scale", torch.zeros(n_c, dtype=torch.float32, device=device), persistent=False)

    def forward(self, x: torch.Tensor, qr: torch.Tensor, freqs: torch.Tensor, offset: int,
                start_pos: int = 0) -> torch.Tensor:
        from .fp8 import fp8_linear
        if self.wq_b is None or self.wq_b_scale is None or self.weights_proj is None or self.compressor is None:
            raise RuntimeError("Indexer.forward needs wq_b / wq_b_scale, weights_proj and a compressor")
        s = x.shape[0]
        h, hd, ratio = self.n_heads, self.head_dim, self.compress_ratio
        end_pos = start_pos + s
        n_c = end_pos // ratio
        if n_c > self.k_fp8.shape[0]:
            raise ValueError(f"end_pos {end_pos} is past the cache of {self.k_fp8.shape[0] * ratio} positions")
        q = fp8_linear(qr.to(torch.bfloat16), self.wq_b, self.wq_b_scale).view(s, h, hd)
        if self.rotary is not None:
            q = torch.cat([q[..., :-self.rope_dim], self.rotary(q[..., -self.rope_dim:], freqs[start_pos:end_pos])],
                          -1)
        if self.hadamard is not None:
            q = self.hadamard(q)
        if self.q_quant is not None:
            q = self.q_quant(q)
        self.compressor(x, start_pos)
        first = start_pos // ratio
        if n_c > first:  # the rows this call's compressor can have written
            kq, ksc = ops.act_quant(self.compressor.kv_cache[first:n_c].reshape(n_c - first, hd), hd, "amax")
            self.k_fp8[first:n_c].copy_(kq.view(torch.uint8))
            self.k_scale[first:n_c].copy_(ksc.reshape(-1))
        k = min(self.index_topk, n_c)
        if k == 0:
            return torch.empty(s, 0, dtype=torch.int32, device=x.device)
        w = ops.router_logits(x, self.weights_proj) * (self.softmax_scale * h ** -0.5)
        q8, qs = ops.act_quant(q.reshape(s * h, hd).to(torch.bfloat16), hd, "amax")
        if start_pos == 0 or s > 1:  # causal: row t sees the first (start_pos + t + 1) // ratio entries
            lengths = ((torch.arange(1, s + 1, device=x.device) + start_pos) // ratio).to(torch.int32)
        else:
            lengths = torch.full((s,), n_c, dtype=torch.int32, device=x.device)
        return ops.dsa_indexer_topk_shared(q8.view(s, h, hd), qs.view(s, h), self.k_fp8[None, :n_c],
                                           self.k_scale[None, :n_c], w, k, lengths, offset)

    def score_topk(self, q_fp8, q_scale, weights, k_cache, k_scale, start_pos: int, offset: int):
        bsz, seqlen, h, d = q_fp8.shape
        ratio = self.compress_ratio
        end_pos = start_pos + seqlen
        n_c = end_pos // ratio
        k = min(self.index_topk, n_c)
        if k == 0:
            return torch.empty(bsz, seqlen, 0, dtype=torch.int32, device=q_fp8.device)
        q2 = q_fp8.reshape(bsz * seqlen, h, d)
        qs2, w2 = q_scale.reshape(bsz * seqlen, h).float(), weights.reshape(bsz * seqlen, h).float()
        if start_pos == 0:  # causal: position i scores the first (i + 1) // ratio compressed entries
            bounds = (torch.arange(1, seqlen + 1, device=q_fp8.device) // ratio).to(torch.int32)
            lengths = bounds.repeat(bsz)
        else:
            lengths = torch.full((bsz * seqlen,), n_c, dtype=torch.int32, device=q_fp8.device)
        # the caches are read in place (their first n_c tokens, cache length = the buffer's)
        idx = ops.dsa_indexer_topk_shared(q2, qs2, k_cache[:, :n_c], k_scale[:, :n_c].float(), w2, k, lengths,
                                          offset)
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

