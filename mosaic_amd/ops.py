"""Typed torch wrappers over the C ABI (device tensors in, device tensors out).

Every function validates shapes/dtypes on the host, allocates its outputs with
``torch.empty`` on the input's device, and enqueues the HIP kernels on torch's
current stream.  Nothing here synchronizes or reads device data back.  There
is no CPU path: a CPU tensor raises ``ValueError``.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib

DT_F32, DT_BF16 = 0, 1
SCORE_FUNCS = {"sigmoid": 0, "softmax": 1, "sqrtsoftplus": 2}
ACT_MODES = {"pow2": 0, "amax": 1, "hf": 2, "legacy": 3}
RECIPES = {"ceil": 0, "floor": 1}


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _cuda(t: torch.Tensor, name: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor (mosaic_amd has no CPU path), got {t.device}")
    return t.contiguous()


def _on_device(t: torch.Tensor, name: str) -> torch.Tensor:
    """The checks of ``_cuda`` without the copy to a contiguous tensor (for
    operands that are read through their strides)."""
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor (mosaic_amd has no CPU path), got {t.device}")
    return t


def _u8(t: torch.Tensor, name: str) -> torch.Tensor:
    t = _cuda(t, name)
    if t.dtype in (torch.uint8, torch.int8, torch.float8_e8m0fnu, torch.float8_e4m3fn):
        return t.view(torch.uint8)
    if hasattr(torch, "float4_e2m1fn_x2") and t.dtype == torch.float4_e2m1fn_x2:
        return t.view(torch.uint8)
    raise ValueError(f"{name}: expected a byte tensor (uint8/int8/e8m0/e4m3/fp4x2), got {t.dtype}")


def _bf16(t: torch.Tensor, name: str) -> torch.Tensor:
    t = _cuda(t, name)
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name}: expected bfloat16, got {t.dtype}")
    return t


# --------------------------------------------------------------- codecs -----
def mx_quantize(w: torch.Tensor, recipe: str = "ceil") -> tuple[torch.Tensor, torch.Tensor]:
    """w [R, C] (bf16/f32) -> (packed u8 [R, C/2], e8m0 u8 [R, C/32]), blocks of
    32 along the last dim."""
    w = _cuda(w, "w")
    if w.dim() != 2:
        raise ValueError(f"mx_quantize expects a 2-D tensor, got {tuple(w.shape)}")
    if w.dtype not in (torch.bfloat16, torch.float32):
        w = w.to(torch.float32)
    r, c = w.shape
    if c % 32:
        raise ValueError(f"last dim {c} must be a multiple of 32")
    packed = torch.empty(r, c // 2, dtype=torch.uint8, device=w.device)
    scale = torch.empty(r, c // 32, dtype=torch.uint8, device=w.device)
    _lib.call("mosaic_mx_quantize", _ptr(w), DT_BF16 if w.dtype == torch.bfloat16 else DT_F32, _ptr(packed),
              _ptr(scale), r, c, RECIPES[recipe], _stream())
    return packed, scale


def mx_dequant(packed: torch.Tensor, scale: torch.Tensor, dtype=torch.bfloat16) -> torch.Tensor:
    """packed [R, C/2] + e8m0 [R, C/32] -> [R, C] (bf16 or f32)."""
    packed = _u8(packed, "packed")
    scale = _u8(scale, "scale")
    if packed.dim() != 2:
        raise ValueError(f"packed must be 2-D, got {tuple(packed.shape)}")
    r, ch = packed.shape
    c = 2 * ch
    if c % 32 or tuple(scale.shape) != (r, c // 32):
        raise ValueError(f"scale shape {tuple(scale.shape)} != ({r}, {c // 32})")
    if dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"dtype {dtype}")
    out = torch.empty(r, c, dtype=dtype, device=packed.device)
    _lib.call("mosaic_mx_dequant", _ptr(packed), _ptr(scale), _ptr(out),
              DT_BF16 if dtype == torch.bfloat16 else DT_F32, r, c, _stream())
    return out


def act_quant(x: torch.Tensor, block: int = 128, mode: str = "pow2") -> tuple[torch.Tensor, torch.Tensor]:
    """x [M, K] -> (e4m3fn codes [M, K], f32 scales [M, K/block])."""
    x = _cuda(x, "x")
    if x.dim() != 2:
        raise ValueError(f"act_quant expects [M, K], got {tuple(x.shape)}")
    if x.dtype not in (torch.bfloat16, torch.float32):
        x = x.to(torch.float32)
    m, k = x.shape
    if k % block:
        raise ValueError(f"K={k} must be a multiple of act block {block}")
    q = torch.empty(m, k, dtype=torch.uint8, device=x.device)
    s = torch.empty(m, k // block, dtype=torch.float32, device=x.device)
    _lib.call("mosaic_act_quant", _ptr(x), DT_BF16 if x.dtype == torch.bfloat16 else DT_F32, _ptr(q), _ptr(s), m, k,
              block, ACT_MODES[mode], _stream())
    return q.view(torch.float8_e4m3fn), s


def rmsnorm_act_quant(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6, mode: str = "pow2",
                      return_y: bool = False):
    """RMSNorm of x [M, H] bf16 (weight [H]) with the 1x128 act_quant fused into
    its epilogue -> (e4m3fn codes [M, H], f32 scales [M, H/128]) [, y bf16
    [M, H]]: the input of ``mxt16_linear_a8(..., prequant=...)`` /
    ``fp8_block_gemm`` without a bf16 round trip through HBM."""
    x = _bf16(x, "x").contiguous()
    if x.dim() != 2:
        raise ValueError(f"rmsnorm_act_quant expects [M, H], got {tuple(x.shape)}")
    m, h = x.shape
    w = _cuda(weight, "weight").to(torch.float32).contiguous()
    if tuple(w.shape) != (h,):
        raise ValueError(f"weight must be [{h}], got {tuple(w.shape)}")
    q = torch.empty(m, h, dtype=torch.uint8, device=x.device)
    s = torch.empty(m, h // 128, dtype=torch.float32, device=x.device)
    y = torch.empty(m, h, dtype=torch.bfloat16, device=x.device) if return_y else None
    _lib.call("mosaic_rmsnorm_act_quant", _ptr(x), _ptr(w), float(eps), m, h, _ptr(y), _ptr(q), _ptr(s),
              ACT_MODES[mode], _stream())
    out = (q.view(torch.float8_e4m3fn), s)
    return out + (y,) if return_y else out


def swiglu_act_quant(gu: torch.Tensor, w_a: torch.Tensor | None, inter: int,
                     swiglu_limit: float = 0.0) -> tuple[torch.Tensor, torch.Tensor]:
    """gu [A, 2*inter] bf16 (gate | up), route weights w_a [A] (None: 1) ->
    (e4m3fn codes [A, inter], f32 pow2 scales [A, inter/128]) of
    z = bf16(silu(min(gate, L)) * clamp(up, +-L) * w); no clamp when L <= 0."""
    gu = _bf16(gu, "gu").contiguous()
    a = gu.shape[0]
    if gu.dim() != 2 or gu.shape[1] != 2 * inter or inter % 128:
        raise ValueError(f"gu must be [A, 2*inter] with inter % 128 == 0, got {tuple(gu.shape)}, inter={inter}")
    w = None
    if w_a is not None:
        w = _cuda(w_a, "w_a").reshape(-1).to(torch.float32).contiguous()
        if w.numel() != a:
            raise ValueError(f"w_a must hold {a} weights, got {w.numel()}")
    q = torch.empty(a, inter, dtype=torch.uint8, device=gu.device)
    s = torch.empty(a, inter // 128, dtype=torch.float32, device=gu.device)
    _lib.call("mosaic_swiglu_act_quant", _ptr(gu), _ptr(w), a, inter, float(swiglu_limit), _ptr(q), _ptr(s),
              _stream())
    return q.view(torch.float8_e4m3fn), s


def routed_reduce(yd: torch.Tensor, slot_rows: torch.Tensor, order: torch.Tensor, h: int) -> torch.Tensor:
    """yd [A, h] bf16 partials, slot_rows / order [k_tok, top_k] -> bf16 [k_tok, h]:
    out[t] = fp32 sum of yd[slot_rows[t, order[t, j]]] over j in that order."""
    yd = _bf16(yd, "yd").contiguous()
    if yd.dim() != 2 or yd.shape[1] != h:
        raise ValueError(f"yd must be [A, {h}], got {tuple(yd.shape)}")
    if slot_rows.dim() != 2 or tuple(order.shape) != tuple(slot_rows.shape):
        raise ValueError(f"slot_rows and order must be [k_tok, top_k], got {tuple(slot_rows.shape)} "
                         f"and {tuple(order.shape)}")
    sr = _cuda(slot_rows, "slot_rows").to(torch.int32).contiguous()
    od = _cuda(order, "order").to(torch.int32).contiguous()
    k_tok, top_k = sr.shape
    out = torch.empty(k_tok, h, dtype=torch.bfloat16, device=yd.device)
    _lib.call("mosaic_routed_reduce", _ptr(yd), _ptr(sr), _ptr(od), _ptr(out), k_tok, top_k, h, yd.shape[0],
              _stream())
    return out


def e4m3_decode(codes: torch.Tensor) -> torch.Tensor:
    codes = _u8(codes, "codes")
    out = torch.empty(codes.shape, dtype=torch.float32, device=codes.device)
    _lib.call("mosaic_e4m3_decode", _ptr(codes), _ptr(out), codes.numel(), _stream())
    return out


def e4m3_encode(x: torch.Tensor) -> torch.Tensor:
    x = _cuda(x, "x").to(torch.float32)
    out = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    _lib.call("mosaic_e4m3_encode", _ptr(x), _ptr(out), x.numel(), _stream())
    return out


def selfcheck_converters(device=None) -> list[int]:
    """Mismatch counts [bf16, e4m3] of gfx950's hardware converters against the
    library's software roundings over every fp32 input (see the C header)."""
    counts = torch.zeros(2, dtype=torch.int64, device=device or torch.device("cuda", torch.cuda.current_device()))
    _lib.call("mosaic_selfcheck_converters", _ptr(counts), _stream())
    return counts.cpu().tolist()


# ------------------------------------------------------------- A16 linear ---
def mx_linear_a16(x: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """y [M, N] bf16 = x [M, K] bf16 . dequant(packed [N, K/2], scale [N, K/32])^T."""
    x = _bf16(x, "x")
    packed = _u8(packed, "packed")
    scale = _u8(scale, "scale")
    if x.dim() != 2 or packed.dim() != 2:
        raise ValueError("x and packed must be 2-D")
    m, k = x.shape
    n, kh = packed.shape
    if kh * 2 != k:
        raise ValueError(f"packed K {kh * 2} != x K {k}")
    if k % 128:
        raise ValueError(f"K={k} must be a multiple of 128")
    if tuple(scale.shape) != (n, k // 32):
        raise ValueError(f"scale shape {tuple(scale.shape)} != ({n}, {k // 32})")
    y = torch.empty(m, n, dtype=torch.bfloat16, device=x.device)
    _lib.call("mosaic_mx_linear_a16", _ptr(x), _ptr(packed), _ptr(scale), _ptr(y), m, n, k, _stream())
    return y


def mx_kn_linear_a16(x: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """y [M, N] bf16 = x [M, K] bf16 . W for a KN-layout MXFP4 weight:
    packed [K, N/2] (low nibble = even n), e8m0 scale [K, N/32]."""
    x = _bf16(x, "x")
    packed = _u8(packed, "packed")
    scale = _u8(scale, "scale")
    if x.dim() != 2 or packed.dim() != 2:
        raise ValueError("x and packed must be 2-D")
    m, k = x.shape
    kp, nh = packed.shape
    n = 2 * nh
    if kp != k:
        raise ValueError(f"packed K={kp} != x K={k}")
    if n % 32 or k % 32:
        raise ValueError(f"N={n} and K={k} must be multiples of 32")
    if tuple(scale.shape) != (k, n // 32):
        raise ValueError(f"scale shape {tuple(scale.shape)} != ({k}, {n // 32})")
    y = torch.empty(m, n, dtype=torch.bfloat16, device=x.device)
    nbytes = _lib.lib().mosaic_mx_kn_linear_a16_workspace_bytes(m, n, k)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device) if nbytes else None
    _lib.call("mosaic_mx_kn_linear_a16", _ptr(x), _ptr(packed), _ptr(scale), _ptr(y), m, n, k, _ptr(ws), nbytes,
              _stream())
    return y


def moe_skinny_forward(x: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor, gu_packed: torch.Tensor,
                       gu_scale: torch.Tensor, d_packed: torch.Tensor, d_scale: torch.Tensor) -> torch.Tensor:
    """fused_moe_skinny arithmetic over KN expert banks: gu [E, H, I] + [E, H, 2I/32]
    (gate columns then up columns), down [E, I, H/2] + [E, I, H/32] -> y [M, H] bf16."""
    x = _bf16(x, "x")
    gu_packed, gu_scale = _u8(gu_packed, "packed_gate_up"), _u8(gu_scale, "scale_gate_up")
    d_packed, d_scale = _u8(d_packed, "packed_down"), _u8(d_scale, "scale_down")
    m, h = x.shape
    if gu_packed.dim() != 3 or d_packed.dim() != 3:
        raise ValueError("expert banks must be [E, K, N/2]")
    e, kh, inter = gu_packed.shape  # N = 2 * inter columns, inter bytes per row
    if kh != h or tuple(gu_scale.shape) != (e, h, 2 * inter // 32):
        raise ValueError(f"gate/up bank {tuple(gu_packed.shape)}/{tuple(gu_scale.shape)} does not match hidden {h}")
    if tuple(d_packed.shape) != (e, inter, h // 2) or tuple(d_scale.shape) != (e, inter, h // 32):
        raise ValueError(f"down bank {tuple(d_packed.shape)}/{tuple(d_scale.shape)} does not match [{e}, {inter}, {h}]")
    ids = _cuda(ids, "expert_ids")
    if m == 0:  # an empty batch: nothing to launch
        return torch.empty(0, h, dtype=torch.bfloat16, device=x.device)
    ids = ids.reshape(m, -1).to(torch.int32).contiguous()
    k = ids.shape[1]
    weights = _cuda(weights, "expert_weights").reshape(m, k).to(torch.float32).contiguous()
    y = torch.empty(m, h, dtype=torch.bfloat16, device=x.device)
    nbytes = _lib.lib().mosaic_moe_skinny_workspace_bytes(m, h, inter, e, k)
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=x.device)
    _lib.call("mosaic_moe_skinny_forward", _ptr(x), _ptr(ids), _ptr(weights), _ptr(gu_packed), _ptr(gu_scale),
              _ptr(d_packed), _ptr(d_scale), _ptr(y), m, h, inter, e, k, _ptr(ws), ws.numel(), _stream())
    return y


# ------------------------------------------------------- MXT16 prepack ------
@dataclass
class MXT16:
    """An MXFP4 NK weight (or a stack of them) prepacked into MFMA tile order.

    ``packed`` keeps the raw tensor's shape [..., N, K/2]; ``scale`` is
    [..., N/16 * ceil(K/512) * 256] bytes.  ``n``/``k`` are the per-matrix dims."""
    packed: torch.Tensor
    scale: torch.Tensor
    n: int
    k: int

    @property
    def lead(self) -> tuple:
        return tuple(self.packed.shape[:-2])


def _t16_scale_bytes(n: int, k: int) -> int:
    return (n // 16) * ((k // 128 + 3) // 4) * 256


def mxt16_prepack(packed: torch.Tensor, scale: torch.Tensor) -> MXT16:
    """Raw NK MXFP4 ([..., N, K/2] + [..., N, K/32]) -> MXT16 (bit-exact permutation)."""
    packed = _u8(packed, "packed")
    scale = _u8(scale, "scale")
    if packed.dim() < 2:
        raise ValueError(f"packed must be [..., N, K/2], got {tuple(packed.shape)}")
    n, kh = packed.shape[-2], packed.shape[-1]
    k = 2 * kh
    if n % 16 or k % 128:
        raise ValueError(f"MXT16 needs N % 16 == 0 and K % 128 == 0, got N={n} K={k}")
    if tuple(scale.shape) != tuple(packed.shape[:-1]) + (k // 32,):
        raise ValueError(f"scale shape {tuple(scale.shape)} != {tuple(packed.shape[:-1]) + (k // 32,)}")
    lead = tuple(packed.shape[:-2])
    rows = packed.numel() // kh
    pt = torch.empty_like(packed)
    st = torch.empty(lead + (_t16_scale_bytes(n, k),), dtype=torch.uint8, device=packed.device)
    _lib.call("mosaic_mxt16_prepack", _ptr(packed), _ptr(scale), _ptr(pt), _ptr(st), rows, k, _stream())
    return MXT16(pt, st, n, k)


def mxt16_unpack(w: MXT16) -> tuple[torch.Tensor, torch.Tensor]:
    """Inverse of ``mxt16_prepack``."""
    rows = w.packed.numel() // (w.k // 2)
    packed = torch.empty_like(w.packed)
    scale = torch.empty(w.lead + (w.n, w.k // 32), dtype=torch.uint8, device=w.packed.device)
    _lib.call("mosaic_mxt16_unpack", _ptr(w.packed), _ptr(w.scale), _ptr(packed), _ptr(scale), rows, w.k, _stream())
    return packed, scale


def mxt16_linear_a16(x: torch.Tensor, w: MXT16) -> torch.Tensor:
    """y [M, N] bf16 = x [M, K] bf16 . dequant(W)^T for a prepacked 2-D weight."""
    x = _bf16(x, "x")
    if w.lead:
        raise ValueError("mxt16_linear_a16 takes a single matrix")
    if x.dim() != 2 or x.shape[1] != w.k:
        raise ValueError(f"x shape {tuple(x.shape)} does not match K={w.k}")
    m = x.shape[0]
    y = torch.empty(m, w.n, dtype=torch.bfloat16, device=x.device)
    _lib.call("mosaic_mxt16_linear_a16", _ptr(x), _ptr(w.packed), _ptr(w.scale), _ptr(y), m, w.n, w.k, _stream())
    return y


def mxt16_linear_a8(x: torch.Tensor | None, w: MXT16, prequant: tuple | None = None) -> torch.Tensor:
    """A8 linear: y [M, N] bf16 from bf16 x (quantized here, 1x128 power-of-two
    e4m3) or ``prequant`` = (codes e4m3 [M, K], scales f32 [M, K/128])."""
    if w.lead:
        raise ValueError("mxt16_linear_a8 takes a single matrix")
    if prequant is None:
        xq, sa = act_quant(x, 128, "pow2")
    else:
        xq, sa = prequant
    xq = _u8(xq, "xq")
    sa = _cuda(sa, "sa").to(torch.float32).contiguous()
    if xq.dim() != 2 or xq.shape[1] != w.k or tuple(sa.shape) != (xq.shape[0], w.k // 128):
        raise ValueError(f"activation shapes {tuple(xq.shape)}/{tuple(sa.shape)} do not match K={w.k}")
    m = xq.shape[0]
    y = torch.empty(m, w.n, dtype=torch.bfloat16, device=xq.device)
    # fp32 partials of the split-K plan (shapes whose tiles cover at most half of the GPU)
    nbytes = _lib.lib().mosaic_mxt16_linear_a8_workspace_bytes(m, w.n, w.k)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=xq.device) if nbytes else None
    _lib.call("mosaic_mxt16_linear_a8_ws", _ptr(xq), _ptr(sa), _ptr(w.packed), _ptr(w.scale), _ptr(y), m, w.n, w.k,
              _ptr(ws), nbytes, _stream())
    return y


# ------------------------------------------------------- FP8 block GEMM -----
FP8_T16_MAX_M = 64  # rows up to which fp8_block_gemm takes a T16-prepacked weight


@dataclass
class FP8T16:
    """An e4m3 weight [N, K] (N % 16 == 0, K % 128 == 0) prepacked for the decode
    kernel: ``codes`` holds the same N * K bytes, each 16-row x 128-K block as
    2 KB in MFMA lane order (``mosaic_fp8_t16_prepack``)."""
    codes: torch.Tensor
    n: int
    k: int


def fp8_t16_prepack(b: torch.Tensor) -> FP8T16:
    """e4m3 codes [N, K] -> FP8T16 (bit-exact permutation)."""
    b = _u8(b, "b")
    if b.dim() != 2:
        raise ValueError(f"b must be [N, K], got {tuple(b.shape)}")
    n, k = b.shape
    if n % 16 or k % 128 or k == 0:
        raise ValueError(f"FP8T16 needs N % 16 == 0 and K a positive multiple of 128, got N={n} K={k}")
    out = torch.empty_like(b)
    _lib.call("mosaic_fp8_t16_prepack", _ptr(b), _ptr(out), n, k, _stream())
    return FP8T16(out, n, k)


def fp8_t16_unpack(w: FP8T16) -> torch.Tensor:
    """Inverse of ``fp8_t16_prepack``: uint8 codes [N, K]."""
    out = torch.empty_like(w.codes)
    _lib.call("mosaic_fp8_t16_unpack", _ptr(w.codes), _ptr(out), w.n, w.k, _stream())
    return out


def fp8_block_gemm(a: torch.Tensor, a_s: torch.Tensor, b: torch.Tensor | FP8T16, b_s: torch.Tensor,
                   out_dtype=torch.bfloat16) -> torch.Tensor:
    """C [M, N] = block-scaled e4m3 GEMM (A [M, K] + a_s [M, K/128], B [N, K] + b_s [ceil(N/128), K/128]).

    ``b`` may be an ``FP8T16`` prepack for M <= 64 (at M <= 16 the same C bit for bit)."""
    a = _u8(a, "a")
    t16 = isinstance(b, FP8T16)
    if not t16:
        b = _u8(b, "b")
    if a.dim() != 2 or (not t16 and b.dim() != 2):
        raise ValueError("a and b must be 2-D")
    m, k = a.shape
    n, kb = (b.n, b.k) if t16 else b.shape
    if t16 and m > FP8_T16_MAX_M:
        raise ValueError(f"a T16-prepacked weight serves M <= {FP8_T16_MAX_M}, got M={m}; pass the [N, K] codes")
    if kb != k:
        raise ValueError(f"K mismatch: a {k}, b {kb}")
    if k % 128:
        raise ValueError(f"K={k} must be a multiple of 128")
    a_s = _cuda(a_s, "a_s").to(torch.float32).contiguous()
    b_s = _cuda(b_s, "b_s").to(torch.float32).contiguous()
    if tuple(a_s.shape) != (m, k // 128):
        raise ValueError(f"a_s shape {tuple(a_s.shape)} != ({m}, {k // 128})")
    if tuple(b_s.shape) != ((n + 127) // 128, k // 128):
        raise ValueError(f"b_s shape {tuple(b_s.shape)} != ({(n + 127) // 128}, {k // 128})")
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"out_dtype {out_dtype}")
    c = torch.empty(m, n, dtype=out_dtype, device=a.device)
    dt = DT_F32 if out_dtype == torch.float32 else DT_BF16
    if t16:
        nbytes = _lib.lib().mosaic_fp8_block_gemm_t16_workspace_bytes(m, n, k)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=a.device) if nbytes else None
        _lib.call("mosaic_fp8_block_gemm_t16", _ptr(a), _ptr(a_s), _ptr(b.codes), _ptr(b_s), _ptr(c), dt, m, n, k,
                  _ptr(ws), nbytes, _stream())
        return c
    # partials of the split-K plan (shapes whose tiles cover under half the GPU)
    nbytes = _lib.lib().mosaic_fp8_block_gemm_workspace_bytes(m, n, k)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=a.device) if nbytes else None
    _lib.call("mosaic_fp8_block_gemm_ws", _ptr(a), _ptr(a_s), _ptr(b), _ptr(b_s), _ptr(c), dt, m, n, k, _ptr(ws),
              nbytes, _stream())
    return c


W8A16_MAX_M = 80  # rows up to which fp8_linear decodes in the GEMM (bench/fp8_core.py:210-221)


def fp8_w8a16_linear(x: torch.Tensor, w: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """y [M, N] bf16 = x [M, K] bf16 . (e4m3 W [N, K] x per-128x128 block scales s)^T,
    the weight decoded inside the GEMM (M <= 80)."""
    x = _bf16(x, "x")
    w = _u8(w, "w_fp8")
    if x.dim() != 2 or w.dim() != 2 or x.shape[1] != w.shape[1]:
        raise ValueError(f"x {tuple(x.shape)} and w {tuple(w.shape)} must be [M, K] and [N, K]")
    m, k = x.shape
    n = w.shape[0]
    if k % 128:
        raise ValueError(f"K={k} must be a multiple of 128")
    if m > W8A16_MAX_M:
        raise ValueError(f"fp8_w8a16_linear decodes in the GEMM for M <= {W8A16_MAX_M}, got {m}")
    s = _cuda(s, "s").to(torch.float32).contiguous()
    if tuple(s.shape) != ((n + 127) // 128, k // 128):
        raise ValueError(f"scale shape {tuple(s.shape)} != ({(n + 127) // 128}, {k // 128})")
    y = torch.empty(m, n, dtype=torch.bfloat16, device=x.device)
    # partials of the split-K plan (shapes whose workgroups cover few CUs in one K pass)
    nbytes = _lib.lib().mosaic_fp8_w8a16_workspace_bytes(m, n, k)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device) if nbytes else None
    _lib.call("mosaic_fp8_w8a16_linear_ws", _ptr(x), _ptr(w), _ptr(s), _ptr(y), m, n, k, _ptr(ws), nbytes,
              _stream())
    return y


def fp8_block_dequant(w: torch.Tensor, s: torch.Tensor, block: tuple[int, int] = (128, 128)) -> torch.Tensor:
    """e4m3 [N, K] + f32 scales [ceil(N/bn), ceil(K/bk)] -> bf16 [N, K]."""
    w = _u8(w, "w")
    if w.dim() != 2:
        raise ValueError("w must be 2-D")
    n, k = w.shape
    bn, bk = block
    s = _cuda(s, "s").to(torch.float32).contiguous()
    if tuple(s.shape) != ((n + bn - 1) // bn, (k + bk - 1) // bk):
        raise ValueError(f"scale shape {tuple(s.shape)} does not tile [{n}, {k}] by {block}")
    out = torch.empty(n, k, dtype=torch.bfloat16, device=w.device)
    _lib.call("mosaic_fp8_block_dequant", _ptr(w), _ptr(s), _ptr(out), n, k, bn, bk, _stream())
    return out


# ---------------------------------------------------------------- routing ---
def moe_route_topk(logits: torch.Tensor, top_k: int, score_func: str = "sigmoid", renorm: bool = True,
                   route_scale: float = 1.0, bias: torch.Tensor | None = None):
    """logits [M, E] -> (ids int32 [M, k], weights f32 [M, k])."""
    logits = _cuda(logits, "logits").to(torch.float32)
    if logits.dim() != 2:
        raise ValueError(f"logits must be [M, E], got {tuple(logits.shape)}")
    m, e = logits.shape
    if bias is not None:
        bias = _cuda(bias, "bias").to(torch.float32)
        if tuple(bias.shape) != (e,):
            raise ValueError(f"bias shape {tuple(bias.shape)} != ({e},)")
    ids = torch.empty(m, top_k, dtype=torch.int32, device=logits.device)
    w = torch.empty(m, top_k, dtype=torch.float32, device=logits.device)
    _lib.call("mosaic_moe_route_topk", _ptr(logits), m, e, top_k, SCORE_FUNCS[score_func], int(renorm),
              float(route_scale), _ptr(bias), _ptr(ids), _ptr(w), _stream())
    return ids, w


def router_logits(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """logits [M, E] f32 = x [M, H] . w [E, H]^T (x, w each bf16 or f32), each
    logit the exact dot product rounded once to fp32."""
    x = _cuda(x, "x")
    w = _cuda(w, "weight")
    if x.dim() != 2 or w.dim() != 2 or x.shape[1] != w.shape[1]:
        raise ValueError(f"x {tuple(x.shape)} and weight {tuple(w.shape)} must be [M, H] and [E, H]")
    dt = {torch.bfloat16: DT_BF16, torch.float32: DT_F32}
    if x.dtype not in dt:
        x = x.to(torch.float32)
    if w.dtype not in dt:
        w = w.to(torch.float32)
    m, h = x.shape
    e = w.shape[0]
    out = torch.empty(m, e, dtype=torch.float32, device=x.device)
    _lib.call("mosaic_router_logits", _ptr(x), dt[x.dtype], _ptr(w), dt[w.dtype], _ptr(out), m, e, h, _stream())
    return out


def _tile_cap(a: int, e_ext: int, block_m: int) -> int:
    u = min(a, e_ext)
    return (a + u * (block_m - 1)) // block_m


def moe_layout(ids: torch.Tensor, weights: torch.Tensor | None, n_experts: int, has_shared: bool = False,
               block_m: int = 16) -> dict:
    """Stable expert sort + tile list of ids [M, k] (+ a shared-expert row per token)."""
    ids = _cuda(ids, "ids")
    if ids.dim() == 1:
        ids = ids.view(-1, 1)
    m, k = ids.shape
    ids32 = ids.to(torch.int32).contiguous()
    if weights is None:
        weights = torch.ones(m, k, dtype=torch.float32, device=ids.device)
    weights = _cuda(weights, "weights").to(torch.float32).reshape(m, k).contiguous()
    a = m * k + (m if has_shared else 0)
    e_ext = n_experts + (1 if has_shared else 0)
    cap = _tile_cap(a, e_ext, block_m)
    dev = ids.device
    i32 = dict(dtype=torch.int32, device=dev)
    out = dict(
        counts=torch.empty(e_ext, **i32), offsets=torch.empty(e_ext + 1, **i32), perm=torch.empty(a, **i32),
        perm_token=torch.empty(a, **i32), perm_weight=torch.empty(a, dtype=torch.float32, device=dev),
        sorted_ids=torch.empty(a, **i32), inv_pos=torch.empty(a, **i32),
        combine_pos=torch.empty(m, k + int(has_shared), **i32), tile_expert=torch.empty(max(cap, 1), **i32),
        tile_start=torch.empty(max(cap, 1), **i32), tile_rows=torch.empty(max(cap, 1), **i32),
        tile_p0=torch.empty(max(cap, 1), **i32), n_tiles=torch.empty(1, **i32))
    nbytes = _lib.lib().mosaic_moe_layout_workspace_bytes(m, k, n_experts, int(has_shared))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev) if nbytes else None
    _lib.call("mosaic_moe_layout", _ptr(ids32), _ptr(weights), m, k, n_experts, int(has_shared), block_m,
              _ptr(out["counts"]), _ptr(out["offsets"]), _ptr(out["perm"]), _ptr(out["perm_token"]),
              _ptr(out["perm_weight"]), _ptr(out["sorted_ids"]), _ptr(out["inv_pos"]), _ptr(out["combine_pos"]),
              _ptr(out["tile_expert"]), _ptr(out["tile_start"]), _ptr(out["tile_rows"]), _ptr(out["tile_p0"]),
              _ptr(out["n_tiles"]), cap, _ptr(ws), nbytes, _stream())
    out["tile_cap"] = cap
    return out


def emit_tiles(counts: torch.Tensor, block_m: int, tile_cap: int):
    """counts [E] -> (expert_index [cap], m_start [cap], n_tiles [1], tile_rows [cap])."""
    counts = _cuda(counts, "counts").to(torch.int32).contiguous()
    e = counts.numel()
    dev = counts.device
    cap = max(int(tile_cap), 1)
    ei = torch.empty(cap, dtype=torch.int32, device=dev)
    ms = torch.empty(cap, dtype=torch.int32, device=dev)
    rows = torch.empty(cap, dtype=torch.int32, device=dev)
    nt = torch.empty(1, dtype=torch.int32, device=dev)
    _lib.call("mosaic_emit_tiles", _ptr(counts), e, block_m, _ptr(ei), _ptr(ms), _ptr(rows), _ptr(nt), int(tile_cap),
              _stream())
    return ei, ms, nt, rows


# ---------------------------------------------------------- A16 MoE layer ---
class MoEWorkspace:
    """Reusable device workspace for the MoE / DSA / MLA wrappers.

    ``get`` returns a buffer of at least the requested bytes.  When a call needs
    more than the current buffer, a larger one is allocated and the old one is
    kept alive for the lifetime of this object, so a HIP graph captured earlier
    on the old pointer still owns valid memory.  One workspace serves one stream
    at a time; calls on different streams need different workspaces.  Without a
    workspace argument the wrappers allocate per call through torch's caching
    allocator, which is stream- and graph-safe."""

    def __init__(self):
        self.buf: torch.Tensor | None = None
        self._retired: list[torch.Tensor] = []

    def get(self, nbytes: int, device) -> torch.Tensor:
        if self.buf is None or self.buf.numel() < nbytes or self.buf.device != torch.device(device):
            if self.buf is not None:
                self._retired.append(self.buf)
            self.buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
        return self.buf


def _workspace(workspace: "MoEWorkspace | None", nbytes: int, device) -> torch.Tensor:
    if workspace is not None:
        return workspace.get(nbytes, device)
    return torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)


def moe_a16_forward(x: torch.Tensor, gate_up: MXT16, down: MXT16, **kw):
    """A16 routed MoE layer (+ optional shared expert) -> (y bf16 [M, H], ids, weights).

    ``gate_up``: MXT16 bank of [E, 2I, H/2] (gate rows then up rows per expert);
    ``down``: MXT16 bank of [E, H, I/2]; ``shared``: (gate_up, down) MXT16 of one
    expert or None.  Either ``logits`` [M, E] (the router runs on the device) or
    ``ids``/``weights`` [M, k] are given."""
    return _moe_forward(False, x, gate_up, down, **kw)


def moe_a8_forward(x: torch.Tensor, gate_up: MXT16, down: MXT16, **kw):
    """A8 routed MoE layer (fused_moe_mxint contract), same arguments as
    ``moe_a16_forward``; ``stage_events`` is a ``StageEvents(MOE_A8_STAGES)``."""
    return _moe_forward(True, x, gate_up, down, **kw)


def _moe_forward(a8: bool, x: torch.Tensor, gate_up: MXT16, down: MXT16, *, logits: torch.Tensor | None = None,
                 ids: torch.Tensor | None = None, weights: torch.Tensor | None = None, top_k: int | None = None,
                 shared: tuple[MXT16, MXT16] | None = None, score_func: str = "sigmoid", renorm: bool = True,
                 route_scale: float = 1.0, route_bias: torch.Tensor | None = None, swiglu_limit: float = 0.0,
                 workspace: MoEWorkspace | None = None, stage_events: "StageEvents | None" = None):
    x = _bf16(x, "x")
    if x.dim() != 2:
        raise ValueError(f"x must be [M, H], got {tuple(x.shape)}")
    m, h = x.shape
    if not isinstance(gate_up, MXT16) or not isinstance(down, MXT16):
        raise TypeError("gate_up/down must be MXT16 banks (ops.mxt16_prepack)")
    if len(gate_up.lead) != 1 or len(down.lead) != 1:
        raise ValueError("gate_up/down must be stacked [E, N, K/2] banks")
    e = gate_up.lead[0]
    inter = gate_up.n // 2
    if gate_up.k != h or gate_up.n % 2:
        raise ValueError(f"gate/up bank N={gate_up.n} K={gate_up.k} does not match hidden {h}")
    if down.lead != (e,) or down.n != h or down.k != inter:
        raise ValueError(f"down bank {down.lead}+[{down.n}, {down.k}] does not match [{e}, {h}, {inter}]")
    sh = [None] * 4
    if shared is not None:
        sgu, sd = shared
        if sgu.lead or sd.lead or (sgu.n, sgu.k) != (2 * inter, h) or (sd.n, sd.k) != (h, inter):
            raise ValueError("shared expert shapes do not match the routed bank")
        sh = [sgu.packed, sgu.scale, sd.packed, sd.scale]
    if logits is not None:
        logits = _cuda(logits, "logits").to(torch.float32)
        if tuple(logits.shape) != (m, e):
            raise ValueError(f"logits shape {tuple(logits.shape)} != ({m}, {e})")
        if top_k is None:
            raise ValueError("top_k is required with logits")
    if m == 0:  # an empty batch: empty outputs, nothing to launch
        if logits is None and (ids is None or weights is None):
            raise ValueError("give logits or ids and weights")
        k = top_k if logits is not None else (ids.shape[1] if ids.dim() == 2 else 0)
        return (torch.empty(0, h, dtype=torch.bfloat16, device=x.device),
                torch.empty(0, k, dtype=torch.int32, device=x.device),
                torch.empty(0, k, dtype=torch.float32, device=x.device))
    if logits is not None:
        ids = torch.empty(m, top_k, dtype=torch.int32, device=x.device)
        weights = torch.empty(m, top_k, dtype=torch.float32, device=x.device)
    else:
        if ids is None or weights is None:
            raise ValueError("give logits or ids and weights")
        ids = _cuda(ids, "ids")
        if ids.dim() == 1:
            ids = ids.view(m, -1)
        top_k = ids.shape[1]
        ids = ids.to(torch.int32).contiguous()
        weights = _cuda(weights, "weights").to(torch.float32).reshape(m, top_k).contiguous()
    if route_bias is not None:
        route_bias = _cuda(route_bias, "route_bias").to(torch.float32)
    has_shared = int(shared is not None)
    kind = "a8" if a8 else "a16"
    nbytes = getattr(_lib.lib(), f"mosaic_moe_{kind}_workspace_bytes")(m, h, inter, e, top_k, has_shared)
    ws = _workspace(workspace, nbytes, x.device)
    y = torch.empty(m, h, dtype=torch.bfloat16, device=x.device)
    args = [_ptr(x), _ptr(logits), _ptr(ids), _ptr(weights), _ptr(gate_up.packed), _ptr(gate_up.scale),
            _ptr(down.packed), _ptr(down.scale), _ptr(sh[0]), _ptr(sh[1]), _ptr(sh[2]), _ptr(sh[3]), _ptr(y), m, h,
            inter, e, top_k, SCORE_FUNCS[score_func], int(renorm), float(route_scale), _ptr(route_bias),
            float(swiglu_limit), _ptr(ws), ws.numel()]
    want = MOE_A8_STAGES if a8 else MOE_STAGES
    if stage_events is not None and stage_events.names != want:
        raise ValueError(f"stage_events must cover {want}")
    args.append(None if stage_events is None else stage_events.array)
    _lib.call(f"mosaic_moe_{kind}_forward", *args, _stream())
    return y, ids, weights


MOE_STAGES = ("layout_sec", "gu_sec", "down_sec", "reduction_sec")
MOE_A8_STAGES = ("layout_sec", "act_quant_sec", "gu_sec", "down_quant_sec", "down_sec", "reduction_sec")


class StageEvents:
    """HIP events recorded by the MoE forward at its stage boundaries; ``times()``
    returns seconds per stage like the reference's ``stage_times`` dict
    (``kernels/mxint.py:1702-1714``).  A16: start, after routing+layout, after
    gate/up+SwiGLU, after down, after combine (``MOE_STAGES``).  A8
    (``MOE_A8_STAGES``): start, after routing+layout, after the token
    act-quant, after gate/up+SwiGLU, after the z requant, after down, after
    combine."""

    def __init__(self, names: tuple = MOE_STAGES):
        self.names = tuple(names)
        self.events = [torch.cuda.Event(enable_timing=True) for _ in range(len(self.names) + 1)]
        for e in self.events:  # torch creates the underlying hipEvent on first record
            e.record()
        torch.cuda.current_stream().synchronize()
        self.array = (ctypes.c_void_p * len(self.events))(*[ctypes.c_void_p(e.cuda_event) for e in self.events])

    def times(self) -> dict:
        ev = self.events
        ev[-1].synchronize()
        out = {k: ev[i].elapsed_time(ev[i + 1]) / 1e3 for i, k in enumerate(self.names)}
        out["total_sec"] = sum(out[k] for k in self.names)
        return out


# ----------------------------------------------------------- DSA decode -----
def _f32(t: torch.Tensor, name: str) -> torch.Tensor:
    t = _cuda(t, name)
    if t.dtype != torch.float32:
        raise ValueError(f"{name}: expected float32, got {t.dtype}")
    return t


def _indexer_args(q, q_s, k, k_s, w):
    q, k = _u8(q, "q"), _u8(k, "k")
    q_s, k_s, w = _f32(q_s, "q_s"), _f32(k_s, "k_s"), _f32(w, "weights")
    if q.dim() != 3 or k.dim() != 3:
        raise ValueError(f"q must be [B, H, D] and k [B, L, D], got {tuple(q.shape)} and {tuple(k.shape)}")
    b, h, d = q.shape
    if k.shape[0] != b or k.shape[2] != d:
        raise ValueError(f"k shape {tuple(k.shape)} does not match q {tuple(q.shape)}")
    l_ = k.shape[1]
    if tuple(q_s.shape) != (b, h) or tuple(w.shape) != (b, h) or tuple(k_s.shape) != (b, l_):
        raise ValueError("q_s and weights must be [B, H], k_s [B, L]")
    return q, q_s, k, k_s, w, b, h, d, l_


def dsa_indexer_topk(q: torch.Tensor, q_s: torch.Tensor, k: torch.Tensor, k_s: torch.Tensor, w: torch.Tensor,
                     topk: int, lengths: torch.Tensor | None = None, offset: int = 0,
                     workspace: MoEWorkspace | None = None) -> torch.Tensor:
    """FP8 lightning indexer + exact top-k -> idx int32 [B, topk] (descending
    canonical score, ties to the lower index, + offset, -1 where fewer than
    topk tokens are valid)."""
    q, q_s, k, k_s, w, b, h, d, l_ = _indexer_args(q, q_s, k, k_s, w)
    if lengths is not None:
        lengths = _cuda(lengths, "lengths").to(torch.int32).contiguous()
        if tuple(lengths.shape) != (b,):
            raise ValueError(f"lengths must be [B], got {tuple(lengths.shape)}")
    idx = torch.empty(b, topk, dtype=torch.int32, device=q.device)
    nbytes = _lib.lib().mosaic_dsa_indexer_workspace_bytes(b, l_)
    ws = _workspace(workspace, nbytes, q.device)
    _lib.call("mosaic_dsa_indexer_topk", _ptr(q), _ptr(q_s), _ptr(k), _ptr(k_s), _ptr(w), _ptr(lengths), _ptr(idx),
              b, h, d, l_, int(topk), int(offset), _ptr(ws), ws.numel(), _stream())
    return idx


def dsa_indexer_topk_shared(q: torch.Tensor, q_s: torch.Tensor, k: torch.Tensor, k_s: torch.Tensor,
                            w: torch.Tensor, topk: int, lengths: torch.Tensor, offset: int = 0,
                            workspace: MoEWorkspace | None = None) -> torch.Tensor:
    """Indexer top-k for R query rows q [R, H, D] sharing key caches k [G, L, D]
    in groups of R / G consecutive rows, each row with its own length.  k and
    k_s may be the first L tokens of longer caches ([G, max_len, D] sliced
    along dim 1): they are read in place when both have unit inner strides and
    the same cache length (k.stride(0) / D == k_s.stride(0))."""
    q = _u8(q, "q")
    k = _on_device(k, "k")
    k = k.view(torch.uint8) if k.dtype in (torch.int8, torch.float8_e4m3fn) else k
    if k.dtype != torch.uint8:
        raise ValueError(f"k: expected e4m3 codes (uint8 / float8_e4m3fn), got {k.dtype}")
    k_s = _on_device(k_s, "k_s")
    if k_s.dtype != torch.float32:
        raise ValueError(f"k_s: expected float32, got {k_s.dtype}")
    q_s, w = _f32(q_s, "q_s"), _f32(w, "weights")
    strided = (k.dim() == 3 and k_s.dim() == 2 and k.stride(2) == 1 and k.stride(1) == k.shape[2] and
               k_s.stride(1) == 1 and k.stride(0) % k.shape[2] == 0 and k.stride(0) // k.shape[2] == k_s.stride(0)
               and k_s.stride(0) >= k_s.shape[1])
    if not strided:
        k, k_s = k.contiguous(), k_s.contiguous()
    if q.dim() != 3 or k.dim() != 3 or q.shape[2] != k.shape[2]:
        raise ValueError(f"q must be [R, H, D] and k [G, L, D], got {tuple(q.shape)} and {tuple(k.shape)}")
    r, h, d = q.shape
    g, l_, _ = k.shape
    if g == 0 or r % g:
        raise ValueError(f"{r} query rows do not split into {g} key caches")
    if tuple(q_s.shape) != (r, h) or tuple(w.shape) != (r, h) or tuple(k_s.shape) != (g, l_):
        raise ValueError("q_s and weights must be [R, H], k_s [G, L]")
    lengths = _cuda(lengths, "lengths").to(torch.int32).contiguous()
    if tuple(lengths.shape) != (r,):
        raise ValueError(f"lengths must be [R], got {tuple(lengths.shape)}")
    idx = torch.empty(r, topk, dtype=torch.int32, device=q.device)
    nbytes = _lib.lib().mosaic_dsa_indexer_workspace_bytes(r, l_)
    ws = _workspace(workspace, nbytes, q.device)
    cache_len = k_s.stride(0) if g > 1 else l_
    _lib.call("mosaic_dsa_indexer_topk_shared", _ptr(q), _ptr(q_s), _ptr(k), _ptr(k_s), _ptr(w), _ptr(lengths),
              _ptr(idx), r, h, d, l_, cache_len, r // g, int(topk), int(offset), _ptr(ws), ws.numel(), _stream())
    return idx


def dsa_indexer_scores(q, q_s, k, k_s, w) -> torch.Tensor:
    """The canonical indexer scores [B, L] f32."""
    q, q_s, k, k_s, w, b, h, d, l_ = _indexer_args(q, q_s, k, k_s, w)
    out = torch.empty(b, l_, dtype=torch.float32, device=q.device)
    _lib.call("mosaic_dsa_indexer_scores", _ptr(q), _ptr(q_s), _ptr(k), _ptr(k_s), _ptr(w), _ptr(out), b, h, d, l_,
              _stream())
    return out


def dsa_indexer_bounds(q, q_s, k, k_s, w) -> tuple[torch.Tensor, torch.Tensor]:
    """The bound stage: (lo, hi) [B, L] f32 enclosing every canonical score."""
    q, q_s, k, k_s, w, b, h, d, l_ = _indexer_args(q, q_s, k, k_s, w)
    lo = torch.empty(b, l_, dtype=torch.float32, device=q.device)
    hi = torch.empty_like(lo)
    _lib.call("mosaic_dsa_indexer_bounds", _ptr(q), _ptr(q_s), _ptr(k), _ptr(k_s), _ptr(w), _ptr(lo), _ptr(hi), b, h,
              d, l_, _stream())
    return lo, hi


def dsa_head_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, topk: int,
                       scale: float) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-head top-k attention of one token: q [H, d], k [ctx, H, d], v [ctx, H, dv]
    (bf16) -> (out [H, dv] bf16, idx [H, topk] int32)."""
    q, k, v = _bf16(q, "q"), _bf16(k, "k_index"), _bf16(v, "v_full")
    if q.dim() != 2 or k.dim() != 3 or v.dim() != 3:
        raise ValueError("q must be [H, d], k_index [ctx, H, d], v_full [ctx, H, dv]")
    h, d = q.shape
    ctx = k.shape[0]
    if tuple(k.shape) != (ctx, h, d) or v.shape[0] != ctx or v.shape[1] != h:
        raise ValueError(f"shapes q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)} do not agree")
    dv = v.shape[2]
    out = torch.empty(h, dv, dtype=torch.bfloat16, device=q.device)
    idx = torch.empty(h, topk, dtype=torch.int32, device=q.device)
    nbytes = _lib.lib().mosaic_dsa_head_attention_workspace_bytes(ctx, h)
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=q.device)
    _lib.call("mosaic_dsa_head_attention", _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(idx), h, ctx, d, dv, int(topk),
              float(scale), _ptr(ws), ws.numel(), _stream())
    return out, idx


def mla_sparse_decode(q: torch.Tensor, kv_latent: torch.Tensor, kv_scale: torch.Tensor, kv_rope: torch.Tensor,
                      idx: torch.Tensor, softmax_scale: float, sink: torch.Tensor | None = None,
                      workspace: MoEWorkspace | None = None) -> torch.Tensor:
    """MLA decode over selected entries: q [B, H, 576] bf16, kv_latent [B, N, 512]
    e4m3, kv_scale [B, N, 512/block] f32, kv_rope [B, N, 64] bf16, idx [B, T]
    int32 -> o [B, H, 512] bf16."""
    q, kv_rope = _bf16(q, "q"), _bf16(kv_rope, "kv_rope")
    kv_latent, kv_scale = _u8(kv_latent, "kv_latent"), _f32(kv_scale, "kv_scale")
    idx = _cuda(idx, "idx").to(torch.int32).contiguous()
    if q.dim() != 3 or kv_latent.dim() != 3 or kv_rope.dim() != 3 or kv_scale.dim() != 3 or idx.dim() != 2:
        raise ValueError("q/kv_latent/kv_scale/kv_rope must be 3-D and idx 2-D")
    b, h, dqk = q.shape
    n, dl = kv_latent.shape[1], kv_latent.shape[2]
    dr = kv_rope.shape[2]
    if dqk != dl + dr or kv_latent.shape[0] != b or tuple(kv_rope.shape[:2]) != (b, n) or \
            tuple(kv_scale.shape[:2]) != (b, n) or idx.shape[0] != b:
        raise ValueError("q / kv / idx shapes do not agree")
    if dl % kv_scale.shape[2]:
        raise ValueError(f"kv_scale last dim {kv_scale.shape[2]} does not divide {dl}")
    scale_block = dl // kv_scale.shape[2]
    if sink is not None:
        sink = _f32(sink, "sink")
        if tuple(sink.shape) != (h,):
            raise ValueError(f"sink must be [H], got {tuple(sink.shape)}")
    topk = idx.shape[1]
    out = torch.empty(b, h, dl, dtype=torch.bfloat16, device=q.device)
    nbytes = _lib.lib().mosaic_mla_decode_workspace_bytes(b, h, topk)
    ws = _workspace(workspace, nbytes, q.device)
    _lib.call("mosaic_mla_sparse_decode", _ptr(q), _ptr(kv_latent), _ptr(kv_scale), _ptr(kv_rope), _ptr(sink),
              _ptr(idx), _ptr(out), b, h, n, topk, dl, dr, scale_block, float(softmax_scale), _ptr(ws), ws.numel(),
              _stream())
    return out


def mla_sparse_decode_bf16(q: torch.Tensor, kv: torch.Tensor, idx: torch.Tensor, softmax_scale: float,
                           sink: torch.Tensor | None = None, workspace: MoEWorkspace | None = None) -> torch.Tensor:
    """Sparse attention over a bf16 KV: q [R, H, D] bf16, kv [B, N, D] bf16 with
    R a multiple of B (query row r reads kv[r // (R // B)]), idx [R, T] int32
    -> o [R, H, 512] bf16 with V = kv[..., :512]; D = 512 or 576."""
    q, kv = _bf16(q, "q"), _bf16(kv, "kv")
    idx = _cuda(idx, "idx").to(torch.int32).contiguous()
    if q.dim() != 3 or kv.dim() != 3 or idx.dim() != 2:
        raise ValueError("q and kv must be 3-D, idx 2-D")
    rows, h, d = q.shape
    nb, n, dk = kv.shape
    if dk != d or idx.shape[0] != rows or nb == 0 or rows % nb:
        raise ValueError(f"shapes q {tuple(q.shape)}, kv {tuple(kv.shape)}, idx {tuple(idx.shape)} do not agree")
    if sink is not None:
        sink = _f32(sink, "sink")
        if tuple(sink.shape) != (h,):
            raise ValueError(f"sink must be [H], got {tuple(sink.shape)}")
    topk = idx.shape[1]
    out = torch.empty(rows, h, 512, dtype=torch.bfloat16, device=q.device)
    nbytes = _lib.lib().mosaic_mla_decode_workspace_bytes(rows, h, topk)
    ws = _workspace(workspace, nbytes, q.device)
    _lib.call("mosaic_mla_sparse_decode_bf16", _ptr(q), _ptr(kv), _ptr(sink), _ptr(idx), _ptr(out), rows, h, n, topk,
              d, rows // nb, float(softmax_scale), _ptr(ws), ws.numel(), _stream())
    return out


def sparse_attn_bf16(q: torch.Tensor, kv: torch.Tensor, idx: torch.Tensor, softmax_scale: float,
                     sink: torch.Tensor | None = None) -> torch.Tensor:
    """Sparse attention with V = K at head dims 64, 128 and 256: q [R, H, D] bf16
    (H a multiple of 16), kv [B, N, D] bf16 with R a multiple of B (query row
    r reads kv[r // (R // B)]), idx [R, T] int32 (-1 masked) -> o [R, H, D] bf16."""
    q, kv = _bf16(q, "q"), _bf16(kv, "kv")
    idx = _cuda(idx, "idx").to(torch.int32).contiguous()
    if q.dim() != 3 or kv.dim() != 3 or idx.dim() != 2:
        raise ValueError("q and kv must be 3-D, idx 2-D")
    rows, h, d = q.shape
    nb, n, dk = kv.shape
    if dk != d or idx.shape[0] != rows or nb == 0 or rows % nb:
        raise ValueError(f"shapes q {tuple(q.shape)}, kv {tuple(kv.shape)}, idx {tuple(idx.shape)} do not agree")
    if sink is not None:
        sink = _f32(sink, "sink")
        if tuple(sink.shape) != (h,):
            raise ValueError(f"sink must be [H], got {tuple(sink.shape)}")
    out = torch.empty(rows, h, d, dtype=torch.bfloat16, device=q.device)
    _lib.call("mosaic_sparse_attn_bf16", _ptr(q), _ptr(kv), _ptr(sink), _ptr(idx), _ptr(out), rows, h, n,
              idx.shape[1], d, rows // nb, float(softmax_scale), _stream())
    return out


def dsa_kv_write(kv: torch.Tensor, cache, slots: torch.Tensor | None = None, rope: int = 64) -> None:
    """Write kv rows [R, D] bf16 into a DSA cache with act_quant_sim on the
    first D - rope dims: ``cache`` is either a bf16 tensor [N, D] (the
    reference's cache) or (codes [N, D - rope] e4m3/uint8, scales [N, (D -
    rope) / 64] fp32, rope [N, rope] bf16), the FP8 cache ``mla_sparse_decode``
    reads.  Row r goes to cache row ``slots[r]`` (default r); slots outside
    [0, N) skip the row."""
    kv = _bf16(kv, "kv").contiguous()
    if kv.dim() != 2:
        raise ValueError(f"kv must be [R, D], got {tuple(kv.shape)}")
    rows, d = kv.shape
    if slots is not None:
        slots = _cuda(slots, "slots").to(torch.int32).contiguous()
        if tuple(slots.shape) != (rows,):
            raise ValueError(f"slots must be [{rows}], got {tuple(slots.shape)}")
    if isinstance(cache, torch.Tensor):
        cache = _bf16(cache, "cache")
        if cache.dim() != 2 or cache.shape[1] != d or not cache.is_contiguous():
            raise ValueError(f"bf16 cache must be a contiguous [N, {d}], got {tuple(cache.shape)}")
        n = cache.shape[0]
        _lib.call("mosaic_dsa_kv_write", _ptr(kv), _ptr(slots), rows, d, rope, n, _ptr(cache), None, None, None,
                  _stream())
        return
    codes, scales, rope_c = cache
    codes = _u8(codes, "codes")
    scales = _f32(scales, "scales")
    rope_c = _bf16(rope_c, "rope")
    n = codes.shape[0]
    dn = d - rope
    if tuple(codes.shape) != (n, dn) or tuple(scales.shape) != (n, dn // 64) or tuple(rope_c.shape) != (n, rope) \
            or not (codes.is_contiguous() and scales.is_contiguous() and rope_c.is_contiguous()):
        raise ValueError(f"fp8 cache must be contiguous [N, {dn}] codes, [N, {dn // 64}] scales, [N, {rope}] rope")
    _lib.call("mosaic_dsa_kv_write", _ptr(kv), _ptr(slots), rows, d, rope, n, None, _ptr(codes), _ptr(scales),
              _ptr(rope_c), _stream())


def dsa_decode_indices(pos: torch.Tensor, window: int, cidx: torch.Tensor | None = None, nc: int | None = None,
                       ratio: int = 4, offset: int | None = None) -> torch.Tensor:
    """Gather indices of one decode step: pos [R] int32 absolute positions ->
    [R, window + nc] int32 = the window ring slots of the last ``window``
    positions (oldest first, -1 padded), then the indexer picks ``cidx`` [R, nc]
    (already offset) or, without them, the static compressed list ``offset`` ..
    ``offset + (p + 1) // ratio - 1`` padded with -1 to ``nc`` entries
    (``offset`` defaults to ``window``)."""
    pos = _cuda(pos, "pos").to(torch.int32).contiguous()
    rows = pos.shape[0]
    if cidx is not None:
        cidx = _cuda(cidx, "cidx").to(torch.int32).contiguous()
        if cidx.dim() != 2 or cidx.shape[0] != rows:
            raise ValueError(f"cidx must be [{rows}, nc], got {tuple(cidx.shape)}")
        nc = cidx.shape[1]
    nc = 0 if nc is None else int(nc)
    offset = window if offset is None else int(offset)
    out = torch.empty(rows, window + nc, dtype=torch.int32, device=pos.device)
    _lib.call("mosaic_dsa_decode_indices", _ptr(pos), rows, window, _ptr(cidx), nc, ratio, offset, _ptr(out),
              _stream())
    return out

