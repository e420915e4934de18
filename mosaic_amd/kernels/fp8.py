"""FP8 / FP4 GEMM operators with the upstream signatures
(``.mosaicvm/source/inference_kernel.py``: act_quant, fp8_gemm, fp4_gemm;
``.mosaicvm/source/hubkernel_matmul.py`` / ``hubkernel_act_quant.py``:
w8a8_block_fp8_matmul, fp8_act_quant; ``bench/fp8_core.py``: fp8_linear;
``runtime/fp8.py``: dequant_fp8)."""
from __future__ import annotations

import torch

from .. import ops
from . import _prepack_cache
from .fp4_source import e8m0_to_fp32


def _scales_f32(s: torch.Tensor) -> torch.Tensor:
    return e8m0_to_fp32(s) if s.dtype == torch.float8_e8m0fnu else s.to(torch.float32)


def act_quant(x: torch.Tensor, block_size: int = 128, scale_fmt: str | None = None,
              scale_dtype: torch.dtype = torch.float32, inplace: bool = False):
    """Block-wise e4m3 quantization (``inference_kernel.py:105-125``): pow2 scales
    when ``scale_fmt`` is set, else amax/448 (amax >= 1e-4); ``inplace`` writes
    the quant-dequant values back into x."""
    n = x.size(-1)
    if n % block_size:
        raise ValueError(f"last dim {n} must be a multiple of {block_size}")
    if scale_dtype == torch.float8_e8m0fnu and scale_fmt is None:
        raise ValueError("e8m0 scales need scale_fmt (power-of-two scales)")
    z = x.reshape(-1, n)
    q, s = ops.act_quant(z, block_size, "pow2" if scale_fmt is not None else "amax")
    if inplace:
        deq = (ops.e4m3_decode(q).view(-1, n // block_size, block_size) * s[..., None]).reshape(z.shape)
        x.copy_(deq.reshape(x.shape).to(x.dtype))
        return x
    s = s.reshape(*x.shape[:-1], n // block_size)
    if scale_dtype == torch.float8_e8m0fnu:
        s = ((s.view(torch.int32) >> 23) & 0xFF).to(torch.uint8).view(torch.float8_e8m0fnu)
    return q.reshape(x.shape), s


def _decode_weight(b: torch.Tensor, m: int):
    """The cached T16 prepack of ``b`` for calls of up to 64 rows (N % 16 == 0), whose
    kernels then read each 1 KB of weight contiguously; ``b`` itself otherwise.
    The prepack is one more copy of the weight, held while ``b`` lives unmodified."""
    if (m <= ops.FP8_T16_MAX_M and b.dim() == 2 and b.size(0) % 16 == 0 and b.size(1) % 128 == 0
            and b.size(1) > 0 and b.is_contiguous() and b.size(0) * b.size(1) < 2 ** 31):
        return _prepack_cache.fp8_t16(b)
    return b


def fp8_gemm(a: torch.Tensor, a_s: torch.Tensor, b: torch.Tensor, b_s: torch.Tensor,
             scale_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """C[M, N] = A[M, K] @ B[N, K]^T with per-128 block scales (``inference_kernel.py:257-273``).
    At M <= 64 the weight's T16 prepack is cached and read instead (at M <= 16 the same C bit for bit)."""
    k = a.size(-1)
    m = a.numel() // k
    n = b.size(0)
    out = torch.get_default_dtype()
    c = ops.fp8_block_gemm(a.reshape(m, k), _scales_f32(a_s).reshape(m, -1), _decode_weight(b, m), _scales_f32(b_s),
                           out_dtype=torch.bfloat16 if out == torch.bfloat16 else torch.float32)
    return c.reshape(*a.shape[:-1], n).to(out)


def fp4_gemm(a: torch.Tensor, a_s: torch.Tensor, b: torch.Tensor, b_s: torch.Tensor,
             scale_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """C = A_fp8[M, K] @ B_fp4[N, K]^T, per-128 act scale, e8m0 per-32 weight scale
    (``inference_kernel.py:518-536``).  The act scales must be powers of two
    (act_quant with scale_fmt; e8m0 scales always are), which the scaled MFMA
    consumes directly.  The kernel checks them on the device: a row whose
    scale is not a positive power of two comes out NaN (no host sync here).
    The weight's MXT16 prepack is cached while ``b``/``b_s`` stay alive and
    unmodified."""
    k = a.size(-1)
    m = a.numel() // k
    sa = _scales_f32(a_s).reshape(m, -1).contiguous()
    w = _prepack_cache.mxt16(b, b_s)
    c = ops.mxt16_linear_a8(None, w, prequant=(a.reshape(m, k), sa))
    return c.reshape(*a.shape[:-1], b.size(0)).to(torch.get_default_dtype())


def w8a8_block_fp8_matmul(A: torch.Tensor, B: torch.Tensor, As: torch.Tensor, Bs: torch.Tensor,
                          block_size: list[int], output_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """``hubkernel_matmul.py:333-360``: C = A @ B.T with [M, K/128] and [N/128, K/128] scales
    (the weight's cached T16 prepack at M <= 64, as in ``fp8_gemm``)."""
    if list(block_size) != [128, 128]:
        raise ValueError(f"block_size {block_size}: only [128, 128] is supported")
    k = A.size(-1)
    m = A.numel() // k
    c = ops.fp8_block_gemm(A.reshape(m, k), As.reshape(m, -1), _decode_weight(B, m), Bs,
                           out_dtype=torch.float32 if output_dtype == torch.float32 else torch.bfloat16)
    return c.reshape(*A.shape[:-1], B.size(0)).to(output_dtype)


def fp8_act_quant(x: torch.Tensor, block_size: int = 128):
    """HF ``fp8_act_quant`` (``hubkernel_act_quant.py:27-35``): s = amax / 448."""
    n = x.size(-1)
    q, s = ops.act_quant(x.reshape(-1, n), block_size, "hf")
    return q.reshape(x.shape), s.reshape(*x.shape[:-1], n // block_size)


def dequant_fp8(weight: torch.Tensor, scale: torch.Tensor, block: int = 128) -> torch.Tensor:
    """e4m3 weight with per-block scales -> bf16 (``runtime/fp8.py:52-64``)."""
    w = weight.reshape(weight.shape[0], -1)
    n, k = w.shape
    s = _scales_f32(scale)
    if s.dim() == 2 and n % s.shape[0] == 0 and k % s.shape[1] == 0:
        return ops.fp8_block_dequant(w, s, (n // s.shape[0], k // s.shape[1]))
    raise ValueError(f"scale {tuple(scale.shape)} does not tile the weight {tuple(w.shape)}")


def fp8_linear(x: torch.Tensor, w_fp8: torch.Tensor, s: torch.Tensor, out: torch.Tensor | None = None):
    """W8A16 ``F.linear(x, decode(w, s))`` (``bench/fp8_core.py:198-231``) with the
    reference's width dispatch: up to 80 rows the e4m3 weight is decoded inside
    the GEMM (``mosaic_fp8_w8a16_linear``: per 128-K block, x . decode(w)^T
    times the block scale added to an fp32 accumulator); above 80 rows it is
    dequantized once by the HIP kernel and multiplied by the library GEMM, as
    the reference does (dequant + cuBLAS there, hipBLASLt here)."""
    x = ops._bf16(x, "x")
    m = x.shape[0]
    if m <= ops.W8A16_MAX_M:
        y = ops.fp8_w8a16_linear(x, w_fp8, _scales_f32(s))
    else:
        y = torch.nn.functional.linear(x, dequant_fp8(w_fp8, s))
    if out is not None:
        out.copy_(y)
        return out
    return y
