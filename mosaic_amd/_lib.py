"""ctypes binding of ``libmosaic_amd.so`` (the C ABI in ``include/mosaic_amd.h``).

The library is loaded from ``mosaic_amd/_lib/`` (built in-tree by
``mosaic_amd.build``).  There is no fallback: a missing library, a missing
symbol or a non-zero status raises.
"""
from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_int64, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libmosaic_amd.so"

P = c_void_p
I64 = c_int64
I = c_int
F = c_float

# name -> (restype, argtypes); mirrors include/mosaic_amd.h
SIGNATURES: dict[str, tuple] = {
    "mosaic_version": (c_int, []),
    "mosaic_last_error": (ctypes.c_char_p, []),
    "mosaic_launch_count": (ctypes.c_uint64, []),
    "mosaic_mx_quantize": (c_int, [P, I, P, P, I64, I64, I, P]),
    "mosaic_mx_dequant": (c_int, [P, P, P, I, I64, I64, P]),
    "mosaic_act_quant": (c_int, [P, I, P, P, I64, I64, I, I, P]),
    "mosaic_e4m3_decode": (c_int, [P, P, I64, P]),
    "mosaic_e4m3_encode": (c_int, [P, P, I64, P]),
    "mosaic_selfcheck_converters": (c_int, [P, P]),
    "mosaic_mx_linear_a16": (c_int, [P, P, P, P, I64, I64, I64, P]),
    "mosaic_mx_kn_linear_a16_workspace_bytes": (c_size_t, [I64, I64, I64]),
    "mosaic_mx_kn_linear_a16": (c_int, [P, P, P, P, I64, I64, I64, P, c_size_t, P]),
    "mosaic_mxt16_prepack": (c_int, [P, P, P, P, I64, I64, P]),
    "mosaic_mxt16_unpack": (c_int, [P, P, P, P, I64, I64, P]),
    "mosaic_mxt16_linear_a16": (c_int, [P, P, P, P, I64, I64, I64, P]),
    "mosaic_fp8_block_gemm": (c_int, [P, P, P, P, P, I, I64, I64, I64, P]),
    "mosaic_fp8_block_gemm_workspace_bytes": (c_size_t, [I64, I64, I64]),
    "mosaic_fp8_block_gemm_ws": (c_int, [P, P, P, P, P, I, I64, I64, I64, P, c_size_t, P]),
    "mosaic_fp8_t16_prepack": (c_int, [P, P, I64, I64, P]),
    "mosaic_fp8_t16_unpack": (c_int, [P, P, I64, I64, P]),
    "mosaic_fp8_block_gemm_t16_workspace_bytes": (c_size_t, [I64, I64, I64]),
    "mosaic_fp8_block_gemm_t16": (c_int, [P, P, P, P, P, I, I64, I64, I64, P, c_size_t, P]),
    "mosaic_mxt16_linear_a8": (c_int, [P, P, P, P, P, I64, I64, I64, P]),
    "mosaic_mxt16_linear_a8_workspace_bytes": (c_size_t, [I64, I64, I64]),
    "mosaic_mxt16_linear_a8_ws": (c_int, [P, P, P, P, P, I64, I64, I64, P, c_size_t, P]),
    "mosaic_fp8_block_dequant": (c_int, [P, P, P, I64, I64, I, I, P]),
    "mosaic_fp8_w8a16_linear": (c_int, [P, P, P, P, I64, I64, I64, P]),
    "mosaic_fp8_w8a16_workspace_bytes": (c_size_t, [I64, I64, I64]),
    "mosaic_fp8_w8a16_linear_ws": (c_int, [P, P, P, P, I64, I64, I64, P, c_size_t, P]),
    "mosaic_moe_route_topk": (c_int, [P, I64, I64, I64, I, I, F, P, P, P, P]),
    "mosaic_router_logits": (c_int, [P, I, P, I, P, I64, I64, I64, P]),
    "mosaic_moe_layout_workspace_bytes": (c_size_t, [I64, I64, I64, I]),
    "mosaic_moe_layout": (c_int, [P, P, I64, I64, I64, I, I, P, P, P, P, P, P, P, P, P, P, P, P, P, I64, P, c_size_t,
                                  P]),
    "mosaic_emit_tiles": (c_int, [P, I64, I, P, P, P, P, I64, P]),
    "mosaic_moe_a16_workspace_bytes": (c_size_t, [I64, I64, I64, I64, I64, I]),
    "mosaic_moe_a8_workspace_bytes": (c_size_t, [I64, I64, I64, I64, I64, I]),
    "mosaic_moe_a8_forward": (c_int, [P, P, P, P, P, P, P, P, P, P, P, P, P, I64, I64, I64, I64, I64, I, I, F, P, F,
                                      P, c_size_t, P, P]),
    "mosaic_moe_a16_forward": (c_int, [P, P, P, P, P, P, P, P, P, P, P, P, P, I64, I64, I64, I64, I64, I, I, F, P, F,
                                       P, c_size_t, P, P]),
    "mosaic_moe_a16_noalloc_max_bytes": (c_size_t, []),
    "mosaic_moe_a16_forward_noalloc": (c_int, [P, P, P, P, P, P, P, P, P, P, P, P, P, I64, I64, I64, I64, I64, I, I, F,
                                               P, F, P]),
    "mosaic_moe_skinny_workspace_bytes": (c_size_t, [I64, I64, I64, I64, I64]),
    "mosaic_moe_skinny_forward": (c_int, [P, P, P, P, P, P, P, P, I64, I64, I64, I64, I64, P, c_size_t, P]),
    "mosaic_dsa_indexer_workspace_bytes": (c_size_t, [I64, I64]),
    "mosaic_dsa_indexer_topk": (c_int, [P, P, P, P, P, P, P, I64, I64, I64, I64, I64, ctypes.c_int32, P, c_size_t,
                                        P]),
    "mosaic_dsa_indexer_topk_shared": (c_int, [P, P, P, P, P, P, P, I64, I64, I64, I64, I64, I64, I64,
                                               ctypes.c_int32, P, c_size_t, P]),
    "mosaic_sparse_attn_bf16": (c_int, [P, P, P, P, P, I64, I64, I64, I64, I64, I64, F, P]),
    "mosaic_dsa_indexer_scores": (c_int, [P, P, P, P, P, P, I64, I64, I64, I64, P]),
    "mosaic_dsa_indexer_bounds": (c_int, [P, P, P, P, P, P, P, I64, I64, I64, I64, P]),
    "mosaic_dsa_head_attention_workspace_bytes": (c_size_t, [I64, I64]),
    "mosaic_dsa_head_attention": (c_int, [P, P, P, P, P, I64, I64, I64, I64, I64, F, P, c_size_t, P]),
    "mosaic_mla_decode_workspace_bytes": (c_size_t, [I64, I64, I64]),
    "mosaic_mla_sparse_decode": (c_int, [P, P, P, P, P, P, P, I64, I64, I64, I64, I64, I64, I64, F, P, c_size_t,
                                         P]),
    "mosaic_mla_sparse_decode_bf16": (c_int, [P, P, P, P, P, I64, I64, I64, I64, I64, I64, F, P, c_size_t, P]),
    "mosaic_dsa_kv_write": (c_int, [P, P, I64, I64, I64, I64, P, P, P, P, P]),
    "mosaic_dsa_decode_indices": (c_int, [P, I64, I64, P, I64, I64, I64, P, P]),
    "mosaic_rmsnorm_act_quant": (c_int, [P, P, F, I64, I64, P, P, P, c_int, P]),
    "mosaic_swiglu_act_quant": (c_int, [P, P, I64, I64, F, P, P, P]),
    "mosaic_routed_reduce": (c_int, [P, P, P, P, I64, I64, I64, I64, P]),
}

_LIB = None


class MosaicError(RuntimeError):
    """A C-ABI call returned a non-zero status."""


def lib():
    """Load the library once; raise if it has not been built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"mosaic_amd HIP library not built ({LIB_PATH} missing); run `python -m mosaic_amd.build`")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)  # AttributeError names a missing export
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def exported_symbols() -> list[str]:
    return list(SIGNATURES)


def call(name: str, *args) -> None:
    """Call ``name`` and raise ``ValueError`` (status < 0) or ``MosaicError``."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().mosaic_last_error().decode(errors="replace")
        if rc < 0:
            raise ValueError(f"{name}: {msg}")
        raise MosaicError(f"{name} failed (status {rc}): {msg}")
