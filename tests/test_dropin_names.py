"""The drop-in modules export the reference's operator names for the path (CPU only: names
and signatures, no GPU calls).  Reference modules: ``mosaicvm/kernels/{mxint,qpa_mma,xsimt,
exact_moe,moe_layout,w4a16_grouped,mxfp4,fp4_source,skinny_fp4,dsa_sparse,dsa_attention}.py``,
``mosaicvm/model/layers.py`` and upstream ``.mosaicvm/source/inference_kernel.py``."""
from __future__ import annotations

import importlib
import inspect

import pytest

NAMES = {
    "mosaic_amd.kernels.mxint": ["fused_moe_mxint", "mxint_dp4a_gemm", "mxint_imma_gemm",
                                 "prepack_expert_bank_mxint", "prepack_expert_bank_mxint_packed4",
                                 "mxint_swiglu_quant_down", "mxint_routed_reduce", "last_launch_count"],
    "mosaic_amd.kernels.qpa_mma": ["qpa_mma_gemm", "fused_moe_qpa", "prepack_qpa", "inverse_prepack_qpa",
                                   "prepack_expert_bank_qpa", "launch_census", "last_launch_count"],
    "mosaic_amd.kernels.xsimt": ["xsimt_gemm", "prepack_xsimt", "inverse_prepack_xsimt", "prepack_expert_bank",
                                 "decode_activation_exact", "last_launch_count"],
    "mosaic_amd.kernels.exact_moe": ["exact_moe", "exact_moe_mxint", "exact_target"],
    "mosaic_amd.kernels.moe_layout": ["layout_assignments"],
    "mosaic_amd.kernels.w4a16_grouped": ["emit_tiles", "last_launch_count"],
    "mosaic_amd.kernels.mxfp4": ["pack_mxfp4", "dequant_mxfp4", "quantize_mxfp4"],
    "mosaic_amd.kernels.fp4_source": ["pack_mxfp4_nk", "e8m0_to_fp32", "decode_e2m1_nk", "decode_e4m3",
                                      "act_quant_ref", "act_quant_legacy_phase27",
                                      "reference_fp4_linear_source_semantics"],
    "mosaic_amd.kernels.skinny_fp4": ["skinny_mxfp4_gemm", "fused_moe_skinny", "pack_gate_up_mxfp4",
                                      "last_launch_count"],
    "mosaic_amd.kernels.fp8": ["act_quant", "fp8_gemm", "fp4_gemm", "w8a8_block_fp8_matmul", "fp8_act_quant",
                               "dequant_fp8", "fp8_linear"],
    "mosaic_amd.kernels.dsa": ["sparse_attn", "sparse_attn_fused", "Indexer", "dsa_decode_attention",
                               "DecodeKVCache", "indexer_topk", "indexer_scores", "mla_decode_fp8"],
    "mosaic_amd.layers": ["Router", "Gate", "grouped_expert_forward"],
    "mosaic_amd.loader": ["ShardIndex", "load_expert_bank", "validate_expert_tensors", "read_expert"],
}


@pytest.mark.parametrize("module", sorted(NAMES))
def test_dropin_module_exports(module):
    mod = importlib.import_module(module)
    missing = [n for n in NAMES[module] if not hasattr(mod, n)]
    assert not missing, f"{module} lacks {missing}"


def test_reference_argument_names():
    """The positional argument names of the most-used operators are the reference's."""
    from mosaic_amd.kernels import mxint, qpa_mma, skinny_fp4, xsimt
    from mosaic_amd.kernels.w4a16_grouped import emit_tiles
    want = {
        mxint.fused_moe_mxint: ["x", "expert_ids", "expert_weights", "packed_gate_up", "scale_gate_up",
                                "packed_down", "scale_down"],
        qpa_mma.fused_moe_qpa: ["x", "expert_ids", "expert_weights", "packed_gate_up", "scale_gate_up",
                                "packed_down", "scale_down"],
        skinny_fp4.fused_moe_skinny: ["x", "expert_ids", "expert_weights", "packed_gate_up", "scale_gate_up",
                                      "packed_down", "scale_down"],
        xsimt.xsimt_gemm: ["x", "packed", "scale_w", "n_out"],
        mxint.mxint_swiglu_quant_down: ["gu", "w_a", "inter", "swiglu_limit"],
        mxint.mxint_routed_reduce: ["yd", "slot_rows", "order", "h"],
        emit_tiles: ["counts", "block_m", "max_tiles"],
    }
    for fn, names in want.items():
        got = list(inspect.signature(fn).parameters)[:len(names)]
        assert got == names, f"{fn.__name__}: {got} != {names}"
