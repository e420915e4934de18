/*
 * mosaic_amd -- C ABI of the MI355X (gfx950) quantized-weight matrix path.
 *
 * Conventions (every entry point):
 *   - returns int status: 0 OK, < 0 invalid argument (message in
 *     mosaic_last_error()), > 0 the hipError_t of a failed launch;
 *   - every pointer is a device pointer owned by the caller (the library never
 *     allocates); shapes are int64_t; `stream` is a hipStream_t (NULL = the
 *     default stream) and work is only enqueued, never synchronized;
 *   - bf16 tensors are passed as raw 16-bit words, e8m0 scales and e4m3 codes
 *     as raw bytes, MXFP4 weights as packed bytes [N, K/2] with the low nibble
 *     holding the even K element and one e8m0 byte per 32 K ([N, K/32]).
 *
 * Each declaration names the reference operator it replaces (paths relative
 * to the reference repository root).
 */
#ifndef MOSAIC_AMD_H
#define MOSAIC_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOSAIC_AMD_ABI_VERSION 1

/* dtype codes */
#define MOSAIC_DTYPE_F32 0
#define MOSAIC_DTYPE_BF16 1

/* router score functions (model/layers.py:110-115, .mosaicvm/source/inference_model.py:572-577) */
#define MOSAIC_SCORE_SIGMOID 0
#define MOSAIC_SCORE_SOFTMAX 1
#define MOSAIC_SCORE_SQRTSOFTPLUS 2

/* ------------------------------------------------------------ runtime ---- */
int mosaic_version(void);
/* Thread-local text of the last non-zero status. */
const char* mosaic_last_error(void);
/* Kernel launches this library has made on the calling thread since the
 * process started.  Backs the reference's per-module last_launch_count()
 * (kernels/skinny_fp4.py:17-22, kernels/mxint.py:33-34,
 * kernels/qpa_mma.py:58-59, kernels/xsimt.py:31-32,
 * kernels/w4a16_grouped.py:15-16), which count the launches of a module's
 * operators since its MoE entry point last reset them. */
uint64_t mosaic_launch_count(void);

/* ------------------------------------------------------------- codecs ---- */
/* MXFP4 quantizer, NK layout: w [n, k] (f32 or bf16) -> packed [n, k/2] + e8m0 [n, k/32].
 * recipe 0 = "ceil" (scale 2^ceil(log2(amax/6)); upstream fp4_quant_kernel,
 *   .mosaicvm/source/inference_kernel.py:128-183), recipe 1 = "floor"
 *   (kernels/fp4_source.py:35-64 pack_mxfp4_nk fallback). */
int mosaic_mx_quantize(const void* w, int w_dtype, uint8_t* packed, uint8_t* scale, int64_t n, int64_t k,
                       int recipe, void* stream);

/* MXFP4 dequant, NK layout -> out [n, k] f32 or bf16.
 * Replaces dequant_mxfp4 (kernels/mxfp4.py:130-160) and the decode kernels
 * decode_e2m1_* (kernels/mxfp4_decode.py:132-223). */
int mosaic_mx_dequant(const uint8_t* packed, const uint8_t* scale, void* out, int out_dtype, int64_t n, int64_t k,
                      void* stream);

/* 1 x block E4M3 activation quantizer: x [m, k] (f32/bf16) -> codes [m, k] + f32 scales [m, k/block].
 * mode 0: power-of-two scale, act_quant_ref (kernels/fp4_source.py:110-129);
 * mode 1: s = max(amax,1e-4)/448, upstream act_quant (.mosaicvm/source/inference_kernel.py:40-125);
 * mode 2: s = amax/448, fp8_act_quant (.mosaicvm/source/hubkernel_act_quant.py:27-35);
 * mode 3: s = amax/448 and 1 for an all-zero block, act_quant_legacy_phase27
 *         (kernels/fp4_source.py:94-107). */
int mosaic_act_quant(const void* x, int x_dtype, uint8_t* q, float* s, int64_t m, int64_t k, int block, int mode,
                     void* stream);

/* E4M3 byte <-> f32 (decode_e4m3 kernels/fp4_source.py:87-91, decode_e4m3_all
 * kernels/mxfp4_decode.py:243; encoder = torch's float8_e4m3fn cast, RNE). */
int mosaic_e4m3_decode(const uint8_t* in, float* out, int64_t n, void* stream);
int mosaic_e4m3_encode(const float* in, uint8_t* out, int64_t n, void* stream);

/* Self-check with no counterpart in the reference: compares gfx950's bf16 and
 * e4m3 converters, which the fused prefill epilogues use, with the library's
 * software roundings over every fp32 input.  counts (2 x uint64, zeroed by the
 * caller) receives the mismatches: [0] bf16 over all non-NaN inputs, [1] e4m3
 * over all inputs after the clamp to [-448, 448].  Both must stay 0. */
int mosaic_selfcheck_converters(unsigned long long* counts, void* stream);

/* ------------------------------------------------------ A16 MXFP4 linear -- */
/* y [m, n] bf16 = x [m, k] bf16 . dequant(W)^T, fp32 accumulation, NK layout.
 * Replaces the A16 "dequant-then-matmul" linear: skinny_mxfp4_gemm semantics
 * (kernels/skinny_fp4.py:113-144) on the checkpoint NK layout. k % 128 == 0. */
int mosaic_mx_linear_a16(const uint16_t* x, const uint8_t* packed, const uint8_t* scale, uint16_t* y, int64_t m,
                         int64_t n, int64_t k, void* stream);

/* A16 MXFP4 linear on the reference's KN layout (skinny_mxfp4_gemm,
 * kernels/skinny_fp4.py:113-144): y [m, n] bf16 = x [m, k] bf16 . W with
 * W [k, n] = E2M1(packed [k, n/2], low nibble = even n) * 2^(scale [k, n/32] - 127),
 * fp32 accumulation.  n % 32 == 0, k % 32 == 0.  K is split over workgroups
 * when the columns alone would not fill the GPU; the fp32 partials then need
 * mosaic_mx_kn_linear_a16_workspace_bytes(m, n, k) bytes of workspace and are
 * summed in a fixed order. */
size_t mosaic_mx_kn_linear_a16_workspace_bytes(int64_t m, int64_t n, int64_t k);
int mosaic_mx_kn_linear_a16(const uint16_t* x, const uint8_t* packed, const uint8_t* scale, uint16_t* y, int64_t m,
                            int64_t n, int64_t k, void* workspace, size_t workspace_bytes, void* stream);

/* MXT16 prepack: bit-exact permutation of an NK MXFP4 matrix (n % 16 == 0,
 * k % 128 == 0) into the 16-row MFMA tile order read by the A16 kernels:
 *   packed_t[g][S][l][16 B] = packed[16g + l%16][16*(4S + l/16) .. +16]
 *   scale_t [g][S4][l][s]   = scale[16g + l%16][4*(4*S4 + s) + l/16]  (0 past k)
 * (g = 16-row group, S = 128-K super-step, S4 = 4 super-steps, l = lane 0..63).
 * packed_t has n*k/2 bytes, scale_t n/16 * ceil(k/512) * 256 bytes.
 * Replaces the reference's bit-exact invertible bank prepacks (prepack_qpa /
 * prepack_expert_bank_mxint*, kernels/qpa_mma.py:90-150, kernels/mxint.py:165-285);
 * mosaic_mxt16_unpack is the inverse. */
int mosaic_mxt16_prepack(const uint8_t* packed, const uint8_t* scale, uint8_t* packed_t, uint8_t* scale_t, int64_t n,
                         int64_t k, void* stream);
int mosaic_mxt16_unpack(const uint8_t* packed_t, const uint8_t* scale_t, uint8_t* packed, uint8_t* scale, int64_t n,
                        int64_t k, void* stream);

/* A16 linear on an MXT16-prepacked weight (same contract as mosaic_mx_linear_a16). */
int mosaic_mxt16_linear_a16(const uint16_t* x, const uint8_t* packed_t, const uint8_t* scale_t, uint16_t* y,
                            int64_t m, int64_t n, int64_t k, void* stream);

/* A8 MXFP4 linear ("source semantics"): y [m, n] bf16 = sum over K32 groups of
 * (A_g . W_g^T) * sa[:, g/4] * sw[:, g] with xq e4m3 [m, k] and power-of-two
 * f32 scales sa [m, k/128] (mosaic_act_quant mode 0), W an MXT16-prepacked
 * MXFP4 weight [n, k]; fp32 accumulation on the scaled MFMA.  Checked on the
 * device, without a host sync: a scale that is not a positive power of two
 * turns its row of y into NaN.
 * Replaces reference_fp4_linear_source_semantics (kernels/fp4_source.py:132-156)
 * and the A8 GEMVs xsimt_gemm / qpa_mma_gemm / mxint_*_gemm (kernels/xsimt.py:292-325,
 * kernels/qpa_mma.py:498-541, kernels/mxint.py:362-401,1014-1054); upstream fp4_gemm
 * (.mosaicvm/source/inference_kernel.py:441-536). */
int mosaic_mxt16_linear_a8(const uint8_t* xq, const float* sa, const uint8_t* packed_t, const uint8_t* scale_t,
                           uint16_t* y, int64_t m, int64_t n, int64_t k, void* stream);
/* Scratch bytes of mosaic_mxt16_linear_a8_ws: the fp32 partials of the split-K
 * plan (shapes whose tiles cover at most half of the GPU), else 0. */
size_t mosaic_mxt16_linear_a8_workspace_bytes(int64_t m, int64_t n, int64_t k);
/* mosaic_mxt16_linear_a8 with a caller workspace for the split-K plan (without
 * one, or with too few bytes, the shape runs unsplit).  Same replacement as
 * above: the upstream fp4_gemm tiles every M and N (block_M 32, block_N 128,
 * .mosaicvm/source/inference_kernel.py:441-515). */
int mosaic_mxt16_linear_a8_ws(const uint8_t* xq, const float* sa, const uint8_t* packed_t, const uint8_t* scale_t,
                              uint16_t* y, int64_t m, int64_t n, int64_t k, void* workspace,
                              size_t workspace_bytes, void* stream);

/* ---------------------------------------------------- FP8 block GEMM ----- */
/* C [m, n] = sum over 128-K blocks of (A_kb . B_kb^T) * a_s[m, kb] * b_s[n/128, kb]
 * with A e4m3 [m, k] + f32 a_s [m, k/128], B e4m3 [n, k] (row-major, the
 * checkpoint layout) + f32 b_s [ceil(n/128), k/128]; fp32 accumulation; C is
 * bf16 or f32 (out_dtype).  k % 128 == 0.
 * Replaces fp8_gemm (.mosaicvm/source/inference_kernel.py:203-273),
 * w8a8_block_fp8_matmul (.mosaicvm/source/hubkernel_matmul.py:333-360) and
 * fp8_linear's fused decode GEMM (bench/fp8_core.py:160-231). */
int mosaic_fp8_block_gemm(const uint8_t* a, const float* a_s, const uint8_t* b, const float* b_s, void* c,
                          int out_dtype, int64_t m, int64_t n, int64_t k, void* stream);

/* Bytes of the fp32 partials workspace that mosaic_fp8_block_gemm_ws uses to
 * split K over up to 8 slices when the output tiles cover fewer than half of
 * the GPU (0: the shape is not split).  No counterpart in the reference, whose
 * fp8_gemm launches allocate nothing; it serves the same call sites. */
size_t mosaic_fp8_block_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k);

/* mosaic_fp8_block_gemm with a caller-provided workspace of workspace_bytes
 * (>= mosaic_fp8_block_gemm_workspace_bytes(m, n, k) to split K; with less,
 * or NULL, it runs unsplit).  The slices' fp32 partials are summed in slice
 * order.  Same call sites as mosaic_fp8_block_gemm (fp8_gemm,
 * .mosaicvm/source/inference_kernel.py:203-273). */
int mosaic_fp8_block_gemm_ws(const uint8_t* a, const float* a_s, const uint8_t* b, const float* b_s, void* c,
                             int out_dtype, int64_t m, int64_t n, int64_t k, void* workspace, size_t workspace_bytes,
                             void* stream);

/* T16 prepack of an e4m3 weight [n, k] (n % 16 == 0, k % 128 == 0) into the
 * decode kernel's lane order, n * k bytes: block (g, kb) of 2048 bytes at
 * (g * k/128 + kb) * 2048 holds byte W[16g + c][128kb + 64h + 16q + j] at
 * 1024h + 16(4c + q) + j (c < 16, q < 4, h < 2, j < 16).  A bit-exact
 * permutation; mosaic_fp8_t16_unpack is its inverse.  No counterpart in the
 * reference, whose fp8_gemm (.mosaicvm/source/inference_kernel.py:203-273)
 * reads the checkpoint layout; it serves the same call sites at decode sizes,
 * where each 1 KB load of the prepacked weight is contiguous. */
int mosaic_fp8_t16_prepack(const uint8_t* w, uint8_t* out, int64_t n, int64_t k, void* stream);
int mosaic_fp8_t16_unpack(const uint8_t* t16, uint8_t* w, int64_t n, int64_t k, void* stream);

/* mosaic_fp8_block_gemm with B given as its T16 prepack (bt, n * k bytes) and
 * m <= 64; b_s as for mosaic_fp8_block_gemm.  m <= 16: the decode kernel, the
 * same MFMA operands as over the checkpoint layout, so the same C bit for bit.
 * 16 < m <= 64: the weight streamed once against 2 or 4 groups of 16 rows
 * of A, K split over the caller's workspace of workspace_bytes when it holds
 * mosaic_fp8_block_gemm_t16_workspace_bytes(m, n, k) (NULL: unsplit).  Same
 * call sites as mosaic_fp8_block_gemm (fp8_gemm, w8a8_block_fp8_matmul). */
size_t mosaic_fp8_block_gemm_t16_workspace_bytes(int64_t m, int64_t n, int64_t k);
int mosaic_fp8_block_gemm_t16(const uint8_t* a, const float* a_s, const uint8_t* bt, const float* b_s, void* c,
                              int out_dtype, int64_t m, int64_t n, int64_t k, void* workspace,
                              size_t workspace_bytes, void* stream);

/* W8A16 linear with the in-GEMM weight decode of fp8_linear's fused kernel
 * (bench/fp8_core.py:160-231): y [m, n] bf16 = sum over 128-K blocks of
 * (x_kb . decode(W_kb)^T) * s[n/128, kb], x bf16 [m, k], W e4m3 [n, k]
 * row-major, s f32 [ceil(n/128), k/128] (e8m0 scales passed as their fp32
 * values), fp32 accumulation.  k % 128 == 0, m <= 80 (the reference takes its
 * dequantize + library GEMM path above 80 rows). */
int mosaic_fp8_w8a16_linear(const uint16_t* x, const uint8_t* w, const float* s, uint16_t* y, int64_t m, int64_t n,
                            int64_t k, void* stream);
/* Bytes of the fp32 partials workspace that mosaic_fp8_w8a16_linear_ws uses to
 * split K for this shape (0: the shape does not split). */
size_t mosaic_fp8_w8a16_workspace_bytes(int64_t m, int64_t n, int64_t k);
/* mosaic_fp8_w8a16_linear with a caller workspace (>= the bytes above to split
 * K where the workgroups of one K pass would cover few CUs: 17..80 rows over
 * N >= 4096, 33..80 rows over 1536 <= N < 4096 with K >= 4096, 12..16 rows
 * over weights of >= 40 MB with K >= 6144; with less, or NULL, the whole K
 * runs in one pass).  Same arguments and result otherwise. */
int mosaic_fp8_w8a16_linear_ws(const uint16_t* x, const uint8_t* w, const float* s, uint16_t* y, int64_t m,
                               int64_t n, int64_t k, void* workspace, size_t workspace_bytes, void* stream);

/* e4m3 [n, k] with one f32 scale per block_n x block_k block -> bf16 [n, k].
 * Replaces dequant_fp8 (runtime/fp8.py:52-64), dsa.dequant_weight
 * (model/dsa.py:72-78) and fp8_core's dequant_kernel (bench/fp8_core.py:60-91). */
int mosaic_fp8_block_dequant(const uint8_t* w, const float* s, uint16_t* out, int64_t n, int64_t k, int block_n,
                             int block_k, void* stream);

/* -------------------------------------------------------------- routing -- */
/* logits [m, e] f32 -> ids [m, top_k] int32 + weights [m, top_k] f32.
 * Replaces Router.forward (model/layers.py:118-150) / Gate.forward
 * (.mosaicvm/source/inference_model.py:569-589).  Picks are listed by
 * descending key (the logit, or score + bias when bias != NULL); equal keys go
 * to the lower expert index.  e <= 512, top_k <= 16. */
int mosaic_moe_route_topk(const float* logits, int64_t m, int64_t e, int64_t top_k, int score_func, int renorm,
                          float route_scale, const float* bias, int32_t* ids, float* weights, void* stream);

/* Router projection: logits [m, e] f32 = x [m, h] . w [e, h]^T with x and w
 * each f32 or bf16 (x_dtype, w_dtype), every logit the exact dot product
 * rounded once to fp32 (products exact in fp64, summed in fp64 in a fixed
 * order, one rounding), so routing keys do not depend on a summation order.
 * Replaces the F.linear(x.float(), W.float()) of Router.forward
 * (model/layers.py:128) and Gate.forward (.mosaicvm/source/inference_model.py:570). */
int mosaic_router_logits(const void* x, int x_dtype, const void* w, int w_dtype, float* logits, int64_t m, int64_t e,
                         int64_t h, void* stream);

/* Stable expert sort + uncapped tile list for ids [m, top_k] (+ one shared
 * expert row per token when has_shared, virtual expert id e).
 * Replaces layout_assignments (kernels/moe_layout.py:8-27) and emit_tiles
 * (kernels/w4a16_grouped.py:151-169).  Above 4096 assignments a multi-workgroup path runs
 * with workspace of mosaic_moe_layout_workspace_bytes() bytes (NULL/0 below).
 * Outputs: counts [e(+1)], offsets [e(+1)+1], perm / perm_token / perm_weight /
 * sorted_ids [A] (by sorted position), inv_pos [A] (by flat assignment),
 * combine_pos [m, top_k(+1)] (each token's sorted positions in ascending
 * expert id, shared last), tile_expert / tile_start / tile_rows / tile_p0
 * [tile_cap], n_tiles [1]. */
/* Scratch bytes mosaic_moe_layout needs (0 up to 4096 assignments). */
size_t mosaic_moe_layout_workspace_bytes(int64_t m, int64_t top_k, int64_t e, int has_shared);

int mosaic_moe_layout(const int32_t* ids, const float* weights, int64_t m, int64_t top_k, int64_t e, int has_shared,
                      int block_m, int32_t* counts, int32_t* offsets, int32_t* perm, int32_t* perm_token,
                      float* perm_weight, int32_t* sorted_ids, int32_t* inv_pos, int32_t* combine_pos,
                      int32_t* tile_expert, int32_t* tile_start, int32_t* tile_rows, int32_t* tile_p0,
                      int32_t* n_tiles, int64_t tile_cap, void* workspace, size_t workspace_bytes, void* stream);

/* Tile list from per-expert counts [e] int32: one (expert, m_start, rows)
 * entry per block_m rows, ascending expert order, no per-expert cap.
 * n_tiles[0] is the true tile total, as the reference returns
 * tile_offsets[-1:]; entries past tile_cap are not written, so a caller
 * sizes tile_cap >= the total (A / block_m + e bounds it).
 * Replaces emit_tiles (kernels/w4a16_grouped.py:151-169; the reference caps
 * each expert at MAX_TILES=32, :55-60).  e <= 4096. */
int mosaic_emit_tiles(const int32_t* counts, int64_t e, int block_m, int32_t* tile_expert, int32_t* tile_start,
                      int32_t* tile_rows, int32_t* n_tiles, int64_t tile_cap, void* stream);

/* --------------------------------------------------- A16 routed MoE layer -- */
/* Workspace bytes needed by mosaic_moe_a16_forward. */
size_t mosaic_moe_a16_workspace_bytes(int64_t m, int64_t hidden, int64_t inter, int64_t n_experts, int64_t top_k,
                                      int has_shared);

/* Full routed-expert MoE layer, A16 contract of grouped_expert_forward
 * (model/layers.py:329-373) + shared expert (model/layers.py:284-297):
 *   x [m, hidden] bf16; if logits != NULL the router runs first and writes
 *   ids/weights [m, top_k], else ids/weights are inputs;
 *   gu_* : routed gate|up bank [e, 2*inter, hidden/2] (gate rows 0..inter-1,
 *          up rows inter..2*inter-1), every expert MXT16-prepacked;
 *   d_*  : routed down bank [e, hidden, inter/2], MXT16-prepacked;
 *   sh_* : the shared expert (one MXT16-prepacked matrix pair) or all NULL;
 *   y [m, hidden] bf16.
 * fp32 gate/up, SwiGLU (clamped when swiglu_limit > 0), x route weight before
 * the down projection, bf16 cast, fp32 down, per-token sum of expert partials
 * in ascending expert id, shared expert last, one bf16 rounding.
 * hidden % 128 == 0, inter % 128 == 0.
 * stage_events: NULL, or 5 hipEvent_t recorded on `stream` at start, after
 * routing+layout, after gate/up+SwiGLU, after down, after combine (the stage
 * boundaries of fused_moe_mxint's stage_times, kernels/mxint.py:1494-1500). */
int mosaic_moe_a16_forward(const uint16_t* x, const float* logits, int32_t* ids, float* weights,
                           const uint8_t* gu_packed, const uint8_t* gu_scale, const uint8_t* d_packed,
                           const uint8_t* d_scale, const uint8_t* sh_gu_packed, const uint8_t* sh_gu_scale,
                           const uint8_t* sh_d_packed, const uint8_t* sh_d_scale, uint16_t* y, int64_t m,
                           int64_t hidden, int64_t inter, int64_t n_experts, int64_t top_k, int score_func,
                           int renorm, float route_scale, const float* route_bias, float swiglu_limit,
                           void* workspace, size_t workspace_bytes, void* const* stage_events, void* stream);

/* Largest scratch (bytes) mosaic_moe_a16_forward_noalloc can serve. */
size_t mosaic_moe_a16_noalloc_max_bytes(void);

/* mosaic_moe_a16_forward without a workspace argument and without any device
 * allocation: the layer's scratch is a static per-GPU device array of
 * mosaic_moe_a16_noalloc_max_bytes() (8 MiB: M <= 16 tokens at hidden 7168,
 * inter 2048, 256 experts, top-8, shared expert).  A shape whose workspace
 * (mosaic_moe_a16_workspace_bytes) is larger is rejected with status < 0.
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (several streams or host threads) race.  No stage events.
 * No counterpart in the reference: it exists for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid allocation). */
int mosaic_moe_a16_forward_noalloc(const uint16_t* x, const float* logits, int32_t* ids, float* weights,
                                   const uint8_t* gu_packed, const uint8_t* gu_scale, const uint8_t* d_packed,
                                   const uint8_t* d_scale, const uint8_t* sh_gu_packed, const uint8_t* sh_gu_scale,
                                   const uint8_t* sh_d_packed, const uint8_t* sh_d_scale, uint16_t* y, int64_t m,
                                   int64_t hidden, int64_t inter, int64_t n_experts, int64_t top_k, int score_func,
                                   int renorm, float route_scale, const float* route_bias, float swiglu_limit,
                                   void* stream);

/* fused_moe_skinny (kernels/skinny_fp4.py:267-322), the reference's A16 KN
 * MoE path with its own arithmetic: stable expert sort of the given ids
 * [m, top_k] int32 (weights [m, top_k] f32), grouped KN gate|up into bf16
 * (gu_packed [e, hidden, inter] + gu_scale [e, hidden, 2*inter/32], gate
 * columns then up columns), z = bf16(bf16(silu(gate)) * up), grouped KN down
 * into bf16 (d_packed [e, inter, hidden/2] + d_scale [e, inter, hidden/32]),
 * each output row times bf16(weight) rounded to bf16, then summed per token in
 * bf16 in assignment order (the reference's bf16 index_add_).  No clamp, no
 * shared expert.  Workspace: mosaic_moe_skinny_workspace_bytes(). */
size_t mosaic_moe_skinny_workspace_bytes(int64_t m, int64_t hidden, int64_t inter, int64_t n_experts, int64_t top_k);
int mosaic_moe_skinny_forward(const uint16_t* x, const int32_t* ids, const float* weights, const uint8_t* gu_packed,
                              const uint8_t* gu_scale, const uint8_t* d_packed, const uint8_t* d_scale, uint16_t* y,
                              int64_t m, int64_t hidden, int64_t inter, int64_t n_experts, int64_t top_k,
                              void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------- A8 routed MoE layer -- */
size_t mosaic_moe_a8_workspace_bytes(int64_t m, int64_t hidden, int64_t inter, int64_t n_experts, int64_t top_k,
                                     int has_shared);

/* Routed-expert MoE layer, A8 contract of fused_moe_mxint (kernels/mxint.py:1435-1739;
 * exact_moe / fused_moe_qpa, kernels/exact_moe.py:12-19, kernels/qpa_mma.py:681-784):
 * tokens act-quantized 1x128 pow2 e4m3, A8 gate/up into bf16, fp32 SwiGLU with
 * the clamps when swiglu_limit > 0, x route weight, bf16, 1x128 pow2 e4m3
 * requant, A8 down into bf16 partials, fp32 sum in ascending expert id (an
 * optional shared expert is added last), bf16.  Arguments as
 * mosaic_moe_a16_forward (MXT16 banks).  stage_events: NULL, or 7 hipEvent_t
 * recorded on `stream` at start, after routing+layout, after the token
 * act-quant, after gate/up+SwiGLU, after the z requant (fused into gate/up at
 * prefill sizes), after down, after combine (fused_moe_mxint's stage_times
 * boundaries, kernels/mxint.py:1702-1714). */
int mosaic_moe_a8_forward(const uint16_t* x, const float* logits, int32_t* ids, float* weights,
                          const uint8_t* gu_packed, const uint8_t* gu_scale, const uint8_t* d_packed,
                          const uint8_t* d_scale, const uint8_t* sh_gu_packed, const uint8_t* sh_gu_scale,
                          const uint8_t* sh_d_packed, const uint8_t* sh_d_scale, uint16_t* y, int64_t m,
                          int64_t hidden, int64_t inter, int64_t n_experts, int64_t top_k, int score_func,
                          int renorm, float route_scale, const float* route_bias, float swiglu_limit,
                          void* workspace, size_t workspace_bytes, void* const* stage_events, void* stream);

/* ----------------------------------------------------------- DSA decode -- */
/* Workspace bytes of mosaic_dsa_indexer_topk for b rows of l cached tokens. */
size_t mosaic_dsa_indexer_workspace_bytes(int64_t b, int64_t l);

/* FP8 lightning indexer + top-k, replacing Indexer.forward's scoring and topk
 * (.mosaicvm/source/inference_model.py:408-439; mosaicvm/model/dsa_layers.py:281-321)
 * and the select kernel (mosaicvm/kernels/dsa_attention.py:19-68):
 *   q [b, h, d] e4m3 + q_s [b, h] f32, k [b, l, d] e4m3 + k_s [b, l] f32,
 *   w [b, h] f32 (weights_proj(x) * softmax_scale * h^-0.5);
 *   score[t] = sum_h w_h ReLU(q_h . k_t q_s[h] k_s[t]) in the canonical order
 *   (exact dot rounded once to fp32, * q_s, * k_s, ReLU, * w_h, fp32 sum over h
 *   ascending); idx_out [b, topk] int32 = tokens by descending score, ties to
 *   the lower index, + offset; tokens t >= lengths[b] (lengths NULL = all l)
 *   are masked and missing slots are -1.  d == 128, h in {16, 32, 48, 64},
 *   topk <= 4096, l <= 2^24.  Non-finite q/k codes or scales give unspecified indices. */
int mosaic_dsa_indexer_topk(const uint8_t* q, const float* q_s, const uint8_t* k, const float* k_s, const float* w,
                            const int32_t* lengths, int32_t* idx_out, int64_t b, int64_t h, int64_t d, int64_t l,
                            int64_t topk, int32_t offset, void* workspace, size_t workspace_bytes, void* stream);

/* mosaic_dsa_indexer_topk for `rows` query rows that share key caches in
 * groups: query row r scores the first l tokens of key cache r / rows_per_k
 * with its own length lengths[r] -- the causal prefill of Indexer.forward
 * (.mosaicvm/source/inference_model.py:430-437; mosaicvm/model/dsa_layers.py:309-321),
 * where every position of a sequence scores the same compressed cache up to
 * its own bound.  The caches are read in place: cache g starts at
 * k + g * cache_len * d (k_s + g * cache_len), so a [G, max_len, d] cache
 * sliced to its first l tokens needs no copy (cache_len >= l).  The
 * workspace is mosaic_dsa_indexer_workspace_bytes(rows, l). */
int mosaic_dsa_indexer_topk_shared(const uint8_t* q, const float* q_s, const uint8_t* k, const float* k_s,
                                   const float* w, const int32_t* lengths, int32_t* idx_out, int64_t rows, int64_t h,
                                   int64_t d, int64_t l, int64_t cache_len, int64_t rows_per_k, int64_t topk,
                                   int32_t offset, void* workspace, size_t workspace_bytes, void* stream);

/* The canonical indexer scores themselves, scores [b, l] f32 (the index_score
 * tensor of Indexer.forward, .mosaicvm/source/inference_model.py:424-425). */
int mosaic_dsa_indexer_scores(const uint8_t* q, const float* q_s, const uint8_t* k, const float* k_s, const float* w,
                              float* scores, int64_t b, int64_t h, int64_t d, int64_t l, void* stream);

/* First stage of mosaic_dsa_indexer_topk on its own: per token an interval
 * [lo, hi] (each [b, l] f32) that contains the canonical score, from the
 * bf16-MFMA pass over the exactly decoded fp8 codes.  Diagnostic; same
 * arguments as the scoring above. */
int mosaic_dsa_indexer_bounds(const uint8_t* q, const float* q_s, const uint8_t* k, const float* k_s, const float* w,
                              float* lo, float* hi, int64_t b, int64_t h, int64_t d, int64_t l, void* stream);

/* Per-head top-k sparse attention of one decoding token, replacing
 * dsa_decode_attention (mosaicvm/kernels/dsa_attention.py:113-154): q [h, d]
 * bf16, k [ctx, h, d] bf16, v [ctx, h, dv] bf16; per head s[t] = fp32(exact
 * q_h . k[t, h]) * scale, idx [h, topk] int32 = the top-k positions by
 * descending score (ties to the lower position), out [h, dv] bf16 =
 * softmax(s[idx]) . v[idx, h] in fp32.  d % 8 == 0, d <= 512, topk <= 2048,
 * topk <= ctx.  Workspace: mosaic_dsa_head_attention_workspace_bytes(ctx, h)
 * (the [h, ctx] fp32 scores). */
size_t mosaic_dsa_head_attention_workspace_bytes(int64_t ctx, int64_t h);
int mosaic_dsa_head_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out, int32_t* idx,
                              int64_t h, int64_t ctx, int64_t d, int64_t dv, int64_t topk, float scale,
                              void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes of mosaic_mla_sparse_decode. */
size_t mosaic_mla_decode_workspace_bytes(int64_t b, int64_t h, int64_t topk);

/* MLA decode over the selected KV entries, replacing sparse_attn
 * (.mosaicvm/source/inference_kernel.py:276-368), sparse_attn_fused
 * (mosaicvm/kernels/dsa_sparse.py:92-110) and sparse_attn_ref (mosaicvm/model/dsa.py:214-242):
 *   q [b, h, d_latent + d_rope] bf16; the cache of each row holds n tokens of
 *   kv_latent [b, n, d_latent] e4m3 with kv_scale [b, n, d_latent/scale_block] f32
 *   (dequantized to bf16, as act_quant_sim, mosaicvm/model/dsa.py:81-90) and
 *   kv_rope [b, n, d_rope] bf16; idx [b, topk] int32 (-1, or >= n, = masked);
 *   sink [h] f32 or NULL.  s_t = q . kv_t * softmax_scale (fp32);
 *   out [b, h, d_latent] bf16 = sum_t bf16(exp(s_t - m)) v_t / (sum_t exp(s_t - m)
 *   + exp(sink - m)), v_t = the latent part.  A row with no valid entry gives 0.
 *   d_latent = 512, d_rope = 64, h in {16, 32, 48, 64} or a multiple of 64 up
 *   to 256, scale_block a power of two in 16..512, topk <= 65536. */
int mosaic_mla_sparse_decode(const uint16_t* q, const uint8_t* kv_latent, const float* kv_scale,
                             const uint16_t* kv_rope, const float* sink, const int32_t* idx, uint16_t* out, int64_t b,
                             int64_t h, int64_t n, int64_t topk, int64_t d_latent, int64_t d_rope,
                             int64_t scale_block, float softmax_scale, void* workspace, size_t workspace_bytes,
                             void* stream);

/* MLA / sparse attention over a bf16 KV, the upstream sparse_attn contract
 * (.mosaicvm/source/inference_kernel.py:355-368) and sparse_attn_fused
 * (mosaicvm/kernels/dsa_sparse.py:92-110): q [rows, h, d] bf16, kv [rows /
 * rows_per_kv, n, d] bf16 (query row r reads KV batch r / rows_per_kv), idx
 * [rows, topk] int32, sink [h] f32 or NULL; out [rows, h, 512] bf16 with
 * V = kv[..., :512].  d = 512 (V = K, the V4 geometry) or 576 (512 latent + 64
 * rope).  Same math and head limits as mosaic_mla_sparse_decode; the workspace
 * is mosaic_mla_decode_workspace_bytes(rows, h, topk). */
int mosaic_mla_sparse_decode_bf16(const uint16_t* q, const uint16_t* kv, const float* sink, const int32_t* idx,
                                  uint16_t* out, int64_t rows, int64_t h, int64_t n, int64_t topk, int64_t d,
                                  int64_t rows_per_kv, float softmax_scale, void* workspace, size_t workspace_bytes,
                                  void* stream);

/* Sparse attention over gathered bf16 KV rows with V = K at head dims 64, 128
 * and 256: o [rows, h, d] bf16 from q [rows, h, d] bf16 (h a multiple of 16),
 * kv [rows / rows_per_kv, n, d] bf16 and idx [rows, topk] int32 (-1 or
 * out-of-range entries excluded); scores q . kv * softmax_scale in fp32,
 * online softmax, bf16 probabilities in the value product over fp32 sums,
 * sink (may be NULL) exp(sink[h] - max) in the denominator only; a row with no
 * valid pick gives 0.  No workspace.
 * Replaces sparse_attn_fused at d in {64, 128, 256} (mosaicvm/kernels/dsa_sparse.py:92-110,
 * the Triton kernel :32-89); d = 512 runs mosaic_mla_sparse_decode_bf16. */
int mosaic_sparse_attn_bf16(const uint16_t* q, const uint16_t* kv, const float* sink, const int32_t* idx,
                            uint16_t* out, int64_t rows, int64_t h, int64_t n, int64_t topk, int64_t d,
                            int64_t rows_per_kv, float softmax_scale, void* stream);

/* RMSNorm with the 1x128 activation quantizer fused into its epilogue: the
 * input side of an A8 linear (linear(), .mosaicvm/source/inference_model.py:
 * 114-124, act_quant on an RMSNorm.forward output, :197-202) in one pass.
 * x [m, h] bf16, w [h] fp32: var = fp32(fp64 sum of x^2 / h), r = fp32(1 /
 * sqrt(var + eps)), y = bf16(w * (x * r)); y [m, h] bf16 is written when
 * non-NULL; q [m, h] e4m3 and s [m, h/128] f32 are mosaic_act_quant's output
 * for y with the same mode (0 power of two, 1 max(amax,1e-4)/448, 2 amax/448),
 * ready for mosaic_mxt16_linear_a8 / mosaic_fp8_gemm.  h % 128 == 0,
 * h <= 16384. */
int mosaic_rmsnorm_act_quant(const uint16_t* x, const float* w, float eps, int64_t m, int64_t h, uint16_t* y,
                             uint8_t* q, float* s, int mode, void* stream);

/* Standalone SwiGLU + route weight + 1x128 act_quant epilogue
 * (mxint_swiglu_quant_down, kernels/mxint.py:1298-1345,1387-1408): gu [a, 2*inter]
 * bf16 (gate | up), w_a [a] f32 route weights (NULL: 1) -> z = bf16(silu(min(gate, L))
 * * clamp(up, -L, L) * w) in fp32 (no clamp when limit <= 0), quantized as
 * mosaic_act_quant mode 0 -> q [a, inter] e4m3 codes, s [a, inter/128] f32.  The
 * reference returns the codes as three int8 limb planes of 512 * value (its dp4a
 * operand); the codes themselves are the scaled-MFMA operand here.  inter % 128 == 0,
 * gu 16-byte and q 8-byte aligned. */
int mosaic_swiglu_act_quant(const uint16_t* gu, const float* w_a, int64_t a, int64_t inter, float limit, uint8_t* q,
                            float* s, void* stream);

/* Deterministic routed combine (mxint_routed_reduce, kernels/mxint.py:1346-1365,
 * 1411-1429): yd [a, h] bf16 expert partials in packed order; for each token t,
 * out[t] = bf16(fp32 sum over j of yd[slot_rows[t, order[t, j]]]), accumulated in the
 * order given (order[t] lists the slots by ascending expert id).  slot_rows and order
 * are int32 [k_tok, top_k]; entries outside [0, a) / [0, top_k) add nothing.
 * h % 8 == 0; yd and out 16-byte aligned; k_tok <= 65535. */
int mosaic_routed_reduce(const uint16_t* yd, const int32_t* slot_rows, const int32_t* order, uint16_t* out,
                         int64_t k_tok, int64_t top_k, int64_t h, int64_t a, void* stream);

/* KV-cache writer of the DSA attention step (the kv rows of ExactAttention.forward
 * and attention_core, mosaicvm/model/dsa_layers.py:550-553 and 579-582, stored
 * as _core_body stores them, :510-534): kv [rows, d] bf16 = [d - rope
 * non-rope dims | rope dims]; row r goes to cache row slots[r] (slots NULL:
 * row r; a slot outside [0, n) skips the row).  The non-rope dims get
 * act_quant_sim (mosaicvm/model/dsa.py:81-93): per 64 values
 * s = 2^ceil(log2(max(amax, 1e-4) / 448)), codes = e4m3(clamp(x / s, +-448)).
 * Either cache_bf16 [n, d] receives bf16(codes * s) | rope (the reference's
 * bf16 cache), or codes [n, d - rope] e4m3, scales [n, (d - rope) / 64] fp32
 * and rope_cache [n, rope] bf16 receive them (the FP8 cache
 * mosaic_mla_sparse_decode reads).  d - rope a multiple of 64, at most 512;
 * rope a multiple of 8. */
int mosaic_dsa_kv_write(const uint16_t* kv, const int32_t* slots, int64_t rows, int64_t d, int64_t rope, int64_t n,
                        uint16_t* cache_bf16, uint8_t* codes, float* scales, uint16_t* rope_cache, void* stream);

/* Gather indices of one decode step per query row, replacing window_topk_idxs
 * + compress_topk_idxs_static (mosaicvm/model/dsa.py:185-212) concatenated as
 * in _core_body (mosaicvm/model/dsa_layers.py:479-481): pos [rows] int32
 * absolute positions; out [rows, window + nc] int32 = the ring slots (position
 * % window) of positions max(0, p - window + 1) .. p, oldest first, -1 padded
 * while p < window - 1, then either cidx [rows, nc] (the indexer's picks,
 * already offset) or, with cidx NULL, offset + 0 .. offset + (p + 1) / ratio - 1,
 * -1 padded to nc. */
int mosaic_dsa_decode_indices(const int32_t* pos, int64_t rows, int64_t window, const int32_t* cidx, int64_t nc,
                              int64_t ratio, int64_t offset, int32_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOSAIC_AMD_H */
