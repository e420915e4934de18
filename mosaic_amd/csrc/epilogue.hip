// Standalone MoE epilogues, for callers that run the expert GEMMs themselves
// (the fused MoE entries do the same work inside their gate/up and down
// kernels):
//
// swiglu_act_quant (mxint_swiglu_quant_down, kernels/mxint.py:1298-1345,
// 1387-1408): gu [A, 2*inter] bf16 (gate | up) and a route weight per row ->
// z = bf16(silu(min(gate, L)) * clamp(up, +-L) * w) in fp32, then the 1x128
// power-of-two act_quant of z -> e4m3 codes [A, inter] + fp32 scales
// [A, inter/128].  The reference splits each code into three int8 limb planes
// of 512 * value for its dp4a GEMMs; the scaled MFMA here consumes the e4m3
// codes as they are, so the codes are the output.
//
// routed_reduce (mxint_routed_reduce, kernels/mxint.py:1346-1365, 1411-1429):
// per token t, acc = sum over s of yd[slot_rows[t, order[t, s]]] in fp32, in
// the order given (ascending expert id), then one bf16 rounding.
//
// Layout: 16 lanes per 128-value block, 8 consecutive values a lane (16-byte
// bf16 loads, 8-byte code stores), as the 1x128 act_quant kernel.
#include "common.h"

namespace mosaic {

__device__ __forceinline__ void load8_bf16(const uint16_t* p, float (&v)[8]) {
  const u32x4_t w = *reinterpret_cast<const u32x4_t*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
  }
}

__global__ void __launch_bounds__(256) swiglu_act_quant_kernel(const uint16_t* __restrict__ gu,
                                                               const float* __restrict__ w_a,
                                                               uint8_t* __restrict__ q, float* __restrict__ s_out,
                                                               int64_t n_chunks, int inter, float limit) {
  const int64_t ch = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // 8-value chunk of z
  if (ch >= n_chunks) return;  // n_chunks is a multiple of 16: whole 16-lane groups leave together
  const int cpr = inter / 8;
  const int64_t row = ch / cpr;
  const int col = (int)(ch % cpr) * 8;
  const uint16_t* g = gu + row * 2 * inter + col;
  float gv[8], uv[8];
  load8_bf16(g, gv);
  load8_bf16(g + inter, uv);
  const float w = w_a ? w_a[row] : 1.0f;
  float z[8];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    z[i] = bf16_f32(f32_bf16(swiglu_f32(gv[i], uv[i], limit) * w));
    amax = fmaxf(amax, fabsf(z[i]));
  }
  // max over the block's 16 lanes (one DPP row)
  amax = fmaxf(amax, __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(amax), 0xB1, 0xF)));
  amax = fmaxf(amax, __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(amax), 0x4E, 0xF)));
  amax = fmaxf(amax, __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(amax), 0x141, 0xF)));
  amax = fmaxf(amax, __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(amax), 0x140, 0xF)));
  const float s = act_scale_pow2(amax);
  const float inv = 1.0f / s;  // exact: s is a power of two
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float y = fminf(fmaxf(z[i] * inv, -448.0f), 448.0f);
    const uint32_t b = e4m3_hw(y);
    if (i < 4) lo |= b << (8 * i);
    else hi |= b << (8 * (i - 4));
  }
  *reinterpret_cast<uint2*>(q + row * inter + col) = uint2{lo, hi};
  if ((threadIdx.x & 15) == 0) s_out[row * (inter / 128) + col / 128] = s;
}

// One thread per 8 columns of one token; rows outside [0, A) and slots outside
// [0, top_k) contribute nothing (they are caller errors that must not fault).
__global__ void __launch_bounds__(128) routed_reduce_kernel(const uint16_t* __restrict__ yd,
                                                            const int32_t* __restrict__ slot_rows,
                                                            const int32_t* __restrict__ order,
                                                            uint16_t* __restrict__ out, int top_k, int H,
                                                            int64_t A) {
  const int64_t t = blockIdx.y;
  const int h = 8 * (blockIdx.x * blockDim.x + threadIdx.x);
  if (h >= H) return;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < top_k; ++j) {
    const int slot = order[t * top_k + j];
    if ((unsigned)slot >= (unsigned)top_k) continue;
    const int64_t r = slot_rows[t * top_k + slot];
    if (r < 0 || r >= A) continue;
    float v[8];
    load8_bf16(yd + r * H + h, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] += v[i];
  }
  u32x4_t o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = (uint32_t)f32_bf16(acc[2 * i]) | ((uint32_t)f32_bf16(acc[2 * i + 1]) << 16);
  *reinterpret_cast<u32x4_t*>(out + t * H + h) = o;
}

}  // namespace mosaic

using namespace mosaic;

extern "C" int mosaic_swiglu_act_quant(const uint16_t* gu, const float* w_a, int64_t a, int64_t inter, float limit,
                                       uint8_t* q, float* s, void* stream) {
  MOSAIC_CHECK_ARG(gu && q && s, "swiglu_act_quant: null pointer");
  MOSAIC_CHECK_ARG(a >= 0 && inter > 0 && inter % 128 == 0 && inter <= (1 << 24),
                   "swiglu_act_quant: inter=%lld must be a positive multiple of 128", (long long)inter);
  MOSAIC_CHECK_ARG(((uintptr_t)gu & 15u) == 0 && ((uintptr_t)q & 7u) == 0,
                   "swiglu_act_quant: gu must be 16-byte and q 8-byte aligned");
  const int64_t chunks = a * inter / 8;
  MOSAIC_CHECK_ARG(chunks < ((int64_t)1 << 31), "swiglu_act_quant: A*inter=%lld too large", (long long)(a * inter));
  if (chunks == 0) return kOk;
  MOSAIC_LAUNCH(swiglu_act_quant_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                gu, w_a, q, s, chunks, (int)inter, limit);
  MOSAIC_RETURN_LAUNCH("swiglu_act_quant");
}

extern "C" int mosaic_routed_reduce(const uint16_t* yd, const int32_t* slot_rows, const int32_t* order, uint16_t* out,
                                    int64_t k_tok, int64_t top_k, int64_t h, int64_t a, void* stream) {
  MOSAIC_CHECK_ARG(out && (k_tok == 0 || (yd && slot_rows && order)), "routed_reduce: null pointer");
  MOSAIC_CHECK_ARG(k_tok >= 0 && k_tok <= 65535 && top_k >= 0 && top_k <= 1024 && a >= 0,
                   "routed_reduce: k_tok=%lld (at most 65535) top_k=%lld", (long long)k_tok, (long long)top_k);
  MOSAIC_CHECK_ARG(h > 0 && h % 8 == 0 && h <= (1 << 24), "routed_reduce: H=%lld must be a positive multiple of 8",
                   (long long)h);
  MOSAIC_CHECK_ARG(((uintptr_t)yd & 15u) == 0 && ((uintptr_t)out & 15u) == 0,
                   "routed_reduce: yd and out must be 16-byte aligned");
  if (k_tok == 0) return kOk;
  MOSAIC_LAUNCH(routed_reduce_kernel, dim3((unsigned)((h / 8 + 127) / 128), (unsigned)k_tok), dim3(128), 0,
                (hipStream_t)stream, yd, slot_rows, order, out, (int)top_k, (int)h, a);
  MOSAIC_RETURN_LAUNCH("routed_reduce");
}
