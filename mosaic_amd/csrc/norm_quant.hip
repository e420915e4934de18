// RMSNorm with the 1x128 activation quantizer fused into its epilogue: the
// producer side of an A8 linear (linear(), .mosaicvm/source/inference_model.py
// :114-124, quantizes its input with act_quant before fp4_gemm / fp8_gemm; the
// input is an RMSNorm output, RMSNorm.forward :197-202).  One pass over the
// row instead of a norm kernel writing bf16 and a quantizer reading it back.
//
// Canonical arithmetic (the reference's order, reductions pinned):
//   ss  = sum_i x_i^2 in fp64 (each square exact), var = fp32(ss / H);
//   r   = fp32(1 / sqrt(fp64(var) + fp64(eps)))  (one rounding);
//   y_i = bf16(fp32(w_i * fp32(x_i * r)))        (RMSNorm.forward's .to(dtype));
//   per 128 values of y: the act_quant scale of `mode` (0: power of two,
//   act_quant_ref; 1: max(amax, 1e-4) * fp32(1/448); 2: amax / 448) and
//   codes = e4m3(clamp(y / s, +-448)) -- the quantizer of mosaic_act_quant.
// One workgroup per row; thread t holds the 8-value chunks t, t + 256, ...;
// the 16 lanes of a DPP row cover one 128-value block.
#include "common.h"
#include "../../include/mosaic_amd.h"

namespace mosaic {
namespace {

constexpr int kNqMaxChunks = 8;  // 8-value chunks per thread: H <= 16384

__device__ __forceinline__ float row16_max_nq(float v) {
  v = fmaxf(v, __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(v), 0xB1, 0xF)));
  v = fmaxf(v, __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(v), 0x4E, 0xF)));
  v = fmaxf(v, __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(v), 0x141, 0xF)));
  return fmaxf(v, __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(v), 0x140, 0xF)));
}

template <int NCH>
__global__ void __launch_bounds__(256) rmsnorm_act_quant_kernel(const uint16_t* __restrict__ x,
                                                                const float* __restrict__ w, float eps, int H,
                                                                uint16_t* __restrict__ y, uint8_t* __restrict__ q,
                                                                float* __restrict__ s_out, int mode) {
  __shared__ double red[4];
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int nch = H / 8;
  const uint16_t* xr = x + (int64_t)row * H;
  float v[NCH][8];
  double ss = 0.0;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = tid + 256 * i;
    u32x4_t raw = {0u, 0u, 0u, 0u};
    if (c < nch) raw = *reinterpret_cast<const u32x4_t*>(xr + 8 * c);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[i][2 * e] = __uint_as_float(raw[e] << 16);
      v[i][2 * e + 1] = __uint_as_float(raw[e] & 0xFFFF0000u);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += (double)v[i][e] * (double)v[i][e];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
  if (lane == 0) red[wv] = ss;
  __syncthreads();
  const double tot = ((red[0] + red[1]) + red[2]) + red[3];
  const float var = (float)(tot / (double)H);
  const float r = (float)(1.0 / sqrt((double)var + (double)eps));
  const int nb = H / 128;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = tid + 256 * i;
    const bool ok = c < nch;  // uniform over each 16-lane block (H % 128 == 0)
    float yv[8];
    uint32_t yw[4];
    float amax = 0.f;
    if (ok) {
      const f32x4_t w0 = *reinterpret_cast<const f32x4_t*>(w + 8 * c);
      const f32x4_t w1 = *reinterpret_cast<const f32x4_t*>(w + 8 * c + 4);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float wv_ = e < 4 ? w0[e] : w1[e - 4];
        yv[e] = wv_ * (v[i][e] * r);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        yw[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{yv[2 * e], yv[2 * e + 1]}, bf16x2_t));
        yv[2 * e] = __uint_as_float(yw[e] << 16);
        yv[2 * e + 1] = __uint_as_float(yw[e] & 0xFFFF0000u);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(yv[e]));
    }
    amax = row16_max_nq(amax);
    if (!ok) continue;
    if (y) *reinterpret_cast<u32x4_t*>(y + (int64_t)row * H + 8 * c) = u32x4_t{yw[0], yw[1], yw[2], yw[3]};
    float s;
    if (mode == 0)
      s = act_scale_pow2(amax);
    else if (mode == 1)
      s = fmaxf(amax, 1e-4f) * 0.002232142925783992f;
    else
      s = amax / 448.0f;
    const float inv = mode == 0 ? 1.0f / s : 0.f;  // exact for a power of two
    uint32_t cw[2] = {0u, 0u};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float t = mode == 0 ? yv[e] * inv : yv[e] / s;
      t = fminf(fmaxf(t, -448.0f), 448.0f);
      cw[e >> 2] |= e4m3_hw(t) << (8 * (e & 3));
    }
    *reinterpret_cast<uint2*>(q + (int64_t)row * H + 8 * c) = uint2{cw[0], cw[1]};
    if ((lane & 15) == 0) s_out[(int64_t)row * nb + c / 16] = s;
  }
}

}  // namespace
}  // namespace mosaic

using namespace mosaic;

extern "C" int mosaic_rmsnorm_act_quant(const uint16_t* x, const float* w, float eps, int64_t m, int64_t h,
                                        uint16_t* y, uint8_t* q, float* s, int mode, void* stream) {
  MOSAIC_CHECK_ARG(x && w && q && s, "rmsnorm_act_quant: null pointer");
  MOSAIC_CHECK_ARG(h > 0 && h % 128 == 0 && h <= 2048 * kNqMaxChunks,
                   "rmsnorm_act_quant: H=%lld must be a positive multiple of 128, at most %d", (long long)h,
                   2048 * kNqMaxChunks);
  MOSAIC_CHECK_ARG(m >= 0 && m < (1ll << 31), "rmsnorm_act_quant: M=%lld out of range", (long long)m);
  MOSAIC_CHECK_ARG(mode >= 0 && mode <= 2, "rmsnorm_act_quant: mode %d (0 pow2, 1 amax, 2 hf)", mode);
  if (m == 0) return kOk;
  hipStream_t st = (hipStream_t)stream;
  const int nchunk = (int)((h / 8 + 255) / 256);
#define NQ_CASE(N)                                                                                               \
  case N:                                                                                                        \
    MOSAIC_LAUNCH(rmsnorm_act_quant_kernel<N>, dim3((unsigned)m), dim3(256), 0, st, x, w, eps, (int)h, y, q, \
                       s, mode);                                                                                 \
    break;
  switch (nchunk) {
    NQ_CASE(1) NQ_CASE(2) NQ_CASE(3) NQ_CASE(4) NQ_CASE(5) NQ_CASE(6) NQ_CASE(7) NQ_CASE(8)
  }
#undef NQ_CASE
  MOSAIC_RETURN_LAUNCH("rmsnorm_act_quant");
}
