// Router projection: logits [m, e] fp32 = x [m, h] . W [e, h]^T, the
// F.linear(x.float(), W.float()) at the head of Router.forward
// (model/layers.py:128) and Gate.forward (.mosaicvm/source/inference_model.py:570).
//
// Each logit is defined as the exact dot product rounded once to fp32: the
// products of fp32 (or bf16) inputs are exact in fp64, and the kernel sums
// them in fp64 (in a fixed order, so the result is reproducible) before one
// rounding to fp32.  The fp64 sum is within n * 2^-53 * sum|terms| of the
// exact one, so the fp32 result is the correctly rounded exact dot unless the
// exact value lies that close to a rounding boundary.  Routing keys therefore
// do not depend on a summation order.
//
// Work split: a workgroup of 256 threads owns ET experts x MT tokens; every
// thread strides over h and keeps MT x ET fp64 partial sums, which a
// wave-level then cross-wave reduction folds.  The weight is the HBM stream
// (e x h, read once per token tile); x rows are re-read from L2 by the
// workgroups of other experts.
#include <hip/hip_runtime.h>

#include "../../include/mosaic_amd.h"
#include "common.h"

namespace mosaic {
namespace {

template <typename T>
__device__ __forceinline__ double load_f64(const T* p, int64_t i);
template <>
__device__ __forceinline__ double load_f64<uint16_t>(const uint16_t* p, int64_t i) {
  return (double)bf16_f32(p[i]);
}
template <>
__device__ __forceinline__ double load_f64<float>(const float* p, int64_t i) {
  return (double)p[i];
}

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <typename TX, typename TW, int MT, int ET>
__global__ void __launch_bounds__(256) router_logits_kernel(const TX* __restrict__ x, const TW* __restrict__ w,
                                                            float* __restrict__ logits, int M, int E, int H) {
  __shared__ double s_part[4][MT * ET];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int e0 = blockIdx.x * ET, m0 = blockIdx.y * MT;
  double acc[MT][ET];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < ET; ++j) acc[i][j] = 0.0;
  for (int h = tid; h < H; h += 256) {
    double wv[ET];
#pragma unroll
    for (int j = 0; j < ET; ++j) wv[j] = (e0 + j < E) ? load_f64(w, (int64_t)(e0 + j) * H + h) : 0.0;
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const double xv = (m0 + i < M) ? load_f64(x, (int64_t)(m0 + i) * H + h) : 0.0;
#pragma unroll
      for (int j = 0; j < ET; ++j) acc[i][j] = fma(xv, wv[j], acc[i][j]);  // the product is exact
    }
  }
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < ET; ++j) {
      const double s = wave_sum_f64(acc[i][j]);
      if (lane == 0) s_part[wave][i * ET + j] = s;
    }
  __syncthreads();
  if (tid < MT * ET) {
    const int i = tid / ET, j = tid % ET;
    const double s = ((s_part[0][tid] + s_part[1][tid]) + s_part[2][tid]) + s_part[3][tid];
    if (m0 + i < M && e0 + j < E) logits[(int64_t)(m0 + i) * E + e0 + j] = (float)s;
  }
}

template <typename TX, typename TW>
void launch_router(const void* x, const void* w, float* logits, int64_t m, int64_t e, int64_t h, hipStream_t st) {
  if (m <= 4) {
    MOSAIC_LAUNCH((router_logits_kernel<TX, TW, 4, 1>), dim3((unsigned)e, (unsigned)((m + 3) / 4)), dim3(256), 0,
                       st, (const TX*)x, (const TW*)w, logits, (int)m, (int)e, (int)h);
  } else {
    MOSAIC_LAUNCH((router_logits_kernel<TX, TW, 8, 2>), dim3((unsigned)((e + 1) / 2), (unsigned)((m + 7) / 8)),
                       dim3(256), 0, st, (const TX*)x, (const TW*)w, logits, (int)m, (int)e, (int)h);
  }
}

}  // namespace
}  // namespace mosaic

extern "C" int mosaic_router_logits(const void* x, int x_dtype, const void* w, int w_dtype, float* logits, int64_t m,
                                    int64_t e, int64_t h, void* stream) {
  using namespace mosaic;
  MOSAIC_CHECK_ARG(x && w && logits, "router_logits: null pointer");
  MOSAIC_CHECK_ARG(m >= 0 && e >= 1 && h >= 1 && m < (1ll << 31) && e <= 65535 && h < (1ll << 31),
                   "router_logits: bad shape m=%lld e=%lld h=%lld", (long long)m, (long long)e, (long long)h);
  MOSAIC_CHECK_ARG((x_dtype == MOSAIC_DTYPE_F32 || x_dtype == MOSAIC_DTYPE_BF16) &&
                       (w_dtype == MOSAIC_DTYPE_F32 || w_dtype == MOSAIC_DTYPE_BF16),
                   "router_logits: dtypes must be f32 or bf16");
  if (m == 0) return kOk;
  hipStream_t st = (hipStream_t)stream;
  const bool xb = x_dtype == MOSAIC_DTYPE_BF16, wb = w_dtype == MOSAIC_DTYPE_BF16;
  if (xb && wb)
    launch_router<uint16_t, uint16_t>(x, w, logits, m, e, h, st);
  else if (xb)
    launch_router<uint16_t, float>(x, w, logits, m, e, h, st);
  else if (wb)
    launch_router<float, uint16_t>(x, w, logits, m, e, h, st);
  else
    launch_router<float, float>(x, w, logits, m, e, h, st);
  MOSAIC_RETURN_LAUNCH("router_logits");
}
