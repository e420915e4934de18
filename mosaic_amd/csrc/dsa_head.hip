// Per-head top-k sparse attention for one decoding token, the contract of
// dsa_decode_attention (mosaicvm/kernels/dsa_attention.py:113-154): every head
// h selects its own top-k context positions by s[h, t] = (q_h . k[t, h]) *
// scale and attends over them with softmax(s) (fp32, no sink).
//
// Scores are defined canonically: the exact dot product rounded once to fp32
// (bf16 x bf16 products are exact; the kernel sums them in fp64), then one
// fp32 multiply by `scale`.  Selection: descending score, equal scores to the
// lower position (the reference's running top-k keeps the earlier position on
// ties), listed in that order.
//
// Three launches: scores [h][ctx] into the workspace (one thread per (t, h),
// q_h in LDS); per head a workgroup finds the k-th largest score by a 3-pass
// radix select on the order-preserving 32-bit key, takes every position above
// it and the lowest positions equal to it, and bitonic-sorts the picks; per
// head a workgroup runs the softmax over its picks and the weighted V sum.
#include <hip/hip_runtime.h>

#include "../../include/mosaic_amd.h"
#include "common.h"

namespace mosaic {
namespace {

constexpr int kHeadMaxTopk = 2048;
constexpr int kHeadMaxDim = 512;

__device__ __forceinline__ uint32_t f32_key(float f) {  // order-preserving, NaN lowest
  if (f != f) return 0u;
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// scores[h][t] = fp32(exact q_h . k[t, h]) * scale; grid (ceil(ctx / 256), H)
__global__ void __launch_bounds__(256) head_scores_kernel(const uint16_t* __restrict__ q,
                                                          const uint16_t* __restrict__ k, float* __restrict__ scores,
                                                          int ctx, int H, int D, float scale) {
  __shared__ float qs[kHeadMaxDim];
  const int h = blockIdx.y;
  for (int i = threadIdx.x; i < D; i += 256) qs[i] = bf16_f32(q[(int64_t)h * D + i]);
  __syncthreads();
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= ctx) return;
  const uint16_t* kr = k + ((int64_t)t * H + h) * D;
  double acc = 0.0;
  for (int i = 0; i < D; i += 8) {
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(kr + i);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc = fma((double)__uint_as_float(v[j] << 16), (double)qs[i + 2 * j], acc);
      acc = fma((double)__uint_as_float(v[j] & 0xFFFF0000u), (double)qs[i + 2 * j + 1], acc);
    }
  }
  scores[(int64_t)h * ctx + t] = (float)acc * scale;
}

// per head: the top-k positions by (score desc, position asc), in that order
__global__ void __launch_bounds__(1024) head_topk_kernel(const float* __restrict__ scores, int32_t* __restrict__ idx,
                                                         int ctx, int topk, int sort_n) {
  __shared__ uint32_t hist[2048];
  __shared__ uint64_t picks[kHeadMaxTopk];
  __shared__ uint32_t s_prefix, s_remaining, s_count, s_eq_base;
  __shared__ uint32_t s_wsum[16];
  const int h = blockIdx.x, tid = threadIdx.x;
  const float* sc = scores + (int64_t)h * ctx;
  // 1. radix select of the topk-th largest 32-bit key: passes of 11, 11, 10 bits
  if (tid == 0) {
    s_prefix = 0u;
    s_remaining = (uint32_t)topk;
  }
  const int shifts[3] = {21, 10, 0};
  const int widths[3] = {11, 11, 10};
  for (int p = 0; p < 3; ++p) {
    for (int i = tid; i < 2048; i += 1024) hist[i] = 0u;
    __syncthreads();
    const int sh = shifts[p], wd = widths[p];
    const uint32_t prefix = s_prefix;
    const int hi_sh = sh + wd;
    for (int t = tid; t < ctx; t += 1024) {
      const uint32_t key = f32_key(sc[t]);
      const bool match = hi_sh >= 32 ? true : ((key >> hi_sh) == (prefix >> hi_sh));
      if (match) atomicAdd(&hist[(key >> sh) & ((1u << wd) - 1u)], 1u);
    }
    __syncthreads();
    if (tid == 0) {
      uint32_t rem = s_remaining;
      int d = (1 << wd) - 1;
      for (; d > 0; --d) {
        if (hist[d] >= rem) break;
        rem -= hist[d];
      }
      s_prefix = prefix | ((uint32_t)d << sh);
      s_remaining = rem;  // how many keys equal to the final threshold are taken
    }
    __syncthreads();
  }
  const uint32_t T = s_prefix;
  const uint32_t need_eq = s_remaining;
  // 2. every key above T, then the lowest positions with key == T
  if (tid == 0) s_count = 0u;
  __syncthreads();
  for (int t = tid; t < ctx; t += 1024) {
    const uint32_t key = f32_key(sc[t]);
    if (key > T) picks[atomicAdd(&s_count, 1u)] = ((uint64_t)key << 32) | (0xFFFFFFFFu - (uint32_t)t);
  }
  if (tid == 0) s_eq_base = 0u;
  __syncthreads();
  const uint32_t n_gt = s_count;
  const int lane = tid & 63, wv = tid >> 6;
  for (int base = 0; base < ctx && s_eq_base < need_eq; base += 1024) {
    const int t = base + tid;
    const bool eq = t < ctx && f32_key(sc[t]) == T;
    const uint64_t bal = __ballot(eq);
    const uint32_t before = (uint32_t)__builtin_popcountll(bal & ((1ull << lane) - 1ull));
    if (lane == 0) s_wsum[wv] = (uint32_t)__builtin_popcountll(bal);
    __syncthreads();
    uint32_t off = s_eq_base;
    for (int i = 0; i < wv; ++i) off += s_wsum[i];
    const uint32_t r = off + before;
    if (eq && r < need_eq) picks[n_gt + r] = ((uint64_t)T << 32) | (0xFFFFFFFFu - (uint32_t)t);
    __syncthreads();
    if (tid == 0) {
      uint32_t tot = 0;
      for (int i = 0; i < 16; ++i) tot += s_wsum[i];
      s_eq_base += tot;
    }
    __syncthreads();
  }
  // 3. bitonic sort of the topk picks, descending (padding sorts last)
  for (int i = topk + tid; i < sort_n; i += 1024) picks[i] = 0ull;
  __syncthreads();
  for (int kk = 2; kk <= sort_n; kk <<= 1) {
    for (int j = kk >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < sort_n; i += 1024) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const uint64_t a = picks[i], b = picks[ixj];
          const bool desc = (i & kk) == 0;
          if (desc ? (a < b) : (a > b)) {
            picks[i] = b;
            picks[ixj] = a;
          }
        }
      }
      __syncthreads();
    }
  }
  for (int i = tid; i < topk; i += 1024)
    idx[(int64_t)h * topk + i] = (int32_t)(0xFFFFFFFFu - (uint32_t)(picks[i] & 0xFFFFFFFFull));
}

// per head: out[h] = sum_i p_i v[idx_i, h] / sum_i p_i, p_i = exp(s_i - s_0)
// (s_0, the first pick, is the largest score); fp32, one bf16 rounding
__global__ void __launch_bounds__(256) head_attend_kernel(const float* __restrict__ scores,
                                                          const int32_t* __restrict__ idx,
                                                          const uint16_t* __restrict__ v, uint16_t* __restrict__ out,
                                                          int ctx, int H, int DV, int topk) {
  __shared__ float p[kHeadMaxTopk];
  __shared__ int32_t pos[kHeadMaxTopk];
  __shared__ float red[4];
  const int h = blockIdx.x, tid = threadIdx.x;
  const int32_t* ih = idx + (int64_t)h * topk;
  const float m = scores[(int64_t)h * ctx + ih[0]];
  float part = 0.f;
  for (int i = tid; i < topk; i += 256) {
    const int t = ih[i];
    const float e = expf(scores[(int64_t)h * ctx + t] - m);
    p[i] = e;
    pos[i] = t;
    part += e;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off, 64);
  if ((tid & 63) == 0) red[tid >> 6] = part;
  __syncthreads();
  const float l = ((red[0] + red[1]) + red[2]) + red[3];
  for (int d = tid; d < DV; d += 256) {
    float acc = 0.f;
    for (int i = 0; i < topk; ++i) acc += p[i] * bf16_f32(v[((int64_t)pos[i] * H + h) * DV + d]);
    out[(int64_t)h * DV + d] = f32_bf16(acc / l);
  }
}

}  // namespace
}  // namespace mosaic

using namespace mosaic;

extern "C" size_t mosaic_dsa_head_attention_workspace_bytes(int64_t ctx, int64_t h) {
  return ctx > 0 && h > 0 ? (size_t)ctx * h * 4 : 0;
}

extern "C" int mosaic_dsa_head_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out,
                                         int32_t* idx, int64_t h, int64_t ctx, int64_t d, int64_t dv, int64_t topk,
                                         float scale, void* workspace, size_t workspace_bytes, void* stream) {
  MOSAIC_CHECK_ARG(q && k && v && out && idx, "dsa_head_attention: null pointer");
  MOSAIC_CHECK_ARG(h >= 1 && h <= 65535 && d >= 8 && d % 8 == 0 && d <= kHeadMaxDim && dv >= 1 && dv <= 65535,
                   "dsa_head_attention: heads %lld, dims %lld / %lld (d a multiple of 8, at most %d)", (long long)h,
                   (long long)d, (long long)dv, kHeadMaxDim);
  MOSAIC_CHECK_ARG(topk >= 1 && topk <= kHeadMaxTopk && topk <= ctx && ctx < (1ll << 31),
                   "dsa_head_attention: topk %lld (1..%d, <= ctx %lld)", (long long)topk, kHeadMaxTopk,
                   (long long)ctx);
  MOSAIC_CHECK_ARG(workspace && workspace_bytes >= (size_t)ctx * h * 4, "dsa_head_attention: workspace %zu < %zu",
                   workspace_bytes, (size_t)ctx * h * 4);
  hipStream_t st = (hipStream_t)stream;
  float* scores = (float*)workspace;
  MOSAIC_LAUNCH(head_scores_kernel, dim3((unsigned)((ctx + 255) / 256), (unsigned)h), dim3(256), 0, st, q, k,
                     scores, (int)ctx, (int)h, (int)d, scale);
  MOSAIC_LAUNCH_CHECK("dsa_head_scores");
  int sort_n = 1;
  while (sort_n < topk) sort_n <<= 1;
  MOSAIC_LAUNCH(head_topk_kernel, dim3((unsigned)h), dim3(1024), 0, st, scores, idx, (int)ctx, (int)topk, sort_n);
  MOSAIC_LAUNCH_CHECK("dsa_head_topk");
  MOSAIC_LAUNCH(head_attend_kernel, dim3((unsigned)h), dim3(256), 0, st, scores, idx, v, out, (int)ctx, (int)h,
                     (int)dv, (int)topk);
  MOSAIC_RETURN_LAUNCH("dsa_head_attend");
}
