// Sparse attention over gathered bf16 KV rows at head dims 64, 128 and 256,
// V = K (sparse_attn_fused, mosaicvm/kernels/dsa_sparse.py:32-110; the
// semantics of the upstream sparse_attn_kernel,
// .mosaicvm/source/inference_kernel.py:276-352):
//   s = q . kv[idx] * scale in fp32, picks with idx == -1 excluded, online
//   softmax, the value product with bf16-rounded probabilities over fp32
//   running sums, the sink exp(sink - max) in the denominator only, o bf16.
// (Head dim 512, and the 512 + 64 MLA layout, run the MLA kernels.)
//
// A workgroup owns one query row and 16 heads; its 4 waves split the row's
// picks into contiguous runs of 32-token blocks and merge their (max, sum, O)
// at the end.  Per block a wave:
//   * loads the 32 gathered K rows straight into MFMA operands (lane (g, c)
//     holds row 16 tg + c, dims 32 s + 8 g .. + 8) and also writes them into
//     its private LDS block;
//   * computes S^T = K Q^T on v_mfma_f32_16x16x32_bf16 (q pinned in registers
//     as the B operand), so lane (g, c) holds the scores of head c for tokens
//     16 tg + 4 g + r: the softmax statistics of a head live in the lanes of
//     column c and reduce across the four lane groups;
//   * adds O^T += V^T P^T on the same MFMA with the block's tokens permuted so
//     that k = 8 g + i is token 4 g + i (i < 4) or 16 + 4 g + i - 4: P^T is then
//     the lane's own probabilities, and V^T comes from two gfx950 transposing
//     LDS reads (ds_read_b64_tr_b16) of rows 4 g .. 4 g + 3 and 16 + 4 g .. + 3.
// O^T keeps a head per lane column, so the rescale by exp(m_old - m_new) is
// the lane's own factor.
#include <hip/hip_runtime.h>

#include <cmath>

#include "../../include/mosaic_amd.h"
#include "common.h"

namespace mosaic {
namespace {

typedef short v4s_t __attribute__((ext_vector_type(4)));
typedef short v8s_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x4_t mfma_bf16_16x16x32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float lane_xor_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 16));
  return fmaxf(v, __shfl_xor(v, 32));
}
__device__ __forceinline__ float lane_xor_sum(float v) {
  v += __shfl_xor(v, 16);
  return v + __shfl_xor(v, 32);
}

template <int D>
__global__ void __launch_bounds__(256) sparse_attn_kernel(const uint16_t* __restrict__ q,
                                                          const uint16_t* __restrict__ kv,
                                                          const int32_t* __restrict__ idx,
                                                          const float* __restrict__ sink, uint16_t* __restrict__ o,
                                                          int H, int T, int64_t N, int rows_per_kv, float scale) {
  constexpr int NS = D / 32;          // 32-dim steps of a score dot
  constexpr int NJ = D / 16;          // 16-dim tiles of O
  constexpr int PITCH = D * 2 + 16;   // bytes per staged K row (rows start on distinct banks)
  constexpr int BLK = 32 * PITCH;     // one wave's staged block
  static_assert(4 * BLK >= 4 * D * 16 * 4, "the merge reuses the staging blocks");
  __shared__ __attribute__((aligned(16))) uint8_t kst[4 * BLK];
  __shared__ float mls[4][2][16];
  const int row = blockIdx.x, ht = blockIdx.y;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, c = lane & 15;
  const uint16_t* kvb = kv + (int64_t)(row / rows_per_kv) * N * D;
  // B operand of S^T: Q^T, lane (g, c) holds q[head c][32 s + 8 g .. + 8]
  const uint16_t* qrow = q + ((int64_t)row * H + 16 * ht + c) * D;
  bf16x8_t qf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) qf[s] = *reinterpret_cast<const bf16x8_t*>(qrow + 32 * s + 8 * g);
  const int nblk = (T + 31) / 32;
  const int b0 = w * nblk / 4, b1 = (w + 1) * nblk / 4;
  const int32_t* irow = idx + (int64_t)row * T;
  uint8_t* kb = kst + w * BLK;
  float m = -INFINITY, l = 0.f;
  f32x4_t acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int b = b0; b < b1; ++b) {
    // tokens 16 tg + c of the block (lane column c)
    bool val[2];
    int64_t tok[2];
#pragma unroll
    for (int tg = 0; tg < 2; ++tg) {
      const int t = 32 * b + 16 * tg + c;
      const int id = t < T ? irow[t] : -1;
      val[tg] = id >= 0 && (int64_t)id < N;
      tok[tg] = val[tg] ? id : 0;
    }
    bf16x8_t kf[2][NS];
#pragma unroll
    for (int tg = 0; tg < 2; ++tg)
#pragma unroll
      for (int s = 0; s < NS; ++s)
        kf[tg][s] = *reinterpret_cast<const bf16x8_t*>(kvb + tok[tg] * D + 32 * s + 8 * g);
    // the previous block's transposing reads are done before its rows are replaced
    wave_lds_fence();
#pragma unroll
    for (int tg = 0; tg < 2; ++tg)
#pragma unroll
      for (int s = 0; s < NS; ++s)
        *reinterpret_cast<bf16x8_t*>(kb + (16 * tg + c) * PITCH + (32 * s + 8 * g) * 2) = kf[tg][s];
    // validity of token 16 tg + j sits in bit j of the ballot (lanes 0..15 hold j = c)
    const uint32_t vm0 = (uint32_t)(__ballot(val[0]) & 0xFFFFu), vm1 = (uint32_t)(__ballot(val[1]) & 0xFFFFu);
    f32x4_t st[2];
#pragma unroll
    for (int tg = 0; tg < 2; ++tg) {
      st[tg] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < NS; ++s) st[tg] = mfma_bf16_16x16x32(kf[tg][s], qf[s], st[tg]);
    }
    float sv[2][4], bmax = -INFINITY;
#pragma unroll
    for (int tg = 0; tg < 2; ++tg)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool v = (((tg ? vm1 : vm0) >> (4 * g + r)) & 1u) != 0;
        sv[tg][r] = v ? st[tg][r] * scale : -INFINITY;
        bmax = fmaxf(bmax, sv[tg][r]);
      }
    bmax = lane_xor_max(bmax);
    const float mn = fmaxf(m, bmax);
    const float alpha = mn == -INFINITY ? 1.f : __expf(m - mn);
    float p[2][4], psum = 0.f;
#pragma unroll
    for (int tg = 0; tg < 2; ++tg)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[tg][r] = mn == -INFINITY ? 0.f : __expf(sv[tg][r] - mn);
        psum += p[tg][r];
      }
    psum = lane_xor_sum(psum);
    l = l * alpha + psum;
    m = mn;
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[j] *= alpha;
    // B of the value product: P^T, k = 8 g + i <-> token (i < 4 ? 4 g + i : 16 + 4 g + i - 4)
    const bf16x2_t p01 = __builtin_convertvector(f32x2_t{p[0][0], p[0][1]}, bf16x2_t);
    const bf16x2_t p23 = __builtin_convertvector(f32x2_t{p[0][2], p[0][3]}, bf16x2_t);
    const bf16x2_t p45 = __builtin_convertvector(f32x2_t{p[1][0], p[1][1]}, bf16x2_t);
    const bf16x2_t p67 = __builtin_convertvector(f32x2_t{p[1][2], p[1][3]}, bf16x2_t);
    const bf16x8_t pb = {p01[0], p01[1], p23[0], p23[1], p45[0], p45[1], p67[0], p67[1]};
    wave_lds_fence();  // the block's rows are in LDS before any lane reads them transposed
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      // A: V^T rows 16 j + c: lane (g, c) receives tokens 4 g .. 4 g + 3 (lo) and
      // 16 + 4 g .. + 3 (hi) at dim 16 j + c; its address is row R + c / 4,
      // dims 16 j + 4 (c % 4) .. + 4 of that row
      const uint8_t* base = kb + (4 * g + (c >> 2)) * PITCH + (16 * j + 4 * (c & 3)) * 2;
      const v4s_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s_t*)(base));
      const v4s_t hi =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s_t*)(base + 16 * PITCH));
      const v8s_t a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      acc[j] = mfma_bf16_16x16x32(__builtin_bit_cast(bf16x8_t, a), pb, acc[j]);
    }
  }
  // merge the waves: O^T tiles as [wave][dim][head] floats in the staging space
  __syncthreads();
  float* ob = reinterpret_cast<float*>(kst);
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) ob[((int64_t)w * D + 16 * j + 4 * g + r) * 16 + c] = acc[j][r];
  if (g == 0) {
    mls[w][0][c] = m;
    mls[w][1][c] = l;
  }
  __syncthreads();
  float mw[4], M = -INFINITY;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    mw[v] = mls[v][0][c];
    M = fmaxf(M, mw[v]);
  }
  float fw[4], L = 0.f;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    fw[v] = mw[v] == -INFINITY ? 0.f : __expf(mw[v] - M);
    L += mls[v][1][c] * fw[v];
  }
  if (sink && M != -INFINITY) L += __expf(sink[16 * ht + c] - M);
  const float inv = L > 0.f ? 1.f / L : 0.f;
  uint16_t* orow = o + ((int64_t)row * H + 16 * ht + c) * D;
  for (int j = w; j < NJ; j += 4) {
    float v4[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = 0.f;
#pragma unroll
      for (int v_ = 0; v_ < 4; ++v_) v += ob[((int64_t)v_ * D + 16 * j + 4 * g + r) * 16 + c] * fw[v_];
      v4[r] = v * inv;
    }
    uint2 pk;
    pk.x = (uint32_t)f32_bf16(v4[0]) | ((uint32_t)f32_bf16(v4[1]) << 16);
    pk.y = (uint32_t)f32_bf16(v4[2]) | ((uint32_t)f32_bf16(v4[3]) << 16);
    *reinterpret_cast<uint2*>(orow + 16 * j + 4 * g) = pk;
  }
}

template <int D>
int launch_sparse_attn(const uint16_t* q, const uint16_t* kv, const int32_t* idx, const float* sink, uint16_t* o,
                       int64_t rows, int64_t h, int64_t n, int64_t t, int64_t rows_per_kv, float scale,
                       hipStream_t st) {
  MOSAIC_LAUNCH((sparse_attn_kernel<D>), dim3((unsigned)rows, (unsigned)(h / 16)), dim3(256), 0, st, q, kv, idx,
                sink, o, (int)h, (int)t, n, (int)rows_per_kv, scale);
  MOSAIC_RETURN_LAUNCH("sparse_attn_bf16");
}

}  // namespace
}  // namespace mosaic

using namespace mosaic;

extern "C" int mosaic_sparse_attn_bf16(const uint16_t* q, const uint16_t* kv, const float* sink, const int32_t* idx,
                                       uint16_t* out, int64_t rows, int64_t h, int64_t n, int64_t topk, int64_t d,
                                       int64_t rows_per_kv, float softmax_scale, void* stream) {
  MOSAIC_CHECK_ARG(q && kv && idx && out, "sparse_attn_bf16: null pointer");
  MOSAIC_CHECK_ARG(d == 64 || d == 128 || d == 256, "sparse_attn_bf16: head dim %lld (64, 128 or 256)",
                   (long long)d);
  MOSAIC_CHECK_ARG(h >= 16 && h % 16 == 0 && h / 16 <= 65535, "sparse_attn_bf16: heads %lld (a multiple of 16)",
                   (long long)h);
  MOSAIC_CHECK_ARG(rows >= 0 && rows < (1ll << 31) && n >= 1 && n < (1ll << 31) && topk >= 0 && topk < (1ll << 30),
                   "sparse_attn_bf16: shape out of range");
  MOSAIC_CHECK_ARG(rows_per_kv >= 1 && rows % rows_per_kv == 0, "sparse_attn_bf16: %lld rows in groups of %lld",
                   (long long)rows, (long long)rows_per_kv);
  if (rows == 0) return kOk;
  hipStream_t st = (hipStream_t)stream;
  switch (d) {
    case 64: return launch_sparse_attn<64>(q, kv, idx, sink, out, rows, h, n, topk, rows_per_kv, softmax_scale, st);
    case 128:
      return launch_sparse_attn<128>(q, kv, idx, sink, out, rows, h, n, topk, rows_per_kv, softmax_scale, st);
    default:
      return launch_sparse_attn<256>(q, kv, idx, sink, out, rows, h, n, topk, rows_per_kv, softmax_scale, st);
  }
}
