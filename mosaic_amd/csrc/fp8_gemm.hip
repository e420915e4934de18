// FP8 e4m3 block-scaled GEMM on gfx950 (upstream fp8_gemm contract):
//   C[m, n] = sum over 128-K blocks kb of (A_kb . B_kb^T) * a_s[m, kb] * b_s[n/128, kb]
// with fp32 scales of any value (not powers of two), fp32 accumulation and a
// bf16 or fp32 output.  Each 128-K block is one v_mfma_scale_f32_16x16x128
// (fp8 x fp8, unit e8m0 scales); its fp32 block product is rescaled by
// a_s * b_s and added to a separate fp32 accumulator, as the upstream kernel
// keeps C_local and C_local_accum apart.
//
// Skinny kernel (M <= 64 per launch row of tiles): a wave owns 16 tokens x
// T*16 output columns and walks its K slice; the KS waves of a workgroup take
// consecutive K slices and meet in LDS.  Operand layout: lane l (c = l%16,
// q = l/16) holds bytes [16q, 16q+16) and [64+16q, 64+16q+16) of the 128-byte
// K block of row c, for both operands (same lane->K map on both sides).
#include "common.h"
#include "../../include/mosaic_amd.h"

namespace mosaic {

// unit-scale fp8 x fp8 block product of one 128-K block
__device__ __forceinline__ f32x4_t mfma_fp8_block(const i32x8_t a, const i32x8_t b) {
  const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 127, 0, 127);
}

template <int T, int KS>
__global__ void __launch_bounds__(KS * 64) fp8_gemm_skinny_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ B,
    const float* __restrict__ Bs, void* __restrict__ C, int M, int N, int K, int out_f32) {
  __shared__ f32x4_t red[KS][T][64];
  const int lane = threadIdx.x & 63, ks = threadIdx.x >> 6;
  const int c = lane & 15, q = lane >> 4;
  const int n0 = blockIdx.x * 16 * T, m0 = blockIdx.y * 16;
  const int nkb = K / 128;
  const int kb0 = nkb * ks / KS, kb1 = nkb * (ks + 1) / KS;
  const bool avalid = (m0 + c) < M;
  const uint8_t* arow = A + (int64_t)(avalid ? m0 + c : 0) * K;
  const uint8_t* brow[T];
  const float* bsrow[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int n = min(n0 + 16 * t + c, N - 1);
    brow[t] = B + (int64_t)n * K;
    bsrow[t] = Bs + (int64_t)(min(n0 + 16 * t, N - 1) / 128) * nkb;
  }
  const float* asrow[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) asrow[r] = As + (int64_t)min(m0 + 4 * q + r, M - 1) * nkb;
  f32x4_t acc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  constexpr int U = 2;
  int kb = kb0;
  for (; kb < kb1; kb += U) {
    i32x8_t bv[U][T], av[U];
    float sa[U][4], sb[U][T];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = min(kb + u, kb1 - 1);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        bv[u][t] = load_fp8_operand_nt(brow[t], k, q);
        sb[u][t] = bsrow[t][k];
      }
      av[u] = avalid ? load_fp8_operand(arow, k, q) : i32x8_t{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int r = 0; r < 4; ++r) sa[u][r] = asrow[r][k];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (kb + u < kb1) {
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const f32x4_t d = mfma_fp8_block(av[u], bv[u][t]);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[t][r] = __builtin_fmaf(d[r], sa[u][r] * sb[u][t], acc[t][r]);
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < T; ++t) red[ks][t][lane] = acc[t];
  __syncthreads();
  if (ks < T) {
    const int t = ks;
    f32x4_t v = red[0][t][lane];
    for (int k2 = 1; k2 < KS; ++k2) v += red[k2][t][lane];
    const int n = n0 + 16 * t + c;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m0 + 4 * q + r;
      if (m < M && n < N) {
        if (out_f32)
          reinterpret_cast<float*>(C)[(int64_t)m * N + n] = v[r];
        else
          reinterpret_cast<uint16_t*>(C)[(int64_t)m * N + n] = f32_bf16(v[r]);
      }
    }
  }
}

template <int T, int KS>
static void launch_fp8_skinny(const uint8_t* a, const float* as, const uint8_t* b, const float* bs, void* c,
                              int64_t m, int64_t n, int64_t k, int out_f32, hipStream_t st) {
  dim3 grid((unsigned)((n + 16 * T - 1) / (16 * T)), (unsigned)((m + 15) / 16));
  hipLaunchKernelGGL((fp8_gemm_skinny_kernel<T, KS>), grid, dim3(KS * 64), 0, st, a, as, b, bs, c, (int)m, (int)n,
                     (int)k, out_f32);
}

// w [N, K] e4m3 with one fp32 scale per (bn x bk) block -> bf16 [N, K]
__global__ void __launch_bounds__(256) fp8_block_dequant_kernel(const uint8_t* __restrict__ w,
                                                                const float* __restrict__ s,
                                                                uint16_t* __restrict__ out, int64_t n, int64_t k,
                                                                int bn, int bk, int64_t sk) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i >= n * k) return;
  const int64_t row = i / k, col = i % k;
  const float sc = s[(row / bn) * sk + col / bk];
  const uint32_t v = *reinterpret_cast<const uint32_t*>(w + i);
  const f32x2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)v, false);
  const f32x2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)v, true);
  uint16_t* o = out + i;
  o[0] = f32_bf16(lo[0] * sc);
  o[1] = f32_bf16(lo[1] * sc);
  o[2] = f32_bf16(hi[0] * sc);
  o[3] = f32_bf16(hi[1] * sc);
}

}  // namespace mosaic

using namespace mosaic;

extern "C" int mosaic_fp8_block_dequant(const uint8_t* w, const float* s, uint16_t* out, int64_t n, int64_t k,
                                        int block_n, int block_k, void* stream) {
  MOSAIC_CHECK_ARG(w && s && out, "fp8_block_dequant: null pointer");
  MOSAIC_CHECK_ARG(n >= 0 && k > 0 && k % 4 == 0 && block_n > 0 && block_k > 0 && block_k % 4 == 0,
                   "fp8_block_dequant: K=%lld, block %dx%d", (long long)k, block_n, block_k);
  if (n == 0) return kOk;
  const int64_t total = n * k / 4;
  hipLaunchKernelGGL(fp8_block_dequant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, w, s, out, n, k, block_n, block_k, (k + block_k - 1) / block_k);
  MOSAIC_RETURN_LAUNCH("fp8_block_dequant");
}

extern "C" int mosaic_fp8_block_gemm(const uint8_t* a, const float* a_s, const uint8_t* b, const float* b_s, void* c,
                                     int out_dtype, int64_t m, int64_t n, int64_t k, void* stream) {
  MOSAIC_CHECK_ARG(a && a_s && b && b_s && c, "fp8_block_gemm: null pointer");
  MOSAIC_CHECK_ARG(k > 0 && k % 128 == 0, "fp8_block_gemm: K=%lld must be a positive multiple of 128",
                   (long long)k);
  MOSAIC_CHECK_ARG(m >= 0 && n >= 0 && m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 31),
                   "fp8_block_gemm: shape out of range");
  MOSAIC_CHECK_ARG(out_dtype == MOSAIC_DTYPE_F32 || out_dtype == MOSAIC_DTYPE_BF16, "fp8_block_gemm: out dtype %d",
                   out_dtype);
  if (m == 0 || n == 0) return kOk;
  hipStream_t st = (hipStream_t)stream;
  const int f32 = out_dtype == MOSAIC_DTYPE_F32;
  const int64_t mt = (m + 15) / 16;
  // columns per wave chosen so the grid covers the chip (>= ~2048 waves)
  if (((n + 63) / 64) * mt * 8 >= 4096)
    launch_fp8_skinny<4, 8>(a, a_s, b, b_s, c, m, n, k, f32, st);
  else if (((n + 31) / 32) * mt * 8 >= 4096)
    launch_fp8_skinny<2, 8>(a, a_s, b, b_s, c, m, n, k, f32, st);
  else
    launch_fp8_skinny<1, 8>(a, a_s, b, b_s, c, m, n, k, f32, st);
  MOSAIC_RETURN_LAUNCH("fp8_block_gemm");
}
