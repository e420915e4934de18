// A8 MXFP4 path ("source semantics") on gfx950: e4m3 activations with a
// power-of-two scale per 1x128 block against MXFP4 weights (E2M1 + e8m0 per
// 32 K) on v_mfma_scale_f32_16x16x128_f8f6f4.  Both scales are powers of two,
// so they go straight into the MFMA's e8m0 operands: the activation scale of
// a lane's 32 K values is the exponent byte of its 1x128 scale, the weight
// scale is the MXT16 scale byte selected by opsel.  Nothing is dequantized
// and no VALU rescale is needed; the MFMA accumulates in fp32.
//
// MFMA operands of super-step S (128 K): lane l (c = l%16, q = l/16) holds
//   A: e4m3 of token row c at K [128S + 16q, +16) and [128S + 64 + 16q, +16)
//      (the MFMA's 8-bit operand order: two 16-byte loads),
//   B: the MXT16 16-byte block (row c, MX block 4S+q) = K [128S + 32q, +32)
//      (the 4-bit operand order: one 16-byte load, low nibble first).
// The activation scale is constant over a super-step, so which lane supplies
// it for which 32-K block does not matter.
#include <algorithm>

#include "common.h"
#include "moe_internal.h"
#include "../../include/mosaic_amd.h"

namespace mosaic {

// e8m0 byte of a power-of-two fp32 scale (its biased exponent)
// A power-of-two fp32 activation scale as its e8m0 byte.  Any other value (a
// mantissa bit or the sign set) maps to 0xFF, the e8m0 NaN, so the scaled MFMA
// turns the affected outputs into NaN instead of silently using a rounded scale.
__device__ __forceinline__ int pow2_e8m0(float s) {
  const uint32_t u = __float_as_uint(s);
  return (u & 0x807FFFFFu) ? 0xFF : (int)(u >> 23);
}

template <int SEL>
__device__ __forceinline__ f32x4_t mfma_a8(const i32x8_t a, int sa, const u32x4_t w, uint32_t sw, f32x4_t acc) {
  const i32x8_t b = {(int)w[0], (int)w[1], (int)w[2], (int)w[3], 0, 0, 0, 0};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc, 0, 4, 0, sa, SEL, (int)sw);
}

__device__ __forceinline__ i32x8_t load_a8_operand(const uint8_t* __restrict__ xrow, int S, int q) {
  const u32x4_t lo = *reinterpret_cast<const u32x4_t*>(xrow + 128 * S + 16 * q);
  const u32x4_t hi = *reinterpret_cast<const u32x4_t*>(xrow + 128 * S + 64 + 16 * q);
  return i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

// 4 super-steps [S, S+4) of T column tiles (S % 4 == 0)
template <int T>
__device__ __forceinline__ void a8_group(const uint8_t* const (&wt)[T], const uint8_t* const (&st)[T],
                                         const uint8_t* __restrict__ xrow, const float* __restrict__ sarow,
                                         bool xvalid, int q, int S, f32x4_t (&acc)[T]) {
  u32x4_t wv[4][T];
  uint32_t sv[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
#pragma unroll
    for (int u = 0; u < 4; ++u) wv[u][t] = load_nt_u32x4(wt[t] + (int64_t)(S + u) * 1024);
    sv[t] = *reinterpret_cast<const uint32_t*>(st[t] + (int64_t)(S >> 2) * 256);
  }
  i32x8_t av[4];
  int sa[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    av[u] = xvalid ? load_a8_operand(xrow, S + u, q) : i32x8_t{0, 0, 0, 0, 0, 0, 0, 0};
    sa[u] = xvalid ? pow2_e8m0(sarow[S + u]) : 127;
  }
#pragma unroll
  for (int t = 0; t < T; ++t) {
    acc[t] = mfma_a8<0>(av[0], sa[0], wv[0][t], sv[t], acc[t]);
    acc[t] = mfma_a8<1>(av[1], sa[1], wv[1][t], sv[t], acc[t]);
    acc[t] = mfma_a8<2>(av[2], sa[2], wv[2][t], sv[t], acc[t]);
    acc[t] = mfma_a8<3>(av[3], sa[3], wv[3][t], sv[t], acc[t]);
  }
}

template <int T>
__device__ __forceinline__ void a8_step(const uint8_t* const (&wt)[T], const uint8_t* const (&st)[T],
                                        const uint8_t* __restrict__ xrow, const float* __restrict__ sarow,
                                        bool xvalid, int q, int S, f32x4_t (&acc)[T]) {
  const i32x8_t av = xvalid ? load_a8_operand(xrow, S, q) : i32x8_t{0, 0, 0, 0, 0, 0, 0, 0};
  const int sa = xvalid ? pow2_e8m0(sarow[S]) : 127;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const u32x4_t w = load_nt_u32x4(wt[t] + (int64_t)S * 1024);
    const uint32_t s4 = *reinterpret_cast<const uint32_t*>(st[t] + (int64_t)(S >> 2) * 256);
    const uint32_t sw = (s4 >> (8 * (S & 3))) & 0xFFu;  // the byte moved to position 0
    acc[t] = mfma_a8<0>(av, sa, w, sw, acc[t]);
  }
}

template <int T>
__device__ __forceinline__ void tile_dot_a8(const uint8_t* const (&wt)[T], const uint8_t* const (&st)[T],
                                            const uint8_t* __restrict__ xrow, const float* __restrict__ sarow,
                                            bool xvalid, int q, int s0, int s1, f32x4_t (&acc)[T]) {
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  int S = s0;
  for (; S + 4 <= s1; S += 4) a8_group<T>(wt, st, xrow, sarow, xvalid, q, S, acc);
  for (; S < s1; ++S) a8_step<T>(wt, st, xrow, sarow, xvalid, q, S, acc);
}

__device__ __forceinline__ void a8_k_slice(int ns, int ks, int KS, int& s0, int& s1) {
  const int ng = ns / 4;
  s0 = 4 * (ng * ks / KS);
  s1 = (ks == KS - 1) ? ns : 4 * (ng * (ks + 1) / KS);
}

__device__ __forceinline__ void a8_ptrs(const uint8_t* pt, const uint8_t* st, int64_t g, int ns, int lane,
                                        const uint8_t*& w, const uint8_t*& s) {
  const int ns4 = (ns + 3) / 4;
  w = pt + (g * ns * 64 + lane) * 16;
  s = st + (g * ns4 * 64 + lane) * 4;
}

// ------------------------------------------------------- single linear -----
// y [M, N] bf16 = A8 linear of (xq e4m3 [M, K], sa f32 pow2 [M, K/128]) with an
// MXT16 weight.  grid (N/(16T), ceil(M/16)), KS waves = K slices.
template <int T, int KS>
__global__ void __launch_bounds__(KS * 64) mx_linear_a8_kernel(const uint8_t* __restrict__ xq,
                                                                const float* __restrict__ sa,
                                                                const uint8_t* __restrict__ packed_t,
                                                                const uint8_t* __restrict__ scale_t,
                                                                uint16_t* __restrict__ y, int M, int N, int K) {
  __shared__ f32x4_t red[KS][T][64];
  const int lane = threadIdx.x & 63, ks = threadIdx.x >> 6;
  const int c = lane & 15, q = lane >> 4;
  const int n0 = blockIdx.x * 16 * T, m0 = blockIdx.y * 16;
  const int ns = K / 128;
  const bool xvalid = (m0 + c) < M;
  const int xr = xvalid ? m0 + c : 0;
  const uint8_t* wt[T];
  const uint8_t* st[T];
#pragma unroll
  for (int t = 0; t < T; ++t) a8_ptrs(packed_t, scale_t, min(n0 / 16 + t, N / 16 - 1), ns, lane, wt[t], st[t]);
  int s0, s1;
  a8_k_slice(ns, ks, KS, s0, s1);
  f32x4_t acc[T];
  tile_dot_a8<T>(wt, st, xq + (int64_t)xr * K, sa + (int64_t)xr * ns, xvalid, q, s0, s1, acc);
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
      const int mi = m0 + 4 * q + r;
      if (mi < M && n < N) y[(int64_t)mi * N + n] = f32_bf16(v[r]);
    }
  }
}

// Decode-shaped A8 linear (M <= 16): a workgroup owns 16 T columns and its KS
// waves take K slices of whole 4-step groups; each wave streams its steps
// through a register ring of D entries (the T tiles' 1 KB MXT16 code blocks
// and scale dwords, the A operand and its 1x128 scale), issued D steps ahead.
// Steps past the wave's slice reload its last step with a zero A operand, so
// the loop has no branches.  A step's operands pass through empty volatile
// asm statements and the loads are pinned in slot order, so the compiler's
// waits keep the ring full.  The K slices meet in LDS in wave order.
template <int T, int KS, int D>
__global__ void __launch_bounds__(KS * 64) mx_gemv_a8_kernel(const uint8_t* __restrict__ xq,
                                                              const float* __restrict__ sa,
                                                              const uint8_t* __restrict__ packed_t,
                                                              const uint8_t* __restrict__ scale_t,
                                                              uint16_t* __restrict__ y, int M, int N, int K) {
  __shared__ f32x4_t red[KS][T][64];
  const int lane = threadIdx.x & 63, ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, q = lane >> 4;
  const int n0 = blockIdx.x * 16 * T;
  const int ns = K / 128;
  const uint8_t* wt[T];
  const uint8_t* st[T];
#pragma unroll
  for (int t = 0; t < T; ++t) a8_ptrs(packed_t, scale_t, min(n0 / 16 + t, N / 16 - 1), ns, lane, wt[t], st[t]);
  int s0, s1;
  a8_k_slice(ns, ks, KS, s0, s1);
  const int nb = s1 - s0;
  const bool xvalid = c < M;
  const uint8_t* xrow = xq + (int64_t)(xvalid ? c : 0) * K;
  const float* sarow = sa + (int64_t)(xvalid ? c : 0) * ns;
  u32x4_t rw[D][T], rx[D][2];
  uint32_t rs[D][T];
  float ra[D];
  auto load = [&](int s, int i) {
    const int S = s0 + (i < nb ? i : nb - 1);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      rw[s][t] = load_nt_u32x4(wt[t] + (int64_t)S * 1024);
      rs[s][t] = *reinterpret_cast<const uint32_t*>(st[t] + (int64_t)(S >> 2) * 256);
    }
    rx[s][0] = *reinterpret_cast<const u32x4_t*>(xrow + 128 * S + 16 * q);
    rx[s][1] = *reinterpret_cast<const u32x4_t*>(xrow + 128 * S + 64 + 16 * q);
    ra[s] = sarow[S];
  };
  f32x4_t acc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int s, int i) {
    const int S = s0 + i;
    asm volatile("" : "+v"(rx[s][0]), "+v"(rx[s][1]), "+v"(ra[s]));
    const bool real = i < nb && xvalid;
    const u32x4_t lo = real ? rx[s][0] : u32x4_t{0u, 0u, 0u, 0u};
    const u32x4_t hi = real ? rx[s][1] : u32x4_t{0u, 0u, 0u, 0u};
    const i32x8_t av = {(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    const int sav = real ? pow2_e8m0(ra[s]) : 127;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      asm volatile("" : "+v"(rw[s][t]), "+v"(rs[s][t]));
      const uint32_t sw = (rs[s][t] >> (8 * (S & 3))) & 0xFFu;
      acc[t] = mfma_a8<0>(av, sav, rw[s][t], sw, acc[t]);
    }
  };
  const int nchunks = (nb + D - 1) / D;
  if (nb > 0) {
#pragma unroll
    for (int s = 0; s < D; ++s) {
      load(s, s);
      asm volatile("" ::: "memory");  // in slot order: the compiler's waits count the later loads
    }
    for (int ch = 0; ch + 1 < nchunks; ++ch) {
#pragma unroll
      for (int s = 0; s < D; ++s) {
        compute(s, ch * D + s);
        load(s, ch * D + s + D);
        asm volatile("" ::: "memory");
      }
    }
#pragma unroll
    for (int s = 0; s < D; ++s) compute(s, (nchunks - 1) * D + s);
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
      const int mi = 4 * q + r;
      if (mi < M && n < N) y[(int64_t)mi * N + n] = f32_bf16(v[r]);
    }
  }
}

// ring plans: few column tiles -> K split 8 ways, more -> 4 or 2 (as the FP8 decode ring)
template <int T, int KS>
static void launch_gemv_a8(const uint8_t* xq, const float* sa, const uint8_t* pt, const uint8_t* st, uint16_t* y,
                           int64_t m, int64_t n, int64_t k, hipStream_t s) {
  const dim3 grid((unsigned)((n + 16 * T - 1) / (16 * T)));
  // 8-deep ring where the wave has at least 8 steps (7 or 6 deep, dividing the
  // steps, measured 5-30% slower)
  const int nb = (int)(k / 128 / KS);
  if (nb >= 8)
    MOSAIC_LAUNCH((mx_gemv_a8_kernel<T, KS, 8>), grid, dim3(KS * 64), 0, s, xq, sa, pt, st, y, (int)m, (int)n, (int)k);
  else
    MOSAIC_LAUNCH((mx_gemv_a8_kernel<T, KS, 4>), grid, dim3(KS * 64), 0, s, xq, sa, pt, st, y, (int)m, (int)n, (int)k);
}

template <int T, int KS>
static void launch_linear_a8(const uint8_t* xq, const float* sa, const uint8_t* pt, const uint8_t* st, uint16_t* y,
                             int64_t m, int64_t n, int64_t k, hipStream_t s) {
  dim3 grid((unsigned)((n + 16 * T - 1) / (16 * T)), (unsigned)((m + 15) / 16));
  MOSAIC_LAUNCH((mx_linear_a8_kernel<T, KS>), grid, dim3(KS * 64), 0, s, xq, sa, pt, st, y, (int)m, (int)n,
                     (int)k);
}

// ---------------------------------------------------- MoE (A8 contract) ----
// fused_moe_mxint semantics (kernels/mxint.py:1587-1722): the gate/up GEMM
// output is a bf16 tensor, SwiGLU runs in fp32 on those bf16 values, the route
// weight scales z before the bf16 cast, z is re-quantized 1x128 pow2 e4m3 for
// the down GEMM, whose output rows are bf16 partials summed in fp32 in
// ascending expert id.
template <int T, int KS>
__global__ void __launch_bounds__(KS * 64) moe_a8_gateup_kernel(
    const uint8_t* __restrict__ xq, const float* __restrict__ xs, const uint8_t* __restrict__ gu_p,
    const uint8_t* __restrict__ gu_s, const uint8_t* __restrict__ sh_p, const uint8_t* __restrict__ sh_s,
    const int32_t* __restrict__ tile_expert, const int32_t* __restrict__ tile_rows,
    const int32_t* __restrict__ tile_p0, const int32_t* __restrict__ n_tiles, const int32_t* __restrict__ perm_token,
    const float* __restrict__ perm_weight, uint16_t* __restrict__ z, int H, int I, int E, float limit) {
  __shared__ f32x4_t red[KS][T][64];
  const int tile = blockIdx.y;
  if (tile >= n_tiles[0]) return;
  const int e = tile_expert[tile], rows = tile_rows[tile], p0 = tile_p0[tile];
  const int lane = threadIdx.x & 63, ks = threadIdx.x >> 6;
  const int c = lane & 15, q = lane >> 4;
  const int j0 = blockIdx.x * 8 * T;
  const int ns = H / 128, ns4 = (ns + 3) / 4;
  const int64_t ebytes = (int64_t)2 * I * (H / 2), sbytes = (int64_t)(2 * I / 16) * ns4 * 256;
  const uint8_t* bp = (e == E) ? sh_p : gu_p + (int64_t)e * ebytes;
  const uint8_t* bs = (e == E) ? sh_s : gu_s + (int64_t)e * sbytes;
  const uint8_t* wt[T];
  const uint8_t* st[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int g = (t < T / 2) ? (j0 / 16 + t) : ((I + j0) / 16 + t - T / 2);
    a8_ptrs(bp, bs, g, ns, lane, wt[t], st[t]);
  }
  const bool xvalid = c < rows;
  const int tok = xvalid ? perm_token[p0 + c] : 0;
  int s0, s1;
  a8_k_slice(ns, ks, KS, s0, s1);
  f32x4_t acc[T];
  tile_dot_a8<T>(wt, st, xq + (int64_t)tok * H, xs + (int64_t)tok * ns, xvalid, q, s0, s1, acc);
#pragma unroll
  for (int t = 0; t < T; ++t) red[ks][t][lane] = acc[t];
  __syncthreads();
  if (ks < T / 2) {
    const int t = ks;
    f32x4_t g = red[0][t][lane], u = red[0][t + T / 2][lane];
#pragma unroll
    for (int k2 = 1; k2 < KS; ++k2) {
      g += red[k2][t][lane];
      u += red[k2][t + T / 2][lane];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int ti = 4 * q + r;
      if (ti < rows) {
        const float gb = bf16_f32(f32_bf16(g[r])), ub = bf16_f32(f32_bf16(u[r]));
        const float zv = swiglu_f32(gb, ub, limit) * perm_weight[p0 + ti];
        z[(int64_t)(p0 + ti) * I + j0 + 16 * t + c] = f32_bf16(zv);
      }
    }
  }
}

template <int T, int KS>
__global__ void __launch_bounds__(KS * 64) moe_a8_down_kernel(
    const uint8_t* __restrict__ zq, const float* __restrict__ zs, const uint8_t* __restrict__ d_p,
    const uint8_t* __restrict__ d_s, const uint8_t* __restrict__ sh_p, const uint8_t* __restrict__ sh_s,
    const int32_t* __restrict__ tile_expert, const int32_t* __restrict__ tile_rows,
    const int32_t* __restrict__ tile_p0, const int32_t* __restrict__ n_tiles, float* __restrict__ yp, int H, int I,
    int E) {
  __shared__ f32x4_t red[KS][T][64];
  const int tile = blockIdx.y;
  if (tile >= n_tiles[0]) return;
  const int e = tile_expert[tile], rows = tile_rows[tile], p0 = tile_p0[tile];
  const int lane = threadIdx.x & 63, ks = threadIdx.x >> 6;
  const int c = lane & 15, q = lane >> 4;
  const int h0 = blockIdx.x * 16 * T;
  const int ns = I / 128, ns4 = (ns + 3) / 4;
  const int64_t ebytes = (int64_t)H * (I / 2), sbytes = (int64_t)(H / 16) * ns4 * 256;
  const uint8_t* bp = (e == E) ? sh_p : d_p + (int64_t)e * ebytes;
  const uint8_t* bs = (e == E) ? sh_s : d_s + (int64_t)e * sbytes;
  const uint8_t* wt[T];
  const uint8_t* st[T];
#pragma unroll
  for (int t = 0; t < T; ++t) a8_ptrs(bp, bs, h0 / 16 + t, ns, lane, wt[t], st[t]);
  const bool xvalid = c < rows;
  const int row = p0 + (xvalid ? c : 0);
  int s0, s1;
  a8_k_slice(ns, ks, KS, s0, s1);
  f32x4_t acc[T];
  tile_dot_a8<T>(wt, st, zq + (int64_t)row * I, zs + (int64_t)row * ns, xvalid, q, s0, s1, acc);
#pragma unroll
  for (int t = 0; t < T; ++t) red[ks][t][lane] = acc[t];
  __syncthreads();
  if (ks < T) {
    const int t = ks;
    f32x4_t v = red[0][t][lane];
#pragma unroll
    for (int k2 = 1; k2 < KS; ++k2) v += red[k2][t][lane];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int ti = 4 * q + r;
      if (ti < rows) yp[(int64_t)(p0 + ti) * H + h0 + 16 * t + c] = bf16_f32(f32_bf16(v[r]));
    }
  }
}

// ------------------------------------------------------ prefill (A8) ------
// Large batches: tiles of 256 sorted assignment rows of one expert, a
// workgroup of 8 waves per (tile, 16 weight groups of 16 rows).  Per 128-K
// step the workgroup stages in LDS the e4m3 rows of its tokens (256 rows of
// 128 bytes, 16-byte chunks XOR-swizzled by (row >> 1) & 7, copied as runs of
// 8 whole rows) and the MXT16 weight blocks (1 KB per group, already in lane
// order); the weight scale dwords and the rows' activation scales move once
// per 4 steps into two chunk buffers.  Everything moves global -> LDS directly
// (global_load_lds) through a ring of three stages, two steps ahead of the
// MFMAs.  The copies are issued from inline asm with explicit vmcnt waits and
// a bare s_barrier: the compiler then neither waits for the in-flight stages
// before each LDS read (which it does for copies it knows about) nor needs
// staging registers.  Each wave owns 64 rows x 8 groups and accumulates
// straight into its MFMA accumulators: both scales are e8m0 operands of
// v_mfma_scale, so there is no per-step VALU rescale.  Tiles of at most 64
// rows take the light-tile path below.
constexpr int kPfBM = 256;     // sorted rows per tile
constexpr int kPfWaves = 8;    // 4 row quarters x 2 column halves
constexpr int kPfStages = 3;
constexpr int kPfNG = 16;      // weight groups (16 rows each) per workgroup
constexpr int kPfA = 0, kPfB = 32768;
constexpr int kPfStage = kPfB + kPfNG * 1024;  // A rows and weight blocks of one step
// Scales move per 4 steps ("chunk", two buffers): the weight scale dwords
// (one dword per lane and group covers 4 steps) and the rows' 1x128 scales,
// 16 bytes (4 steps) per row, so the row-scale gather touches each row's
// line once per 4 steps instead of once per step.
constexpr int kPfCBs = 0, kPfCAs = kPfNG * 256, kPfChunk = kPfCAs + kPfBM * 16;
// copies per wave per step: its A runs holding tile rows (0..4, 8 rows each)
// and 2 weight runs; on steps 4c also the chunk: 2 weight-scale runs and
// (waves 0..3) one 16-byte row-scale run

__device__ __forceinline__ uint32_t lds_u32(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ void lds_copy16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(__builtin_amdgcn_readfirstlane(lds)),
               "v"(g) : "memory", "m0");
}
__device__ __forceinline__ void lds_copy4(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off" ::"s"(__builtin_amdgcn_readfirstlane(lds)),
               "v"(g) : "memory", "m0");
}

// Tile coordinates of a 1-D grid of n_col x ceil8(n_tile) workgroups: the
// dispatcher deals workgroups round-robin to the 8 XCDs, so ids that share
// id % 8 run on one XCD; all column tiles of a row tile get the same id % 8 and
// share that XCD's L2 copy of the tile's activation rows.
__device__ __forceinline__ void pf_coords(int id, int n_col, int& col, int& tile) {
  col = (id / 8) % n_col;
  tile = (id % 8) + 8 * (id / (8 * n_col));
}

// this lane's sources for the wave's copy runs of one stage (add the step offsets)
struct PfSrc {
  const uint8_t* a[4];   // A run 4 wv + i: rows 8 (4 wv + i) .. + 7, this lane's 16-byte chunk (swizzled)
  const uint8_t* b[2];   // weight group 2 wv + i, this lane's 16 bytes
  const uint8_t* bs[2];  // its scale dword
  const float* as;       // row 64 (wv & 3) + lane: its 1x128 scale row (waves 0..3)
};

// copies of one step by this wave (see pf_issue)
__device__ __forceinline__ int pf_ops(int S, int n_a, int wv) { return n_a + 2 + ((S & 3) == 0 ? (wv < 4 ? 3 : 2) : 0); }

// A runs 4 wv + i (8 rows each) past the tile's rows are not copied (no wave
// computes on them); n_a is 0..4, uniform over the wave.  Steps 4c also copy
// chunk c (into chunk buffer c & 1).
__device__ __forceinline__ void pf_issue(const PfSrc& src, int S, uint8_t* stage, uint8_t* chunk, int n_a) {
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t base = lds_u32(stage);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (i < n_a) lds_copy16(src.a[i] + 128 * S, base + kPfA + (4 * wv + i) * 1024);
#pragma unroll
  for (int i = 0; i < 2; ++i) lds_copy16(src.b[i] + (int64_t)S * 1024, base + kPfB + (2 * wv + i) * 1024);
  if ((S & 3) == 0) {
    const uint32_t cb = lds_u32(chunk + ((S >> 2) & 1) * kPfChunk);
#pragma unroll
    for (int i = 0; i < 2; ++i) lds_copy4(src.bs[i] + (int64_t)(S >> 2) * 256, cb + kPfCBs + (2 * wv + i) * 256);
    if (wv < 4) lds_copy16(src.as + S, cb + kPfCAs + wv * 1024);
  }
}

// One wave's MFMAs of one staged step: its row tiles (rows 64 (wv >> 1) + 16 mt,
// the first MT of them: the tiles past the workgroup's valid rows are skipped)
// x the 8 staged groups in wg.
template <int MT>
__device__ __forceinline__ void pf_compute(const uint8_t* stage, const uint8_t* chunk, const int (&wg)[8], int S,
                                           f32x4_t (&acc)[4][8]) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, c = lane & 15;
  const int sh = 8 * (S & 3);
  i32x8_t a[MT];
  int sa[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int mtg = 4 * (wv >> 1) + mt;
    // row r of the tile is 128 bytes at r * 128, its 16-byte chunks XOR-swizzled by (r >> 1) & 7
    const int row = 16 * mtg + c, swz = (row >> 1) & 7, q = lane >> 4;
    const uint8_t* rp = stage + kPfA + row * 128;
    const u32x4_t lo = *reinterpret_cast<const u32x4_t*>(rp + ((q ^ swz) << 4));
    const u32x4_t hi = *reinterpret_cast<const u32x4_t*>(rp + (((q + 4) ^ swz) << 4));
    a[mt] = i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    sa[mt] = pow2_e8m0(*reinterpret_cast<const float*>(chunk + kPfCAs + (16 * mtg + c) * 16 + (S & 3) * 4));
  }
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    const u32x4_t wb = *reinterpret_cast<const u32x4_t*>(stage + kPfB + wg[n] * 1024 + lane * 16);
    const int sw = (int)((*reinterpret_cast<const uint32_t*>(chunk + kPfCBs + wg[n] * 256 + lane * 4) >> sh) & 0xFFu);
    const i32x8_t b = {(int)wb[0], (int)wb[1], (int)wb[2], (int)wb[3], 0, 0, 0, 0};
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      acc[mt][n] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[mt], b, acc[mt][n], 0, 4, 0, sa[mt], 0, sw);
  }
}

// row tiles of this wave that hold valid rows (0..4), uniform over the wave
__device__ __forceinline__ int pf_live_tiles(int rows) {
  const int wv = threadIdx.x >> 6;
  const int r = rows - 64 * (wv >> 1);
  return r <= 0 ? 0 : (r >= 64 ? 4 : (r + 15) / 16);
}

// wait until this wave has at most `ops` copies in flight, then the workgroup barrier
template <int N>
__device__ __forceinline__ void pf_wait_n() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}
__device__ __forceinline__ void pf_wait_ops(int ops) {
  switch (ops) {
    case 9: pf_wait_n<9>(); break;
    case 8: pf_wait_n<8>(); break;
    case 7: pf_wait_n<7>(); break;
    case 6: pf_wait_n<6>(); break;
    case 5: pf_wait_n<5>(); break;
    case 4: pf_wait_n<4>(); break;
    case 3: pf_wait_n<3>(); break;
    case 2: pf_wait_n<2>(); break;
    case 1: pf_wait_n<1>(); break;
    default: pf_wait_n<0>(); break;
  }
}

template <int LIVE>
__device__ __forceinline__ void pf_kloop_t(const PfSrc& src, int ns, const int (&wg)[8], f32x4_t (&acc)[4][8],
                                           uint8_t (*ring)[kPfStage], uint8_t* chunk, int n_a, int wv) {
  for (int S = 0; S < ns; ++S) {
    // step S landed (every wave's copies: the barrier), step S + 1 may still fly
    pf_wait_ops(S + 1 < ns ? pf_ops(S + 1, n_a, wv) : 0);
    // the step's MFMAs first, then step S + 2's copies (slot (S + 2) % 3 was
    // step S - 1's, which every wave finished before the barrier above)
    if constexpr (LIVE > 0) pf_compute<LIVE>(ring[S % kPfStages], chunk + ((S >> 2) & 1) * kPfChunk, wg, S, acc);
    if (S + 2 < ns) pf_issue(src, S + 2, ring[(S + 2) % kPfStages], chunk, n_a);
  }
}

__device__ __forceinline__ void pf_kloop(const PfSrc& src, int ns, int rows, const int (&wg)[8],
                                         f32x4_t (&acc)[4][8], uint8_t (*ring)[kPfStage], uint8_t* chunk) {
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int n = 0; n < 8; ++n) acc[mt][n] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // A runs of this wave: rows 32 wv + 8 i .. + 7 (i < 4), those holding tile rows
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n_a = min(4, max(0, (rows - 32 * wv + 7) / 8));
  pf_issue(src, 0, ring[0], chunk, n_a);
  if (ns > 1) pf_issue(src, 1, ring[1], chunk, n_a);
  // the wave's row tiles past the valid rows are skipped (one loop per count)
  switch (pf_live_tiles(rows)) {
    case 4: pf_kloop_t<4>(src, ns, wg, acc, ring, chunk, n_a, wv); break;
    case 3: pf_kloop_t<3>(src, ns, wg, acc, ring, chunk, n_a, wv); break;
    case 2: pf_kloop_t<2>(src, ns, wg, acc, ring, chunk, n_a, wv); break;
    case 1: pf_kloop_t<1>(src, ns, wg, acc, ring, chunk, n_a, wv); break;
    default: pf_kloop_t<0>(src, ns, wg, acc, ring, chunk, n_a, wv); break;
  }
}

// this lane's copy sources; rows past the tile's end read the tile's first row
// (their results are never stored)
__device__ __forceinline__ void pf_sources(PfSrc& src, const uint8_t* const (&rowp)[4], const uint8_t* bank_p,
                                           const uint8_t* bank_s, const int (&groups)[2], int ns, const float* as_row) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < 4; ++i) {  // run 4 wv + i: row rowp[i] (row 32 wv + 8 i + lane / 8), chunk swizzled
    const int row = 32 * (threadIdx.x >> 6) + 8 * i + (lane >> 3);
    src.a[i] = rowp[i] + 16 * ((lane & 7) ^ ((row >> 1) & 7));
  }
  const int ns4 = (ns + 3) / 4;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    src.b[i] = bank_p + ((int64_t)groups[i] * ns) * 1024 + lane * 16;
    src.bs[i] = bank_s + ((int64_t)groups[i] * ns4) * 256 + lane * 4;
  }
  src.as = as_row;
}

// ---- light tiles (at most 64 rows): weight streaming -------------------------
// A tile of <= 64 rows does a quarter of the MFMAs of a full one for the same
// weight bytes, so its time is the weight stream's: what matters is how many
// weight bytes are in flight.  Such tiles stage only their 64 rows (8 KB) with
// the 16 weight groups (16 KB) and scales: a 28.3 KB stage, five stages, four
// steps ahead (64 KB of weights in flight per CU instead of 32 KB).  Every wave
// then owns two staged groups and the tile's (up to 4) 16-row tiles.
constexpr int kPfLStages = 5;
constexpr int kPfLA = 0, kPfLB = 8192, kPfLBs = kPfLB + kPfNG * 1024, kPfLAs = kPfLBs + kPfNG * 256;
constexpr int kPfLStage = kPfLAs + 256;
// copies per wave per stage: 1 A run, 2 weight runs, 2 scale runs, and (wave 0) 1 row-scale run
static_assert(kPfLStages * kPfLStage <= kPfStages * kPfStage, "light ring must fit the prefill ring");

struct PfLSrc {
  const uint8_t* a;      // A run wv: rows 8 wv .. + 7 (row 8 wv + lane / 8), this lane's 16-byte chunk (swizzled)
  const uint8_t* b[2];   // weight group 2 wv + i, this lane's 16 bytes
  const uint8_t* bs[2];  // its scale dword
  const float* as;       // row lane: its 1x128 scale row
};

__device__ __forceinline__ void pfl_issue(const PfLSrc& src, int S, uint8_t* stage) {
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t base = lds_u32(stage);
  lds_copy16(src.a + 128 * S, base + kPfLA + wv * 1024);
#pragma unroll
  for (int i = 0; i < 2; ++i) lds_copy16(src.b[i] + (int64_t)S * 1024, base + kPfLB + (2 * wv + i) * 1024);
#pragma unroll
  for (int i = 0; i < 2; ++i) lds_copy4(src.bs[i] + (int64_t)(S >> 2) * 256, base + kPfLBs + (2 * wv + i) * 256);
  if (wv == 0) lds_copy4(src.as + S, base + kPfLAs);  // wave 0 copies the 64 row scales
}

// wait until this wave has `ahead` later stages in flight, then the barrier
__device__ __forceinline__ void pfl_wait(int ahead, int wv) {
  if (wv == 0) {
    if (ahead >= 3) pf_wait_n<18>(); else if (ahead == 2) pf_wait_n<12>(); else if (ahead == 1) pf_wait_n<6>(); else pf_wait_n<0>();
  } else {
    if (ahead >= 3) pf_wait_n<15>(); else if (ahead == 2) pf_wait_n<10>(); else if (ahead == 1) pf_wait_n<5>(); else pf_wait_n<0>();
  }
}

// one wave's MFMAs of one staged step: 16-row tiles 0..MT-1 x staged groups ga, gb
template <int MT>
__device__ __forceinline__ void pfl_compute(const uint8_t* stage, int ga, int gb, int S, f32x4_t (&acc)[4][2]) {
  const int lane = threadIdx.x & 63, c = lane & 15;
  const int sh = 8 * (S & 3);
  i32x8_t a[MT];
  int sa[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    // row r at r * 128, 16-byte chunks XOR-swizzled by (r >> 1) & 7
    const int row = 16 * mt + c, swz = (row >> 1) & 7, q = lane >> 4;
    const uint8_t* rp = stage + kPfLA + row * 128;
    const u32x4_t lo = *reinterpret_cast<const u32x4_t*>(rp + ((q ^ swz) << 4));
    const u32x4_t hi = *reinterpret_cast<const u32x4_t*>(rp + (((q + 4) ^ swz) << 4));
    a[mt] = i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    sa[mt] = pow2_e8m0(*reinterpret_cast<const float*>(stage + kPfLAs + (16 * mt + c) * 4));
  }
#pragma unroll
  for (int gi = 0; gi < 2; ++gi) {
    const int g = gi ? gb : ga;
    const u32x4_t wb = *reinterpret_cast<const u32x4_t*>(stage + kPfLB + g * 1024 + lane * 16);
    const int sw = (int)((*reinterpret_cast<const uint32_t*>(stage + kPfLBs + g * 256 + lane * 4) >> sh) & 0xFFu);
    const i32x8_t b = {(int)wb[0], (int)wb[1], (int)wb[2], (int)wb[3], 0, 0, 0, 0};
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      acc[mt][gi] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[mt], b, acc[mt][gi], 0, 4, 0, sa[mt], 0, sw);
  }
}

template <int MT>
__device__ __forceinline__ void pfl_kloop_t(const PfLSrc& src, int ns, int ga, int gb, f32x4_t (&acc)[4][2],
                                            uint8_t* ring) {
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  for (int S = 0; S < ns; ++S) {
    pfl_wait(min(kPfLStages - 2, ns - 1 - S), wv);  // step S landed, later issued steps may fly
    // the step's MFMAs go out first: a wave stalls at a copy until the address
    // unit takes it, and issued MFMAs keep running meanwhile
    pfl_compute<MT>(ring + (S % kPfLStages) * kPfLStage, ga, gb, S, acc);
    if (S + kPfLStages - 1 < ns)
      pfl_issue(src, S + kPfLStages - 1, ring + ((S + kPfLStages - 1) % kPfLStages) * kPfLStage);
  }
}

__device__ __forceinline__ void pfl_kloop(const PfLSrc& src, int ns, int rows, int ga, int gb, f32x4_t (&acc)[4][2],
                                          uint8_t* ring) {
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) acc[mt][0] = acc[mt][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int st = 0; st < kPfLStages - 1 && st < ns; ++st) pfl_issue(src, st, ring + st * kPfLStage);
  switch ((rows + 15) / 16) {
    case 4: pfl_kloop_t<4>(src, ns, ga, gb, acc, ring); break;
    case 3: pfl_kloop_t<3>(src, ns, ga, gb, acc, ring); break;
    case 2: pfl_kloop_t<2>(src, ns, ga, gb, acc, ring); break;
    default: pfl_kloop_t<1>(src, ns, ga, gb, acc, ring); break;
  }
}

// light-tile copy sources: A run wv is rows 8 wv .. + 7, lane l row 8 wv + l / 8
// (rows past the tile's end read its first row; their results are never stored)
__device__ __forceinline__ void pfl_sources(PfLSrc& src, const uint8_t* rowp, const uint8_t* bank_p,
                                            const uint8_t* bank_s, const int (&groups)[2], int ns,
                                            const float* as_row) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int row = 8 * wv + (lane >> 3);
  src.a = rowp + 16 * ((lane & 7) ^ ((row >> 1) & 7));
  const int ns4 = (ns + 3) / 4;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    src.b[i] = bank_p + ((int64_t)groups[i] * ns) * 1024 + lane * 16;
    src.bs[i] = bank_s + ((int64_t)groups[i] * ns4) * 256 + lane * 4;
  }
  src.as = as_row;
}

// gate/up + SwiGLU: 1-D grid of (I / 128) x ceil8(tiles); z [A, I] bf16 in
// sorted order.  Staged groups: 0..7 gate (z columns j0 + 16 g), 8..15 up;
// wave (rows 64 (wv >> 1), z columns j0 + 64 (wv & 1)) owns gate groups
// 4 (wv & 1) + n and the matching up groups.
__global__ void __launch_bounds__(kPfWaves * 64, 1) moe_a8_gateup_prefill_kernel(
    const uint8_t* __restrict__ xq, const float* __restrict__ xs, const uint8_t* __restrict__ gu_p,
    const uint8_t* __restrict__ gu_s, const uint8_t* __restrict__ sh_p, const uint8_t* __restrict__ sh_s,
    const int32_t* __restrict__ tile_expert, const int32_t* __restrict__ tile_rows,
    const int32_t* __restrict__ tile_p0, const int32_t* __restrict__ n_tiles, const int32_t* __restrict__ perm_token,
    const float* __restrict__ perm_weight, uint8_t* __restrict__ zq, float* __restrict__ zs, int H, int I, int E,
    float limit) {
  __shared__ __attribute__((aligned(16))) uint8_t ring[kPfStages][kPfStage];
  __shared__ __attribute__((aligned(16))) uint8_t chunk[2 * kPfChunk];
  int colt, tile;
  pf_coords(blockIdx.x, I / 128, colt, tile);
  if (tile >= n_tiles[0]) return;
  const int e = tile_expert[tile], rows = tile_rows[tile], p0 = tile_p0[tile];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, c = lane & 15, q = lane >> 4;
  const int j0 = colt * 128;
  const int ns = H / 128, ns4 = (ns + 3) / 4;
  const int64_t ebytes = (int64_t)2 * I * (H / 2), sbytes = (int64_t)(2 * I / 16) * ns4 * 256;
  const uint8_t* bp = (e == E) ? sh_p : gu_p + (int64_t)e * ebytes;
  const uint8_t* bsc = (e == E) ? sh_s : gu_s + (int64_t)e * sbytes;
  int groups[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int g = 2 * wv + i;
    groups[i] = g < 8 ? j0 / 16 + g : (I + j0) / 16 + g - 8;
  }
  const int nbk = I / 128;
  if (rows <= 64) {
    // light tile: wave wv owns gate group wv and up group 8 + wv (z columns j0 + 16 wv)
    const int arow = 8 * wv + (lane >> 3);
    PfLSrc lsrc;
    pfl_sources(lsrc, xq + (int64_t)perm_token[p0 + (arow < rows ? arow : 0)] * H, bp, bsc, groups, ns,
                xs + (int64_t)perm_token[p0 + (lane < rows ? lane : 0)] * ns);
    const float wl = perm_weight[p0 + (lane < rows ? lane : 0)];  // row lane's route weight
    f32x4_t lacc[4][2];
    uint8_t* lring = &ring[0][0];
    pfl_kloop(lsrc, ns, rows, wv, 8 + wv, lacc, lring);
    uint32_t lmax[4][4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * mt + 4 * q + r;
        const float wgt = __shfl(wl, row, 64);
        const float gb = bf16_round_hw(lacc[mt][0][r]), ub = bf16_round_hw(lacc[mt][1][r]);
        const float zb = bf16_round_hw(swiglu_fast_f32(gb, ub, limit) * wgt);
        lacc[mt][0][r] = zb;
        uint32_t u = __float_as_uint(fabsf(zb));
        u = max(u, MOSAIC_DPP(0u, u, 0xB1, 0xF));
        u = max(u, MOSAIC_DPP(0u, u, 0x4E, 0xF));
        u = max(u, MOSAIC_DPP(0u, u, 0x141, 0xF));
        u = max(u, MOSAIC_DPP(0u, u, 0x140, 0xF));
        lmax[mt][r] = u;
      }
    // the 1x128 block of a row spans the 8 waves' 16 columns: row maxima through the idle ring
    __syncthreads();
    uint32_t* pam = reinterpret_cast<uint32_t*>(lring);  // [8 waves][64 rows]
    if (c == 0) {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) pam[wv * 64 + 16 * mt + 4 * q + r] = lmax[mt][r];
    }
    __syncthreads();
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * mt + 4 * q + r;
        uint32_t um = pam[row];
#pragma unroll
        for (int w2 = 1; w2 < 8; ++w2) um = max(um, pam[w2 * 64 + row]);
        const float sc = act_scale_pow2(__uint_as_float(um));
        if (row < rows) {
          const int64_t pp = p0 + row;
          const float y = fminf(fmaxf(lacc[mt][0][r] * (1.0f / sc), -448.0f), 448.0f);  // sc = 2^e: exact
          zq[pp * I + j0 + 16 * wv + c] = (uint8_t)e4m3_hw(y);
          if (wv == 0 && c == 0) zs[pp * nbk + j0 / 128] = sc;
        }
      }
    return;
  }
  const uint8_t* rowp[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 32 * wv + 8 * i + (lane >> 3);
    rowp[i] = xq + (int64_t)perm_token[p0 + (row < rows ? row : 0)] * H;
  }
  const int srow = 64 * (wv & 3) + lane;
  const float* as_row = xs + (int64_t)perm_token[p0 + (srow < rows ? srow : 0)] * ns;
  PfSrc src;
  pf_sources(src, rowp, bp, bsc, groups, ns, as_row);
  const int hc = wv & 1;
  int wg[8];
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    wg[n] = 4 * hc + n;
    wg[n + 4] = 8 + 4 * hc + n;
  }
  // route weight of the wave's row 64 (wv >> 1) + lane: one load, read back by
  // lane shuffles (the epilogue's per-row loads each waited out a full memory
  // round trip)
  const int wrow = 64 * (wv >> 1) + lane;
  const float wl = perm_weight[p0 + (wrow < rows ? wrow : 0)];
  f32x4_t acc[4][8];
  pf_kloop(src, ns, rows, wg, acc, ring, chunk);
  // z = bf16(SwiGLU(bf16 gate, bf16 up) * route weight) in acc[mt][n][r], and
  // the amax of each row over this wave's 64 columns (DPP max over the 16
  // lanes of the row, on the bits of non-negative floats).  The roundings use
  // the hardware converters: 64 values a lane made the software ones (with
  // their divergent branches) a quarter of the workgroup's time.
  uint32_t rmax[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float wgt = __shfl(wl, 16 * mt + 4 * q + r, 64);  // row 64 (wv >> 1) + 16 mt + 4 q + r
      float m = 0.f;
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const float gb = bf16_round_hw(acc[mt][n][r]), ub = bf16_round_hw(acc[mt][n + 4][r]);
        const float zb = bf16_round_hw(swiglu_fast_f32(gb, ub, limit) * wgt);
        acc[mt][n][r] = zb;
        m = fmaxf(m, fabsf(zb));
      }
      uint32_t u = __float_as_uint(m);
      u = max(u, MOSAIC_DPP(0u, u, 0xB1, 0xF));
      u = max(u, MOSAIC_DPP(0u, u, 0x4E, 0xF));
      u = max(u, MOSAIC_DPP(0u, u, 0x141, 0xF));
      u = max(u, MOSAIC_DPP(0u, u, 0x140, 0xF));
      rmax[mt][r] = u;
    }
  // the 1x128 quantization block of a row spans this wave's columns and those
  // of wave wv ^ 1: exchange the row maxima through the (now idle) ring
  __syncthreads();
  uint32_t* pam = reinterpret_cast<uint32_t*>(&ring[0][0]);  // [8 waves][64 rows]
  if (c == 0) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) pam[wv * 64 + 16 * mt + 4 * q + r] = rmax[mt][r];
  }
  __syncthreads();
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 64 * (wv >> 1) + 16 * mt + 4 * q + r;
      const float amax = __uint_as_float(max(rmax[mt][r], pam[(wv ^ 1) * 64 + 16 * mt + 4 * q + r]));
      const float sc = act_scale_pow2(amax);
      if (row < rows) {
        const int64_t pp = p0 + row;
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          const float y = fminf(fmaxf(acc[mt][n][r] * (1.0f / sc), -448.0f), 448.0f);  // sc = 2^e: exact
          zq[pp * I + j0 + 64 * hc + 16 * n + c] = (uint8_t)e4m3_hw(y);
        }
        if (hc == 0 && c == 0) zs[pp * nbk + j0 / 128] = sc;
      }
    }
}

// down: 1-D grid of (H / 256) x ceil8(tiles); bf16 partial rows yb [A, H] in
// sorted order.  Wave (rows 64 (wv >> 1), columns h0 + 128 (wv & 1)).
__global__ void __launch_bounds__(kPfWaves * 64, 1) moe_a8_down_prefill_kernel(
    const uint8_t* __restrict__ zq, const float* __restrict__ zs, const uint8_t* __restrict__ d_p,
    const uint8_t* __restrict__ d_s, const uint8_t* __restrict__ sh_p, const uint8_t* __restrict__ sh_s,
    const int32_t* __restrict__ tile_expert, const int32_t* __restrict__ tile_rows,
    const int32_t* __restrict__ tile_p0, const int32_t* __restrict__ n_tiles, uint16_t* __restrict__ yb, int H,
    int I, int E) {
  __shared__ __attribute__((aligned(16))) uint8_t ring[kPfStages][kPfStage];
  __shared__ __attribute__((aligned(16))) uint8_t chunk[2 * kPfChunk];
  int colt, tile;
  pf_coords(blockIdx.x, H / 256, colt, tile);
  if (tile >= n_tiles[0]) return;
  const int e = tile_expert[tile], rows = tile_rows[tile], p0 = tile_p0[tile];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, c = lane & 15, q = lane >> 4;
  const int h0 = colt * 256;
  const int ns = I / 128, ns4 = (ns + 3) / 4;
  const int64_t ebytes = (int64_t)H * (I / 2), sbytes = (int64_t)(H / 16) * ns4 * 256;
  const uint8_t* bp = (e == E) ? sh_p : d_p + (int64_t)e * ebytes;
  const uint8_t* bsc = (e == E) ? sh_s : d_s + (int64_t)e * sbytes;
  const int groups[2] = {h0 / 16 + 2 * wv, h0 / 16 + 2 * wv + 1};
  if (rows <= 64) {
    // light tile: wave wv owns staged groups 2 wv and 2 wv + 1 (columns h0 + 32 wv)
    const int arow = 8 * wv + (lane >> 3);
    PfLSrc lsrc;
    pfl_sources(lsrc, zq + (int64_t)(p0 + (arow < rows ? arow : 0)) * I, bp, bsc, groups, ns,
                zs + (int64_t)(p0 + (lane < rows ? lane : 0)) * ns);
    f32x4_t lacc[4][2];
    pfl_kloop(lsrc, ns, rows, 2 * wv, 2 * wv + 1, lacc, &ring[0][0]);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int gi = 0; gi < 2; ++gi)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 16 * mt + 4 * q + r;
          if (row < rows) yb[(int64_t)(p0 + row) * H + h0 + 32 * wv + 16 * gi + c] = f32_bf16_hw(lacc[mt][gi][r]);
        }
    return;
  }
  const uint8_t* rowp[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 32 * wv + 8 * i + (lane >> 3);
    rowp[i] = zq + (int64_t)(p0 + (row < rows ? row : 0)) * I;
  }
  const int srow = 64 * (wv & 3) + lane;
  const float* as_row = zs + (int64_t)(p0 + (srow < rows ? srow : 0)) * ns;
  PfSrc src;
  pf_sources(src, rowp, bp, bsc, groups, ns, as_row);
  const int hc = wv & 1;
  int wg[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) wg[n] = 8 * hc + n;
  f32x4_t acc[4][8];
  pf_kloop(src, ns, rows, wg, acc, ring, chunk);
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int n = 0; n < 8; ++n)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 64 * (wv >> 1) + 16 * mt + 4 * q + r;
        if (row < rows) yb[(int64_t)(p0 + row) * H + h0 + 128 * hc + 16 * n + c] = f32_bf16_hw(acc[mt][n][r]);
      }
}

// ------------------------------------------------------- dense A8 GEMM -----
// y [M, N] = A8 linear of (xq e4m3 [M, K] + pow2 scales sa [M, K/128]) with one
// MXT16 weight, on the staged scaled-MFMA loops of the prefill kernels: tiles of
// `tr` rows (64: the light-tile loop; 256: the full-tile loop, or the light one
// when a tile holds at most 64 rows) x 256 columns, and K split into `splits`
// slices of whole 512-K chunks.  Unsplit, a tile stores bf16 y; split, it stores
// fp32 partials part[slice][M][N] that mx_gemm_a8_reduce_kernel sums in slice
// order.  The columns of the last tile past N read the last weight group and
// are not stored.
struct DenseA8Plan {
  int tr, n_row, n_col, splits, row_fastest;
};

// Workgroup id -> (row tile, column tile, K slice).  The dispatcher deals ids
// round-robin to the 8 XCDs (id % 8), so each XCD takes one contiguous run of
// the linear work order: with the row tile fastest, the row tiles of one
// (column tile, slice) share the XCD's L2 copy of that weight slice; otherwise
// the order walks pairs of row tiles column by column, so the workgroups an
// XCD runs at once cover a block of 2 row tiles x a run of column tiles and
// share both operands' slices in its L2 (M = 4096: 18432 x 7168 from 536-540
// to 517-519 us and 7168 x 16384 from 491-494 to 472-473 us against the plain
// column-fastest order).  Every XCD gets work however few row tiles there are.
__device__ __forceinline__ bool dense_coords(int id, int nwork, int per_xcd, const DenseA8Plan& p, int& rt, int& ct,
                                             int& ks) {
  const int lin = (id % 8) * per_xcd + id / 8;
  if (lin >= nwork) return false;
  const int per_ks = p.n_row * p.n_col;
  ks = lin / per_ks;
  const int l = lin % per_ks;
  if (p.row_fastest) {
    rt = l % p.n_row;
    ct = l / p.n_row;
  } else {
    constexpr int GM = 2;  // row tiles per group
    const int r0 = l / (GM * p.n_col) * GM, gr = min(p.n_row - r0, GM), w = l % (GM * p.n_col);
    rt = r0 + w % gr;
    ct = w / gr;
  }
  return true;
}

__global__ void __launch_bounds__(kPfWaves * 64, 1) mx_gemm_a8_kernel(
    const uint8_t* __restrict__ xq, const float* __restrict__ sa, const uint8_t* __restrict__ pt,
    const uint8_t* __restrict__ st, uint16_t* __restrict__ y, float* __restrict__ part, int M, int N, int K,
    DenseA8Plan plan, int per_xcd) {
  __shared__ __attribute__((aligned(16))) uint8_t ring[kPfStages][kPfStage];
  __shared__ __attribute__((aligned(16))) uint8_t chunk[2 * kPfChunk];
  int rt, ct, ks;
  if (!dense_coords(blockIdx.x, plan.n_row * plan.n_col * plan.splits, per_xcd, plan, rt, ct, ks)) return;
  const int p0 = rt * plan.tr, rows = min(plan.tr, M - p0);
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, c = lane & 15, q = lane >> 4;
  const int h0 = ct * 256;
  const int ns = K / 128, nch = ns / 4;
  // this slice's steps [s0, s0 + nsl): whole 4-step chunks, so the chunked
  // scale copies of the loops stay aligned; the sources start at s0
  const int s0 = 4 * (nch * ks / plan.splits), nsl = 4 * (nch * (ks + 1) / plan.splits) - s0;
  const int ng = N / 16;
  const int groups[2] = {min(h0 / 16 + 2 * wv, ng - 1), min(h0 / 16 + 2 * wv + 1, ng - 1)};
  float* pslice = part ? part + (int64_t)ks * M * N : nullptr;
  if (rows <= 64) {
    // light tile: wave wv owns staged groups 2 wv and 2 wv + 1 (columns h0 + 32 wv)
    const int arow = 8 * wv + (lane >> 3);
    PfLSrc lsrc;
    pfl_sources(lsrc, xq + (int64_t)(p0 + (arow < rows ? arow : 0)) * K, pt, st, groups, ns,
                sa + (int64_t)(p0 + (lane < rows ? lane : 0)) * ns);
    lsrc.a += 128 * s0;
    lsrc.as += s0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      lsrc.b[i] += (int64_t)s0 * 1024;
      lsrc.bs[i] += (int64_t)(s0 / 4) * 256;
    }
    f32x4_t lacc[4][2];
    pfl_kloop(lsrc, nsl, rows, 2 * wv, 2 * wv + 1, lacc, &ring[0][0]);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int gi = 0; gi < 2; ++gi) {
        const int col = h0 + 32 * wv + 16 * gi + c;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 16 * mt + 4 * q + r;
          if (row < rows && col < N) {
            const int64_t o = (int64_t)(p0 + row) * N + col;
            if (pslice)
              pslice[o] = lacc[mt][gi][r];
            else
              y[o] = f32_bf16_hw(lacc[mt][gi][r]);
          }
        }
      }
    return;
  }
  const uint8_t* rowp[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 32 * wv + 8 * i + (lane >> 3);
    rowp[i] = xq + (int64_t)(p0 + (row < rows ? row : 0)) * K;
  }
  const int srow = 64 * (wv & 3) + lane;
  const float* as_row = sa + (int64_t)(p0 + (srow < rows ? srow : 0)) * ns;
  PfSrc src;
  pf_sources(src, rowp, pt, st, groups, ns, as_row);
#pragma unroll
  for (int i = 0; i < 4; ++i) src.a[i] += 128 * s0;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    src.b[i] += (int64_t)s0 * 1024;
    src.bs[i] += (int64_t)(s0 / 4) * 256;
  }
  src.as += s0;
  const int hc = wv & 1;
  int wg[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) wg[n] = 8 * hc + n;
  f32x4_t acc[4][8];
  pf_kloop(src, nsl, rows, wg, acc, ring, chunk);
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      const int col = h0 + 128 * hc + 16 * n + c;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 64 * (wv >> 1) + 16 * mt + 4 * q + r;
        if (row < rows && col < N) {
          const int64_t o = (int64_t)(p0 + row) * N + col;
          if (pslice)
            pslice[o] = acc[mt][n][r];
          else
            y[o] = f32_bf16_hw(acc[mt][n][r]);
        }
      }
    }
}

// y = bf16 of the sum of the S fp32 partial slices, in slice order
__global__ void __launch_bounds__(256) mx_gemm_a8_reduce_kernel(const float* __restrict__ part, int S, int64_t mn,
                                                                uint16_t* __restrict__ y) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= mn) return;  // mn % 4 == 0 (N % 16 == 0)
  f32x4_t v = *reinterpret_cast<const f32x4_t*>(part + i);
  for (int sl = 1; sl < S; ++sl) v += *reinterpret_cast<const f32x4_t*>(part + (int64_t)sl * mn + i);
  uint2 o;
  o.x = (uint32_t)f32_bf16(v[0]) | ((uint32_t)f32_bf16(v[1]) << 16);
  o.y = (uint32_t)f32_bf16(v[2]) | ((uint32_t)f32_bf16(v[3]) << 16);
  *reinterpret_cast<uint2*>(y + i) = o;
}

// The dense plan: the staged kernel holds one workgroup per CU (160 KB of LDS),
// so a plan aims at one round of at most 256 workgroups.  Up to 256 rows the
// tiles are mostly 64 rows (the light loop streams the weight at the full per-CU rate
// and the row tiles of a weight slice share it in L2); above, 256 rows (the
// full loop does four times the MFMAs per staged weight byte).  K is split
// while the tiles cover at most half of the CUs, at most 8 ways and into whole
// 512-K chunks; the weight is then re-read by fewer workgroups than rows would
// need.  Small-M plans keep the row tiles of one weight slice on one XCD (row
// tile fastest), large-M plans the column tiles of one activation slice.
static DenseA8Plan dense_a8_plan_tr(int64_t m, int64_t n, int64_t k, int tr) {
  DenseA8Plan p;
  p.tr = tr;
  p.n_row = (int)((m + p.tr - 1) / p.tr);
  p.n_col = (int)((n + 255) / 256);
  const int tiles = p.n_row * p.n_col, nch = (int)(k / 512);
  p.splits = 1;
  if (tiles * 2 <= 256) p.splits = std::max(1, std::min({8, nch, 256 / tiles}));
  p.row_fastest = p.tr == 64 ? 1 : 0;
  return p;
}
static DenseA8Plan dense_a8_plan(int64_t m, int64_t n, int64_t k) {
  if (m > 256) return dense_a8_plan_tr(m, n, k, 256);
  // up to 256 rows: 64-row tiles, unless they leave over a third of the CUs idle
  // and one 256-row tile per column (split further) fills more of them
  // (128 x 18432 x 7168: 144 workgroups at 44.4 us, 216 at 40.5 us)
  const DenseA8Plan p64 = dense_a8_plan_tr(m, n, k, 64), p256 = dense_a8_plan_tr(m, n, k, 256);
  const int w64 = p64.n_row * p64.n_col * p64.splits, w256 = p256.n_row * p256.n_col * p256.splits;
  return (w64 < 160 && w256 > w64 && w256 <= 256) ? p256 : p64;
}

// the staged dense kernel runs when K is whole 512-K chunks and the rows are
// not decode-sized (up to 32 rows the 16-row kernel streams the weight once per
// 16 rows, which is at most twice)
static bool dense_a8_staged(int64_t m, int64_t n, int64_t k) { return m > 32 && k % 512 == 0 && m < (1 << 30); }

static size_t dense_a8_ws_bytes(int64_t m, int64_t n, int64_t k) {
  if (!dense_a8_staged(m, n, k)) return 0;
  const DenseA8Plan p = dense_a8_plan(m, n, k);
  return p.splits > 1 ? (size_t)p.splits * (size_t)m * (size_t)n * 4 : 0;
}

// y[t][h] = bf16(sum over j of yb[combine_pos[t][j]][h]), bf16 partials; a
// thread sums 8 consecutive columns (16-byte loads), in ascending j.  W <=
// kCombineMaxW: every partial load is issued before the in-order sum.
__global__ void __launch_bounds__(128) moe_combine_bf16_kernel(const uint16_t* __restrict__ yb,
                                                               const int32_t* __restrict__ combine_pos,
                                                               uint16_t* __restrict__ y, int M, int W, int H) {
  const int t = blockIdx.y;
  const int h = 8 * (blockIdx.x * blockDim.x + threadIdx.x);
  if (t >= M || h >= H) return;
  u32x4_t pv[kCombineMaxW];
  bool ok[kCombineMaxW];
#pragma unroll
  for (int j = 0; j < kCombineMaxW; ++j) {
    const int p = j < W ? combine_pos[(int64_t)t * W + j] : -1;
    ok[j] = p >= 0;
    pv[j] = ok[j] ? *reinterpret_cast<const u32x4_t*>(yb + (int64_t)p * H + h) : u32x4_t{0u, 0u, 0u, 0u};
  }
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < kCombineMaxW; ++j) {
    if (!ok[j]) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s[2 * i] += bf16_f32((uint16_t)(pv[j][i] & 0xFFFFu));
      s[2 * i + 1] += bf16_f32((uint16_t)(pv[j][i] >> 16));
    }
  }
  u32x4_t o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = (uint32_t)f32_bf16(s[2 * i]) | ((uint32_t)f32_bf16(s[2 * i + 1]) << 16);
  *reinterpret_cast<u32x4_t*>(y + (int64_t)t * H + h) = o;
}

}  // namespace mosaic

using namespace mosaic;

static int mxt16_linear_a8_impl(const uint8_t* xq, const float* sa, const uint8_t* packed_t, const uint8_t* scale_t,
                                uint16_t* y, int64_t m, int64_t n, int64_t k, void* workspace, size_t workspace_bytes,
                                void* stream) {
  MOSAIC_CHECK_ARG(xq && sa && packed_t && scale_t && y, "mxt16_linear_a8: null pointer");
  MOSAIC_CHECK_ARG(k > 0 && k % 128 == 0, "mxt16_linear_a8: K=%lld must be a positive multiple of 128",
                   (long long)k);
  MOSAIC_CHECK_ARG(n > 0 && n % 16 == 0, "mxt16_linear_a8: N=%lld must be a positive multiple of 16", (long long)n);
  MOSAIC_CHECK_ARG(m >= 0 && m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 31),
                   "mxt16_linear_a8: shape out of range");
  if (m == 0) return kOk;
  hipStream_t st = (hipStream_t)stream;
  if (dense_a8_staged(m, n, k) && m * n < (1ll << 40)) {
    DenseA8Plan plan = dense_a8_plan(m, n, k);
    float* part = nullptr;
    if (plan.splits > 1) {
      if (workspace && workspace_bytes >= dense_a8_ws_bytes(m, n, k))
        part = (float*)workspace;
      else
        plan.splits = 1;  // no workspace: the unsplit plan
    }
    const int nwork = plan.n_row * plan.n_col * plan.splits;
    const int per_xcd = (nwork + 7) / 8;
    MOSAIC_LAUNCH(mx_gemm_a8_kernel, dim3((unsigned)(8 * per_xcd)), dim3(kPfWaves * 64), 0, st, xq, sa, packed_t,
                  scale_t, y, part, (int)m, (int)n, (int)k, plan, per_xcd);
    MOSAIC_LAUNCH_CHECK("mxt16_linear_a8_staged");
    if (part) {
      const int64_t mn = m * n;
      MOSAIC_LAUNCH(mx_gemm_a8_reduce_kernel, dim3((unsigned)((mn / 4 + 255) / 256)), dim3(256), 0, st, part,
                    plan.splits, mn, y);
    }
    MOSAIC_RETURN_LAUNCH("mxt16_linear_a8_reduce");
  }
  const int64_t mt = (m + 15) / 16;
  // one row: the ring kernel (18432 x 7168: 18.6 -> 17.0 us, 24576 x 1536: 7.9 ->
  // 6.4 us); from two rows the 16-row kernel's shared A operand wins on some shapes
  if (m == 1) {
    const int64_t t16 = n / 16;
    if (t16 <= 256)
      launch_gemv_a8<1, 8>(xq, sa, packed_t, scale_t, y, m, n, k, st);
    else if (t16 <= 1152)
      launch_gemv_a8<1, 4>(xq, sa, packed_t, scale_t, y, m, n, k, st);
    else
      launch_gemv_a8<1, 2>(xq, sa, packed_t, scale_t, y, m, n, k, st);
    MOSAIC_RETURN_LAUNCH("mxt16_linear_a8");
  }
  if (((n + 63) / 64) * mt * 8 >= 4096)
    launch_linear_a8<4, 8>(xq, sa, packed_t, scale_t, y, m, n, k, st);
  else if (((n + 31) / 32) * mt * 8 >= 4096)
    launch_linear_a8<2, 8>(xq, sa, packed_t, scale_t, y, m, n, k, st);
  else
    launch_linear_a8<1, 8>(xq, sa, packed_t, scale_t, y, m, n, k, st);
  MOSAIC_RETURN_LAUNCH("mxt16_linear_a8");
}

extern "C" int mosaic_mxt16_linear_a8(const uint8_t* xq, const float* sa, const uint8_t* packed_t,
                                      const uint8_t* scale_t, uint16_t* y, int64_t m, int64_t n, int64_t k,
                                      void* stream) {
  return mxt16_linear_a8_impl(xq, sa, packed_t, scale_t, y, m, n, k, nullptr, 0, stream);
}

extern "C" size_t mosaic_mxt16_linear_a8_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0 || k % 128 || n % 16) return 0;
  return dense_a8_ws_bytes(m, n, k);
}

extern "C" int mosaic_mxt16_linear_a8_ws(const uint8_t* xq, const float* sa, const uint8_t* packed_t,
                                         const uint8_t* scale_t, uint16_t* y, int64_t m, int64_t n, int64_t k,
                                         void* workspace, size_t workspace_bytes, void* stream) {
  return mxt16_linear_a8_impl(xq, sa, packed_t, scale_t, y, m, n, k, workspace, workspace_bytes, stream);
}

extern "C" size_t mosaic_moe_a8_workspace_bytes(int64_t m, int64_t hidden, int64_t inter, int64_t n_experts,
                                                int64_t top_k, int has_shared) {
  return carve_moe_workspace(nullptr, m, hidden, inter, n_experts, top_k, has_shared, kMoeBlockM, true).bytes;
}

extern "C" int mosaic_moe_a8_forward(const uint16_t* x, const float* logits, int32_t* ids, float* weights,
                                     const uint8_t* gu_packed, const uint8_t* gu_scale, const uint8_t* d_packed,
                                     const uint8_t* d_scale, const uint8_t* sh_gu_packed, const uint8_t* sh_gu_scale,
                                     const uint8_t* sh_d_packed, const uint8_t* sh_d_scale, uint16_t* y, int64_t m,
                                     int64_t hidden, int64_t inter, int64_t n_experts, int64_t top_k, int score_func,
                                     int renorm, float route_scale, const float* route_bias, float swiglu_limit,
                                     void* workspace, size_t workspace_bytes, void* const* stage_events,
                                     void* stream) {
  MOSAIC_CHECK_ARG(x && ids && weights && gu_packed && gu_scale && d_packed && d_scale && y && workspace,
                   "moe_a8_forward: null pointer");
  const int has_shared = sh_gu_packed != nullptr;
  MOSAIC_CHECK_ARG(!has_shared || (sh_gu_scale && sh_d_packed && sh_d_scale),
                   "moe_a8_forward: shared expert needs all four tensors");
  MOSAIC_CHECK_ARG(hidden > 0 && hidden % 128 == 0, "moe_a8_forward: hidden=%lld must be a multiple of 128",
                   (long long)hidden);
  MOSAIC_CHECK_ARG(inter > 0 && inter % 128 == 0, "moe_a8_forward: inter=%lld must be a multiple of 128",
                   (long long)inter);
  MOSAIC_CHECK_ARG(m >= 1, "moe_a8_forward: m=%lld", (long long)m);
  MoeWorkspace w =
      carve_moe_workspace((char*)workspace, m, hidden, inter, n_experts, top_k, has_shared, kMoeBlockM, true);
  MOSAIC_CHECK_ARG(workspace_bytes >= w.bytes, "moe_a8_forward: workspace %zu < %zu bytes", workspace_bytes,
                   w.bytes);
  hipStream_t st = (hipStream_t)stream;
  auto mark = [&](int i) {
    if (stage_events && stage_events[i]) (void)hipEventRecord((hipEvent_t)stage_events[i], st);
  };
  mark(0);
  LayoutOut lo{w.counts, w.offsets, w.perm, w.perm_token, w.perm_weight, w.sorted_ids, w.inv_pos,
               w.combine_pos, w.tile_expert, w.tile_start, w.tile_rows, w.tile_p0, w.n_tiles, nullptr, 0, 1,
               w.chunk_counts, w.chunk_base};
  const int64_t A = m * top_k + (has_shared ? m : 0);
  // large batches (>= 24 assignments per expert on average): 128-row tiles
  // the prefill kernels copy 4 row scales (16 bytes) at a time: H / 128 and I / 128 multiples of 4
  const bool prefill = m * top_k >= 24 * n_experts && hidden % 512 == 0 && inter % 512 == 0;
  const int block_m = prefill ? kPfBM : kMoeBlockM;
  const int64_t e_ext = n_experts + (has_shared ? 1 : 0);
  const int64_t tcap = prefill ? (A + std::min(A, e_ext) * (kPfBM - 1)) / kPfBM : w.tile_cap;
  int rc = launch_route_layout(logits, route_bias, ids, weights, ids, weights, m, n_experts, top_k, score_func,
                               renorm, route_scale, has_shared, block_m, tcap, lo, st);
  if (rc != 0) return rc;
  mark(1);
  rc = mosaic_act_quant(x, MOSAIC_DTYPE_BF16, w.xq, w.xs, m, hidden, 128, 0, stream);
  if (rc != 0) return rc;
  mark(2);
  if (prefill) {
    uint16_t* yb = reinterpret_cast<uint16_t*>(w.yp);  // bf16 partials in the fp32 partial buffer
    const int64_t tcap8 = (tcap + 7) / 8 * 8;
    // the gate/up epilogue writes z already quantized (1x128 pow2 e4m3, as act_quant mode 0)
    MOSAIC_LAUNCH(moe_a8_gateup_prefill_kernel, dim3((unsigned)(inter / 128 * tcap8)), dim3(kPfWaves * 64), 0, st,
                       w.xq, w.xs, gu_packed, gu_scale, sh_gu_packed, sh_gu_scale, w.tile_expert, w.tile_rows,
                       w.tile_p0, w.n_tiles, w.perm_token, w.perm_weight, w.zq, w.zs, (int)hidden, (int)inter,
                       (int)n_experts, swiglu_limit);
    MOSAIC_LAUNCH_CHECK("moe_a8_gateup_prefill");
    mark(3);
    mark(4);  // the z requant is fused into the gate/up epilogue
    MOSAIC_LAUNCH(moe_a8_down_prefill_kernel, dim3((unsigned)(hidden / 256 * tcap8)), dim3(kPfWaves * 64), 0, st,
                       w.zq, w.zs, d_packed, d_scale, sh_d_packed, sh_d_scale, w.tile_expert, w.tile_rows, w.tile_p0,
                       w.n_tiles, yb, (int)hidden, (int)inter, (int)n_experts);
    MOSAIC_LAUNCH_CHECK("moe_a8_down_prefill");
    mark(5);
    MOSAIC_LAUNCH(moe_combine_bf16_kernel, dim3((unsigned)((hidden / 8 + 127) / 128), (unsigned)m), dim3(128),
                       0, st, yb, w.combine_pos, y, (int)m, (int)(top_k + has_shared), (int)hidden);
    MOSAIC_LAUNCH_CHECK("moe_a8_combine_bf16");
    mark(6);
    return kOk;
  }
  constexpr int GT = 2, GKS = 4, DT = 2, DKS = 4;
  MOSAIC_LAUNCH((moe_a8_gateup_kernel<GT, GKS>), dim3((unsigned)(inter / (8 * GT)), (unsigned)tcap), dim3(GKS * 64), 0,
                     st, w.xq, w.xs, gu_packed, gu_scale, sh_gu_packed, sh_gu_scale, w.tile_expert, w.tile_rows,
                     w.tile_p0, w.n_tiles, w.perm_token, w.perm_weight, w.z, (int)hidden, (int)inter,
                     (int)n_experts, swiglu_limit);
  MOSAIC_LAUNCH_CHECK("moe_a8_gateup");
  mark(3);
  // rows of z past the real assignments are never read by the down kernel
  rc = mosaic_act_quant(w.z, MOSAIC_DTYPE_BF16, w.zq, w.zs, A, inter, 128, 0, stream);
  if (rc != 0) return rc;
  mark(4);
  MOSAIC_LAUNCH((moe_a8_down_kernel<DT, DKS>), dim3((unsigned)(hidden / (16 * DT)), (unsigned)tcap), dim3(DKS * 64), 0,
                     st, w.zq, w.zs, d_packed, d_scale, sh_d_packed, sh_d_scale, w.tile_expert, w.tile_rows,
                     w.tile_p0, w.n_tiles, w.yp, (int)hidden, (int)inter, (int)n_experts);
  MOSAIC_LAUNCH_CHECK("moe_a8_down");
  mark(5);
  MOSAIC_LAUNCH(moe_combine_kernel, dim3((unsigned)((hidden + 255) / 256), (unsigned)m), dim3(256), 0, st,
                     w.yp, w.combine_pos, y, (int)m, (int)(top_k + has_shared), (int)hidden);
  MOSAIC_LAUNCH_CHECK("moe_a8_combine");
  mark(6);
  return kOk;
}
