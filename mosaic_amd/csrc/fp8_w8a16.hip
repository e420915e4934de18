// W8A16 linear: y [m, n] = x [m, k] bf16 . decode(W)^T with W e4m3 [n, k]
// (row-major, the checkpoint layout) and one fp32 scale per 128 x 128 block,
// s [ceil(n/128), k/128]: the fused in-GEMM decode of fp8_linear
// (bench/fp8_core.py:160-231): per 128-K block the fp32 product of x and the
// unscaled decoded weight is multiplied by the block scale and added to the
// fp32 accumulator (acc += dot(x, decode(w)) * s), then one bf16 rounding.
//
// Decode-shaped kernel (16 tokens per launch row): MFMA roles transposed, so a
// lane (c = l%16, q = l/16) holds weight row n0 + 16t + c and token m0 + c of
// x; of every 128-byte K block it holds weight bytes [16q, 16q + 16) and
// [64 + 16q, +16), which v_cvt_scalef32_pk_bf16_fp8 turns into exact bf16
// (unit scale), and the x elements at the same 32 K indices, as four
// K-steps of v_mfma_f32_16x16x32_bf16 (the sum over K does not care which K
// a lane holds as long as both operands agree).  A workgroup owns 16 T
// columns; its KS waves split the K blocks and meet in LDS.  Each wave streams
// its blocks through a register ring of D entries issued D blocks ahead with
// buffer loads (rows past n / m read zeros; entries past the wave's range are
// scaled by 0), as the FP8 x FP8 decode kernel does.
#include <algorithm>

#include "common.h"
#include "../../include/mosaic_amd.h"

namespace mosaic {
namespace {

__device__ __forceinline__ __amdgpu_buffer_rsrc_t w8_rsrc(const void* base, int64_t records) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)records, 0x00020000);
}

// 8 e4m3 bytes (two dwords) -> 8 exact bf16
__device__ __forceinline__ bf16x8_t e4m3x8_bf16(uint32_t w0, uint32_t w1) {
  const bf16x2_t p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false);
  const bf16x2_t p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true);
  const bf16x2_t p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false);
  const bf16x2_t p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true);
  return bf16x8_t{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

template <int T, int KS, int D>
__global__ void __launch_bounds__(KS * 64) w8a16_gemv_kernel(const uint16_t* __restrict__ X,
                                                             const uint8_t* __restrict__ W,
                                                             const float* __restrict__ Ws, uint16_t* __restrict__ Y,
                                                             int M, int N, int K) {
  __shared__ f32x4_t red[KS][T][64];
  const int lane = threadIdx.x & 63, ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, q = lane >> 4;
  const int n0 = blockIdx.x * 16 * T, m0 = blockIdx.y * 16;
  const int nkb = K / 128;
  const int kb0 = nkb * ks / KS, nb = nkb * (ks + 1) / KS - kb0;
  const __amdgpu_buffer_rsrc_t rw = w8_rsrc(W + (int64_t)n0 * K, (int64_t)min(N - n0, 16 * T) * K);
  const __amdgpu_buffer_rsrc_t rx = w8_rsrc(X + (int64_t)m0 * K, (int64_t)min(M - m0, 16) * K * 2);
  const uint32_t x_row = (uint32_t)(c * K * 2) + 32u * q;  // byte offset of x[m0 + c][16 q]
  const float* s_row[T];
#pragma unroll
  for (int t = 0; t < T; ++t) s_row[t] = Ws + (int64_t)(min(n0 + 16 * t, N - 1) / 128) * nkb;
  u32x4_t rwv[D][T][2], rxv[D][4];
  float rs[D][T];
  auto load = [&](int s, int i) {
    const int kb = kb0 + (i < nb ? i : nb - 1);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint32_t off = (uint32_t)((16 * t + c) * K + kb * 128 + 16 * q);
      rwv[s][t][0] = __builtin_amdgcn_raw_buffer_load_b128(rw, (int)off, 0, 0);
      rwv[s][t][1] = __builtin_amdgcn_raw_buffer_load_b128(rw, (int)(off + 64), 0, 0);
      rs[s][t] = s_row[t][kb];
    }
    const int xo = (int)(x_row + kb * 256);
    rxv[s][0] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo, 0, 0);
    rxv[s][1] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 16, 0, 0);
    rxv[s][2] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 128, 0, 0);
    rxv[s][3] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 144, 0, 0);
  };
  f32x4_t acc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int s, int i) {
    // this step's operands pass through empty volatile asm statements, which
    // keep its MFMAs behind the previous step's loads: hoisted, their waits
    // drained the ring
#pragma unroll
    for (int j = 0; j < 4; ++j) asm volatile("" : "+v"(rxv[s][j]));
#pragma unroll
    for (int t = 0; t < T; ++t) {
      asm volatile("" : "+v"(rwv[s][t][0]), "+v"(rwv[s][t][1]));
      f32x4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u32x4_t& wv = rwv[s][t][j >> 1];
        const bf16x8_t wb = e4m3x8_bf16(wv[2 * (j & 1)], wv[2 * (j & 1) + 1]);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wb, __builtin_bit_cast(bf16x8_t, rxv[s][j]), d, 0, 0, 0);
      }
      // the scale read here, not hoisted to the chunk's start (where its wait
      // would drain every load in flight)
      float sv = rs[s][t];
      asm volatile("" : "+v"(sv));
      const float sc = i < nb ? sv : 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[t][r] = __builtin_fmaf(d[r], sc, acc[t][r]);
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
  if (ks < T && m0 + c < M) {
    const int t = ks;
    f32x4_t v = red[0][t][lane];
#pragma unroll
    for (int k2 = 1; k2 < KS; ++k2) v += red[k2][t][lane];
    // lane (c, q): y[m0 + c][n .. n + 3], n = n0 + 16 t + 4 q
    const int n = n0 + 16 * t + 4 * q;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (n + r < N) Y[(int64_t)(m0 + c) * N + n + r] = f32_bf16(v[r]);
  }
}

// 17..80 rows: the weight streamed once against G groups of 16 rows of x
// (rows past m read row m - 1, their results are not stored).  A workgroup
// owns 16 NW columns: NW compute waves, a 16-column tile each, streaming their
// weight blocks through an 8-deep register ring with exact waits (step
// operands pinned behind the previous step's loads), and one copier wave that
// alone copies the x blocks (G x 16 rows x 256 bytes; the 16-byte chunks of
// row r XOR-swizzled by r % 16) into a four-stage LDS ring three blocks ahead
// with global -> LDS copies, so its copy wait is exact.  One barrier per block
// hands a stage over.  As in the decode kernel, lane (c, q) of MFMA step j
// takes K indices 16q + 8(j & 1) + 64(j >> 1) + 0..7 of both operands.
constexpr int kW8LA = 3, kW8DA = kW8LA + 1, kW8LB = 8;

__device__ __forceinline__ uint32_t w8_lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// one 16-byte global -> LDS copy per lane; the LDS address of lane i is base + 16 i
__device__ __forceinline__ void w8_copy16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(__builtin_amdgcn_readfirstlane(lds)),
               "v"(g) : "memory", "m0");
}

template <int G, int NW>
__global__ void __launch_bounds__((NW + 1) * 64) w8a16_mid_kernel(const uint16_t* __restrict__ X, const uint8_t* __restrict__ W,
                                                        const float* __restrict__ Ws, uint16_t* __restrict__ Y, int M,
                                                        int N, int K, float* __restrict__ part) {
  constexpr int LA = kW8LA, DA = kW8DA, LB = kW8LB;
  constexpr int RUNS = 4 * G;             // 1 KB x runs per block: 4 rows of 256 bytes each
  constexpr int STAGE = G * 4096;
  static_assert((LA - 1) * RUNS <= 63, "the copy wait count fits vmcnt");
  __shared__ __attribute__((aligned(16))) uint8_t lds[DA][STAGE];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, q = lane >> 4;
  // K slice blockIdx.y of gridDim.y (at least 8 blocks each when split)
  const int nkb = K / 128, ntile = (N + 15) / 16, S = gridDim.y;
  const int kb0 = nkb * (int)blockIdx.y / S, nb = nkb * ((int)blockIdx.y + 1) / S - kb0;
  const int nchunks = (nb + LB - 1) / LB;
  if (wv == NW) {
    // copier wave: run r is rows 4 r .. 4 r + 3; lane l copies physical chunk
    // l % 16 of row 4 r + l / 16, which holds logical chunk (l % 16) ^ (row % 16)
    const uint8_t* gsrc[RUNS];
#pragma unroll
    for (int r = 0; r < RUNS; ++r) {
      const int row = 4 * r + (lane >> 4);
      const int logical = (lane & 15) ^ (row & 15);
      gsrc[r] = reinterpret_cast<const uint8_t*>(X + (int64_t)min(row, M - 1) * K) + logical * 16;
    }
    auto issue = [&](int st, int kb) {
      const uint32_t base = w8_lds_addr(lds[st]);
#pragma unroll
      for (int r = 0; r < RUNS; ++r) w8_copy16(gsrc[r] + (int64_t)kb * 256, base + (uint32_t)(r * 1024));
    };
#pragma unroll
    for (int j = 0; j < LA; ++j) issue(j, kb0 + (j < nb ? j : nb - 1));
    for (int ch = 0; ch < nchunks; ++ch) {
#pragma unroll
      for (int u = 0; u < LB; ++u) {
        const int i = ch * LB + u;
        // block i has landed: after its copies only those of the LA - 1 next blocks were issued
        asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((LA - 1) * RUNS) : "memory");
        issue((u + LA) % DA, kb0 + (i + LA < nb ? i + LA : nb - 1));
      }
    }
    // the copies issued past K land before the LDS is released
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return;
  }
  const int tile = __builtin_amdgcn_readfirstlane((int)blockIdx.x * NW + wv), tile_c = min(tile, ntile - 1);
  const int n0 = tile_c * 16;
  const __amdgpu_buffer_rsrc_t rw = w8_rsrc(W + (int64_t)n0 * K, (int64_t)min(N - n0, 16) * K);
  const float* s_row = Ws + (int64_t)(n0 / 128) * nkb;
  u32x4_t rwv[LB][2];
  float rs[LB];
  auto load = [&](int s, int i) {
    const int kb = kb0 + (i < nb ? i : nb - 1);
    const uint32_t off = (uint32_t)(c * K + kb * 128 + 16 * q);
    rwv[s][0] = __builtin_amdgcn_raw_buffer_load_b128(rw, (int)off, 0, 0);
    rwv[s][1] = __builtin_amdgcn_raw_buffer_load_b128(rw, (int)(off + 64), 0, 0);
    rs[s] = s_row[kb];
  };
  f32x4_t acc[G];
#pragma unroll
  for (int g = 0; g < G; ++g) acc[g] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < LB; ++s) {
    load(s, s);
    asm volatile("" ::: "memory");  // in slot order: the compiler's waits count the later loads
  }
  for (int ch = 0; ch < nchunks; ++ch) {
#pragma unroll
    for (int u = 0; u < LB; ++u) {
      const int i = ch * LB + u;
      // this wave's reads of the stage the copier refills next are done
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      const uint8_t* stg = lds[u % DA];
      asm volatile("" : "+v"(rwv[u][0]), "+v"(rwv[u][1]));
      bf16x8_t wb[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) wb[j] = e4m3x8_bf16(rwv[u][j >> 1][2 * (j & 1)], rwv[u][j >> 1][2 * (j & 1) + 1]);
      const float sc = i < nb ? rs[u] : 0.f;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const int row = 16 * g + c;
        const uint8_t* xr = stg + row * 256;
        f32x4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int chunk = 2 * q + (j & 1) + 8 * (j >> 1);
          const u32x4_t xv = *reinterpret_cast<const u32x4_t*>(xr + ((chunk ^ (row & 15)) << 4));
          d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wb[j], __builtin_bit_cast(bf16x8_t, xv), d, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[g][r] = __builtin_fmaf(d[r], sc, acc[g][r]);
      }
      load(u, i + LB);
      asm volatile("" ::: "memory");
    }
  }
  if (tile >= ntile) return;
  // lane (c, q) of group g: y[16 g + c][n .. n + 3], n = 16 tile + 4 q
  const int n = tile * 16 + 4 * q;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int m = 16 * g + c;
    if (m >= M) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (n + r < N) {
        if (part)
          part[((int64_t)blockIdx.y * M + m) * N + n + r] = acc[g][r];
        else
          Y[(int64_t)m * N + n + r] = f32_bf16(acc[g][r]);
      }
  }
}

template <int KS>
void launch_w8a16(const uint16_t* x, const uint8_t* w, const float* s, uint16_t* y, int64_t m, int64_t n, int64_t k,
                  hipStream_t st) {
  const int nb = (int)(k / 128 / KS);
  const dim3 grid((unsigned)((n + 15) / 16), (unsigned)((m + 15) / 16));
  if (nb % 4 == 0 || nb >= 8)
    MOSAIC_LAUNCH((w8a16_gemv_kernel<1, KS, 4>), grid, dim3(KS * 64), 0, st, x, w, s, y, (int)m, (int)n, (int)k);
  else
    MOSAIC_LAUNCH((w8a16_gemv_kernel<1, KS, 2>), grid, dim3(KS * 64), 0, st, x, w, s, y, (int)m, (int)n, (int)k);
}


// y = sum over the S slices of part, in slice order, as bf16; 4 elements a thread
__global__ void __launch_bounds__(256) w8a16_splitk_reduce_kernel(const float* __restrict__ part, int S, int64_t mn,
                                                                  uint16_t* __restrict__ Y) {
  const int64_t i0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t i = i0 + j;
    if (i >= mn) break;
    float v = part[i];
    for (int sl = 1; sl < S; ++sl) v += part[(int64_t)sl * mn + i];
    Y[i] = f32_bf16(v);
  }
}

// Mid-kernel plan.  Every workgroup copies all of x for its K slice, so wider
// workgroups copy it fewer times: NW compute waves (4..8; 7 for 5 row groups,
// whose 8-wave build spills) and S K slices of at least 12 blocks (S > 1 only
// with a partials workspace) are chosen for the widest grid that stays
// within one workgroup per CU, the fewest slices and then the fewest waves on
// ties.  Split against one pass, weights cold, M = 17 / 32 / 64 / 80:
// 7168 x 16384 67.2 / 67.5 / 86.1 / 106.1 -> 38.4 / 39.8 / 46.6 / 51.6 us,
// 4096 x 7168 31.0 / 31.4 / 39.0 / 50.5 -> 16.8 / 17.7 / 21.5 / 25.3 us;
// slices of 8 blocks (7168 x 2048) gained nothing (11.9-18.4 against
// 11.4-18.4 us).  4..16 rows take the mid kernel (one row group, unsplit) only where K
// has >= 48 blocks and N gives >= 224 workgroups; there the decode ring's time
// grows with the rows (x re-read once per 16-column tile) while the mid
// kernel's stays flat.  Weights cold, M = 4 / 8 / 16, ring against mid:
// 18432 x 7168 38.3 / 44.9 / 57.6 -> 30.1 / 30.4 / 31.9 us, 32768 x 7168
// 57.1 / 65.5 / 81.1 -> 48.4 / 49.1 / 49.6 us, 16384 x 7168 33.7 / 38.6 /
// 47.2 -> 29.8 / 29.5 / 30.2 us; not taken: 192 workgroups (12288 x 7168:
// 26.1 / 30.0 against 28.6 / 28.5 us at M = 4 / 8).  1..3 rows take it only
// with 5 or more compute waves a workgroup (M = 1: 18432 x 7168 33.1 -> 30.2,
// 32768 x 7168 51.3 -> 48.6 us); with 4 the ring stays faster (16384 x 6144
// at M = 1: 23.6 against 25.4 us).
struct W8MidPlan {
  bool mid;
  int nw, S;
};
static W8MidPlan w8_mid_plan(int64_t m, int64_t n, int64_t k, bool allow_split) {
  const int64_t tiles = (n + 15) / 16, nkb = k / 128;
  const int nw_max = m > 64 ? 7 : 8;
  auto pick = [&](int64_t smax, int64_t& best) {
    W8MidPlan p{true, nw_max, 1};
    best = 0;
    for (int64_t sl = 1; sl <= smax; ++sl)
      for (int v = 4; v <= nw_max; ++v) {
        const int64_t wgs = (tiles + v - 1) / v * sl;
        if (wgs <= 256 && wgs > best) {
          best = wgs;
          p = {true, v, (int)sl};
        }
      }
    return p;
  };
  int64_t best = 0;
  const int64_t smax = allow_split ? std::max<int64_t>(1, std::min<int64_t>(8, nkb / 12)) : 1;
  if (m > 16 && n >= 4096) return pick(smax, best);
  // 33..80 rows over 1536..4095 columns with K >= 32 blocks: only with a K
  // split (the m-tile ring re-reads the weight once per 16 rows; unsplit, the
  // mid kernel's few workgroups lose).  Ring against split mid at M = 64 / 80:
  // 1536 x 7168 23.8 / 23.8 -> 19.5 / 22.3 us, 2048 x 7168 24.1 / 34.4 -> 19.9 /
  // 22.4 us; 576 columns, K = 2048 and 32 rows or fewer stay on the ring.
  if (smax > 1 && m > 32 && n >= 1536 && nkb >= 32) return pick(smax, best);
  const W8MidPlan p = pick(1, best);
  if (m <= 16 && nkb >= 48 && best >= 224 && (m >= 4 || p.nw >= 5)) return p;
  // shorter K (12..47 blocks) from 12 rows: ring against mid at M = 12 / 16,
  // 24576 x 1536 14.3 / 16.1 -> 13.6 / 13.8 us, 18432 x 2048 14.9 / 16.6 ->
  // 11.9 / 12.1 us, 16384 x 4096 22.8 / 24.6 -> 18.6 / 18.8 us (at 4..8 rows
  // the ring won on some of them: 24576 x 1536 at M = 8 12.7 against 13.4 us)
  if (m >= 12 && m <= 16 && nkb >= 12 && best >= 224) return p;
  // 12..16 rows over a narrower N with a weight of >= 40 MB: the K split fills
  // the grid (ring against split mid at M = 12 / 16: 7168 x 16384 40.8 / 46.2
  // -> 35.9 / 36.3 us, 7168 x 8192 22.0 / 24.3 -> 19.6 / 19.8 us, 8192 x 7168
  // 22.2 / 24.6 -> 19.3 / 19.2 us); below 40 MB the split's fixed cost loses
  // (4096 x 7168: 12.2 / 13.6 against 14.4 / 14.6 us), and so do 8 rows or fewer
  if (allow_split && m >= 12 && m <= 16 && nkb >= 48 && n * k >= (40ll << 20)) {
    const W8MidPlan q = pick(std::max<int64_t>(1, std::min<int64_t>(8, nkb / 12)), best);
    if (best >= 224) return q;
  }
  return {false, 0, 1};
}

}  // namespace
}  // namespace mosaic

using namespace mosaic;

static int w8a16_linear_impl(const uint16_t* x, const uint8_t* w, const float* s, uint16_t* y, int64_t m, int64_t n,
                             int64_t k, void* workspace, size_t workspace_bytes, void* stream) {
  MOSAIC_CHECK_ARG(x && w && s && y, "fp8_w8a16_linear: null pointer");
  MOSAIC_CHECK_ARG(k > 0 && k % 128 == 0, "fp8_w8a16_linear: K=%lld must be a positive multiple of 128", (long long)k);
  MOSAIC_CHECK_ARG(n > 0 && m >= 0 && m <= 80, "fp8_w8a16_linear: m=%lld (0..80) n=%lld", (long long)m, (long long)n);
  MOSAIC_CHECK_ARG(n * k < (1ll << 31) && m * k * 2 < (1ll << 31), "fp8_w8a16_linear: operands beyond 2 GiB");
  if (m == 0) return kOk;
  hipStream_t st = (hipStream_t)stream;
  // 17..80 rows and N >= 4096 (at least 256 16-column tiles): the mid kernel,
  // the weight read once (18432 x 7168 at M = 64: 172.5 -> 89.3 us with four
  // compute waves a workgroup and no K split); narrower N keeps the m-tile
  // grid (1536 x 7168 at M = 64: 24.0 against 42.0 us)
  W8MidPlan plan = w8_mid_plan(m, n, k, true);
  float* part = nullptr;
  if (plan.mid && plan.S > 1) {
    if (workspace && workspace_bytes >= (size_t)plan.S * m * n * 4)
      part = reinterpret_cast<float*>(workspace);
    else
      plan = w8_mid_plan(m, n, k, false);  // no partials workspace: the whole K in one slice
  }
  const int64_t tiles = (n + 15) / 16;
  if (plan.mid) {
    const int nw = plan.nw;
    const dim3 pgrid(1, (unsigned)plan.S);
#define W8_MID(GV, NWV)                                                                                             \
  MOSAIC_LAUNCH((w8a16_mid_kernel<GV, NWV>), dim3((unsigned)((tiles + NWV - 1) / NWV), pgrid.y), dim3((NWV + 1) * 64), \
                0, st, x, w, s, y, (int)m, (int)n, (int)k, part)
#define W8_MID_G(GV)                  \
  switch (nw) {                       \
    case 5: W8_MID(GV, 5); break;     \
    case 6: W8_MID(GV, 6); break;     \
    case 7: W8_MID(GV, 7); break;     \
    case 8: if constexpr (GV < 5) W8_MID(GV, 8); else W8_MID(GV, 7); break; \
    default: W8_MID(GV, 4); break;    \
  }
    if (m <= 16) {
      W8_MID_G(1)
    } else if (m <= 32) {
      W8_MID_G(2)
    } else if (m <= 64) {
      W8_MID_G(4)
    } else {
      W8_MID_G(5)
    }
#undef W8_MID_G
#undef W8_MID
    if (part) {
      const int64_t mn = m * n;
      MOSAIC_LAUNCH(w8a16_splitk_reduce_kernel, dim3((unsigned)((mn + 1023) / 1024)), dim3(256), 0, st, part,
                    plan.S, mn, y);
    }
    MOSAIC_RETURN_LAUNCH("fp8_w8a16_linear");
  }
  const int64_t mtiles = tiles * ((m + 15) / 16);
  if (mtiles <= 256 && (k / 128) >= 16)
    launch_w8a16<8>(x, w, s, y, m, n, k, st);
  else if (mtiles <= 1152 && (k / 128) >= 8)
    launch_w8a16<4>(x, w, s, y, m, n, k, st);
  else
    launch_w8a16<2>(x, w, s, y, m, n, k, st);
  MOSAIC_RETURN_LAUNCH("fp8_w8a16_linear");
}

extern "C" int mosaic_fp8_w8a16_linear(const uint16_t* x, const uint8_t* w, const float* s, uint16_t* y, int64_t m,
                                       int64_t n, int64_t k, void* stream) {
  return w8a16_linear_impl(x, w, s, y, m, n, k, nullptr, 0, stream);
}

extern "C" size_t mosaic_fp8_w8a16_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || m > 80 || n <= 0 || k <= 0 || k % 128) return 0;
  const W8MidPlan plan = w8_mid_plan(m, n, k, true);
  return plan.mid && plan.S > 1 ? (size_t)plan.S * (size_t)m * (size_t)n * 4 : 0;
}

extern "C" int mosaic_fp8_w8a16_linear_ws(const uint16_t* x, const uint8_t* w, const float* s, uint16_t* y, int64_t m,
                                          int64_t n, int64_t k, void* workspace, size_t workspace_bytes,
                                          void* stream) {
  return w8a16_linear_impl(x, w, s, y, m, n, k, workspace, workspace_bytes, stream);
}
