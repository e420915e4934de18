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

// Decode-shaped GEMM (M <= 16, wide N): MFMA roles transposed (rows are 16 B
// rows, columns the M tokens, so a lane's column has one a_s per K-block); a
// workgroup owns 16 T columns of C and its KS waves split K.  Each wave streams
// its K-blocks through a register ring of D entries (the T tiles' B operands,
// the A operand, a_s and the T b_s values of one block), issued D blocks ahead
// with buffer loads: B rows past N and A rows past M read zeros, entries past
// the wave's range reload its last block and are scaled by 0, so the loop has
// no branches.  The K parts meet in LDS in wave order.
// B layouts (L): 0, checkpoint [N, K] rows, each load reads 64 bytes of 16
// rows (lane (c, q): row c, bytes 16q.. and 64 + 16q..).  1, the same rows,
// each load reading whole 128-byte lines: the first covers rows 0..7 of the
// tile (lane c < 8: row c, bytes 16q..; lane c >= 8: row c - 8, bytes
// 64 + 16q..), the second rows 8..15 the same way, and two DPP moves per
// dword (row rotate by 8, half the lanes written) give lane (c, q) row c's
// bytes [16q, 16q + 16) and [64 + 16q, 64 + 16q + 16), the A operand's map.
// 2, the T16 prepack (fp8_t16_pack_kernel): each 16-row x 128-K block is 2 KB
// in lane order, so each load reads 1 KB contiguous.  All three hand the MFMA
// the same operands, so their results are identical.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t fp8_rsrc(const void* base, int64_t records) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)records, 0x00020000);
}

template <int T, int KS, int D, int L>
__global__ void __launch_bounds__(KS * 64) fp8_gemv_kernel(const uint8_t* __restrict__ A, const float* __restrict__ As,
                                                           const uint8_t* __restrict__ B,
                                                           const float* __restrict__ Bs, void* __restrict__ C, int M,
                                                           int N, int K, int out_f32) {
  __shared__ f32x4_t red[KS][T][64];
  const int lane = threadIdx.x & 63, ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, q = lane >> 4;
  const int n0 = blockIdx.x * 16 * T;
  const int nkb = K / 128;
  const int kb0 = nkb * ks / KS, nb = nkb * (ks + 1) / KS - kb0;
  const __amdgpu_buffer_rsrc_t rb = fp8_rsrc(B + (int64_t)n0 * K, (int64_t)min(N - n0, 16 * T) * K);
  const __amdgpu_buffer_rsrc_t ra = fp8_rsrc(A, (int64_t)M * K);
  const __amdgpu_buffer_rsrc_t rs = fp8_rsrc(As, (int64_t)M * nkb * 4);
  const uint32_t a_row = c < M ? (uint32_t)(c * K) + 16u * q : 0x80000000u;  // rows past M: out of range
  const uint32_t s_row = c < M ? (uint32_t)(c * nkb) * 4u : 0x80000000u;
  const float* bs_row[T];
#pragma unroll
  for (int t = 0; t < T; ++t) bs_row[t] = Bs + (int64_t)(min(n0 + 16 * t, N - 1) / 128) * nkb;
  u32x4_t rbv[D][T][2], rav[D][2];
  float rsa[D], rsb[D][T];
  auto load = [&](int s, int i) {
    const int kb = kb0 + (i < nb ? i : nb - 1);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      if (L == 2) {
        const uint32_t off = (uint32_t)(16 * t * K + kb * 2048 + 16 * (4 * c + q));
        rbv[s][t][0] = __builtin_amdgcn_raw_buffer_load_b128(rb, (int)off, 0, 0);
        rbv[s][t][1] = __builtin_amdgcn_raw_buffer_load_b128(rb, (int)(off + 1024), 0, 0);
      } else if (L == 1) {
        const uint32_t off = (uint32_t)((16 * t + (c & 7)) * K + kb * 128 + 16 * (q + 4 * (c >> 3)));
        rbv[s][t][0] = __builtin_amdgcn_raw_buffer_load_b128(rb, (int)off, 0, 0);
        rbv[s][t][1] = __builtin_amdgcn_raw_buffer_load_b128(rb, (int)(off + 8 * K), 0, 0);
      } else {
        const uint32_t off = (uint32_t)((16 * t + c) * K + kb * 128 + 16 * q);
        rbv[s][t][0] = __builtin_amdgcn_raw_buffer_load_b128(rb, (int)off, 0, 0);
        rbv[s][t][1] = __builtin_amdgcn_raw_buffer_load_b128(rb, (int)(off + 64), 0, 0);
      }
      rsb[s][t] = bs_row[t][kb];
    }
    rav[s][0] = __builtin_amdgcn_raw_buffer_load_b128(ra, (int)(a_row + kb * 128), 0, 0);
    rav[s][1] = __builtin_amdgcn_raw_buffer_load_b128(ra, (int)(a_row + kb * 128 + 64), 0, 0);
    rsa[s] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, (int)(s_row + kb * 4), 0, 0));
  };
  f32x4_t acc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int s, int i) {
    // a_s read here, not hoisted to the chunk's start (where it would wait for every load in flight)
    float sa = rsa[s];
    asm volatile("" : "+v"(sa));
    const i32x8_t a = {(int)rav[s][0][0], (int)rav[s][0][1], (int)rav[s][0][2], (int)rav[s][0][3],
                       (int)rav[s][1][0], (int)rav[s][1][1], (int)rav[s][1][2], (int)rav[s][1][3]};
#pragma unroll
    for (int t = 0; t < T; ++t) {
      i32x8_t bo;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int x0 = (int)rbv[s][t][0][j], x1 = (int)rbv[s][t][1][j];
        bo[j] = L == 1 ? __builtin_amdgcn_update_dpp(x0, x1, 0x128, 0xF, 0xC, false) : x0;
        bo[4 + j] = L == 1 ? __builtin_amdgcn_update_dpp(x1, x0, 0x128, 0xF, 0x3, false) : x1;
      }
      const f32x4_t d = mfma_fp8_block(bo, a);
      const float sc = i < nb ? sa * rsb[s][t] : 0.f;
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
  if (ks < T && c < M) {
    const int t = ks;
    f32x4_t v = red[0][t][lane];
#pragma unroll
    for (int k2 = 1; k2 < KS; ++k2) v += red[k2][t][lane];
    // lane (c, q): C[c][n .. n + 3], n = n0 + 16 t + 4 q
    const int n = n0 + 16 * t + 4 * q;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (n + r < N) {
        if (out_f32)
          reinterpret_cast<float*>(C)[(int64_t)c * N + n + r] = v[r];
        else
          reinterpret_cast<uint16_t*>(C)[(int64_t)c * N + n + r] = f32_bf16(v[r]);
      }
    }
  }
}

// Ring depth D: a divisor of the wave's block count where one exists, so no
// ring entry reloads a block past the wave's range (each such reload is a
// wasted 2 KB read per tile; with 1.5 blocks a wave and D = 4 the launch ran
// 1.7x slower).
template <int T, int KS, int L>
static void launch_fp8_gemv(const uint8_t* a, const float* as, const uint8_t* b, const float* bs, void* c, int64_t m,
                            int64_t n, int64_t k, int out_f32, hipStream_t st) {
  const int nb = (int)(k / 128 / KS);
  const dim3 grid((unsigned)((n + 16 * T - 1) / (16 * T)));
#define FP8_GEMV(DV) \
  MOSAIC_LAUNCH((fp8_gemv_kernel<T, KS, DV, L>), grid, dim3(KS * 64), 0, st, a, as, b, bs, c, (int)m, (int)n, (int)k, \
                out_f32)
  if (nb % 8 == 0)
    FP8_GEMV(8);
  else if (nb % 7 == 0)
    FP8_GEMV(7);
  else if (nb % 6 == 0)
    FP8_GEMV(6);
  else if (nb % 5 == 0)
    FP8_GEMV(5);
  else if (nb % 4 == 0)
    FP8_GEMV(4);
  else if (nb % 3 == 0)
    FP8_GEMV(3);
  else
    FP8_GEMV(4);
#undef FP8_GEMV
}

// Ring-kernel plans: few rows, one 16-column tile per workgroup (more
// workgroups), K split wider where there are few column tiles; more rows, two
// tiles share each A fragment, except where that leaves under 192 workgroups
// (measured with the weights cold in HBM, M = 1 and 16, N = 4096..24576).
// Short K (at most 16 blocks): the widest split of 8, 4 or 2 waves that
// divides the blocks and leaves each wave at least 3 (K = 1536: 4 waves of 3
// blocks, 3.3-4.0 against 4.5-6.0 us at N = 576..4096 with the T16 layout),
// except for two-tile workgroups over the checkpoint layout, whose whole-line
// loads ran faster with 2 waves (M = 16, N = 7168, K = 2048: 5.7 against 6.4 us).
template <int L>
static void dispatch_fp8_gemv(const uint8_t* a, const float* as, const uint8_t* b, const float* bs, void* c,
                              int64_t m, int64_t n, int64_t k, int out_f32, hipStream_t st) {
  const int64_t t16 = (n + 15) / 16, nkb = k / 128;
  int T = 1, KS;
  if (m <= 4)
    KS = t16 <= 256 ? 8 : t16 <= 1152 ? 4 : 2;
  else if ((n + 31) / 32 < 192)
    KS = 8;
  else
    T = 2, KS = 2;
  if (nkb <= 16 && (L == 2 || T == 1)) {
    KS = 8;
    while (KS > 2 && (nkb % KS || nkb / KS < 3)) KS /= 2;
  }
#define FP8_PLAN(TT, KK) \
  if (T == TT && KS == KK) return launch_fp8_gemv<TT, KK, L>(a, as, b, bs, c, m, n, k, out_f32, st);
  FP8_PLAN(1, 8) FP8_PLAN(1, 4) FP8_PLAN(1, 2) FP8_PLAN(2, 8) FP8_PLAN(2, 4) FP8_PLAN(2, 2)
#undef FP8_PLAN
}

template <int T, int KS>
static void launch_fp8_skinny(const uint8_t* a, const float* as, const uint8_t* b, const float* bs, void* c,
                              int64_t m, int64_t n, int64_t k, int out_f32, hipStream_t st) {
  dim3 grid((unsigned)((n + 16 * T - 1) / (16 * T)), (unsigned)((m + 15) / 16));
  MOSAIC_LAUNCH((fp8_gemm_skinny_kernel<T, KS>), grid, dim3(KS * 64), 0, st, a, as, b, bs, c, (int)m, (int)n,
                     (int)k, out_f32);
}

// Tiled kernel (M >= 96, MFMA-bound at large M): a workgroup of BM/32 waves
// owns a BM x 128 block of C (its 128 columns share one b_s row); each wave
// owns a 64x64 quarter (4x4 MFMA tiles).  Each 128-K block's A and B tiles and
// its scales (BM a_s values, one b_s) go global -> LDS directly
// (global_load_lds, 16 bytes a lane into 1 KB runs, 4 bytes a lane for the
// scales) through a ring of three stages, two blocks ahead of the MFMAs.  All
// copies in the loop are issued from inline asm so the compiler neither waits
// for the in-flight stages before each LDS read (as it does for copies it can
// see) nor needs staging registers; every wave issues the same number of
// copies per stage, so `s_waitcnt vmcnt(ops)` + a bare s_barrier hands a stage
// over.  LDS rows are 128 bytes with their 16-byte chunks XOR-swizzled by
// (row >> 1) & 7 (applied on the global side of the copy), so the 16 rows one
// MFMA operand read touches fall in distinct banks.  Workgroups are remapped so
// that the ones on one XCD (dispatch goes round-robin over 8) take
// neighbouring tiles, grouped 4 M-tiles deep.  The K loop has the big kernel's
// schedule: transposed MFMA roles (one a_s per lane and tile, 4 consecutive C
// columns per lane), the next A fragment read during the MFMAs, each tile's
// rescale issued after the next tile's MFMAs.
constexpr int kTileN = 128, kStages = 3;

__device__ __forceinline__ void tile_coords(int id, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int T = tiles_m * tiles_n;
  const int full = (T / 8) * 8;
  const int r = id < full ? (id % 8) * (T / 8) + id / 8 : id;
  constexpr int GM = 4;  // M = 4096 shapes: 0.5-5% faster than groups of 8 or 16; 2 was mixed
  const int per_group = GM * tiles_n;
  const int g = r / per_group;
  const int first_m = g * GM;
  const int gm = min(GM, tiles_m - first_m);
  const int in = r % per_group;
  tm = first_m + in % gm;
  tn = in / gm;
}

__device__ __forceinline__ i32x8_t lds_fp8_operand(const uint8_t* tile, int row, int q) {
  const int swz = (row >> 1) & 7;
  const uint8_t* p = tile + row * 128;
  const u32x4_t lo = *reinterpret_cast<const u32x4_t*>(p + ((q ^ swz) << 4));
  const u32x4_t hi = *reinterpret_cast<const u32x4_t*>(p + (((q + 4) ^ swz) << 4));
  return i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

__device__ __forceinline__ uint32_t fp8_lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// one 16-byte (resp. 4-byte) global -> LDS copy per lane; the LDS address of
// lane i is base + 16 i (resp. 4 i)
__device__ __forceinline__ void fp8_copy16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(__builtin_amdgcn_readfirstlane(lds)),
               "v"(g) : "memory", "m0");
}
__device__ __forceinline__ void fp8_copy4(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off" ::"s"(__builtin_amdgcn_readfirstlane(lds)),
               "v"(g) : "memory", "m0");
}

template <int BM>
struct Fp8Tile {
  static constexpr int NT = BM * 2;                   // threads
  static constexpr int NW = NT / 64;                  // waves
  static constexpr int AB = (BM + kTileN) * 128;      // A and B bytes of a stage
  static constexpr int SA = AB;                       // a_s: BM floats
  static constexpr int SB = SA + BM * 4;              // b_s: 64 copies of one float
  static constexpr int STAGE = SB + 256;
  static constexpr int RUNS = AB / 1024 / NW;         // 1 KB A/B runs per wave per stage
  static constexpr int SRUNS = BM / 64;               // 256-byte a_s runs per stage
  static constexpr int OPS = RUNS + 1;                // copies per wave per stage
  static_assert(AB / 1024 % NW == 0, "stage does not split evenly over the waves");
  static_assert(SRUNS + 1 <= NW, "one scale copy per wave");
};

// Split-K (blockIdx.y = K slice of kps blocks): with `part` the slice writes its
// fp32 partial tile to part[slice][M][N] (fp8_splitk_reduce_kernel sums the
// slices in order); without it the tile goes to C.
template <int BM>
__global__ void __launch_bounds__(BM * 2, 1) fp8_gemm_tiled_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ B,
    const float* __restrict__ Bs, void* __restrict__ C, int M, int N, int K, int out_f32, int kps,
    float* __restrict__ part) {
  using TT = Fp8Tile<BM>;
  __shared__ __attribute__((aligned(16))) uint8_t lds[kStages][TT::STAGE];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int c = lane & 15, q = lane >> 4;
  int tm, tn;
  tile_coords(blockIdx.x, (M + BM - 1) / BM, (N + kTileN - 1) / kTileN, tm, tn);
  const int m0 = tm * BM, n0 = tn * kTileN;
  const int wm = (wv >> 1) * 64, wn = (wv & 1) * 64;
  const int nkb = K / 128;
  // this lane's source row and 16-byte chunk for each of the wave's A/B runs
  const uint8_t* gsrc[TT::RUNS];
  int ldsoff[TT::RUNS];
#pragma unroll
  for (int ii = 0; ii < TT::RUNS; ++ii) {
    const int i = wv * TT::RUNS + ii;
    const int row = (i < BM / 8 ? 8 * i : 8 * (i - BM / 8)) + (lane >> 3);
    const int logical = (lane & 7) ^ ((row >> 1) & 7);
    gsrc[ii] = i < BM / 8 ? A + (int64_t)min(m0 + row, M - 1) * K + logical * 16
                          : B + (int64_t)min(n0 + row, N - 1) * K + logical * 16;
    ldsoff[ii] = i * 1024;
  }
  // the wave's scale copy: waves < SRUNS take 64 a_s rows each, wave SRUNS the
  // b_s value (every lane the same), the others repeat it into the same slot
  const float* ssrc;
  int sdst;
  if (wv < TT::SRUNS) {
    ssrc = As + (int64_t)min(m0 + 64 * wv + lane, M - 1) * nkb;
    sdst = TT::SA + 256 * wv;
  } else {
    ssrc = Bs + (int64_t)(n0 / 128) * nkb;
    sdst = TT::SB;
  }
  auto issue = [&](int st, int kb) {
    const uint32_t base = fp8_lds_addr(lds[st]);
#pragma unroll
    for (int ii = 0; ii < TT::RUNS; ++ii) fp8_copy16(gsrc[ii] + (int64_t)kb * 128, base + ldsoff[ii]);
    fp8_copy4(ssrc + kb, base + sdst);
  };
  f32x4_t acc[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  f32x4_t dp[4];  // product of the previous tile, rescaled one tile later
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) dp[nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float sp = 0.f;
  const int kb0 = (int)blockIdx.y * kps, cnt = min(nkb, kb0 + kps) - kb0;
  // a slice past K (never launched) copies nothing and writes zero partials
  if (cnt > 0) issue(0, kb0);
  if (cnt > 1) issue(1, kb0 + 1);
  for (int i = 0; i < cnt; ++i) {
    // block kb0 + i landed for every wave (its copies, then the barrier); the next may still fly
    if (i + 1 < cnt)
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(TT::OPS) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (i + 2 < cnt) issue((i + 2) % kStages, kb0 + i + 2);
    const uint8_t* stg = lds[i % kStages];
    const uint8_t* ta = stg;
    const uint8_t* tb = stg + BM * 128;
    const float sb = *reinterpret_cast<const float*>(stg + TT::SB);
    i32x8_t bop[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) bop[nt] = lds_fp8_operand(tb, wn + 16 * nt + c, q);
    i32x8_t aop[2];
    aop[0] = lds_fp8_operand(ta, wm + c, q);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      if (mt + 1 < 4) aop[(mt + 1) & 1] = lds_fp8_operand(ta, wm + 16 * (mt + 1) + c, q);
      // transposed roles: rows are B rows (n), columns A rows (m = wm + 16 mt + c)
      f32x4_t d[4];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) d[nt] = mfma_fp8_block(bop[nt], aop[mt & 1]);
      const int pm = mt == 0 ? 3 : mt - 1;  // the previous tile (tile 3 of the previous block at mt == 0)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[pm][nt][r] = __builtin_fmaf(dp[nt][r], sp, acc[pm][nt][r]);
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) dp[nt] = d[nt];
      sp = *reinterpret_cast<const float*>(stg + TT::SA + 4 * (wm + 16 * mt + c)) * sb;
    }
  }
#pragma unroll
  for (int nt = 0; nt < 4; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[3][nt][r] = __builtin_fmaf(dp[nt][r], sp, acc[3][nt][r]);
  // lane (c, q) of tile (mt, nt) holds C[m0 + wm + 16 mt + c][n .. n + 3], n = n0 + wn + 16 nt + 4 q
  // 4-column vector stores: N % 4 == 0 and an output base aligned for them (16 B covers both widths)
  const bool vec = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(part ? (const void*)part : C) & 15) == 0;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int m = m0 + wm + 16 * mt + c;
    if (m >= M) continue;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int n = n0 + wn + 16 * nt + 4 * q;
      const f32x4_t v = acc[mt][nt];
      if (part || out_f32) {
        float* o = part ? part + ((int64_t)blockIdx.y * M + m) * N + n : reinterpret_cast<float*>(C) + (int64_t)m * N + n;
        if (vec && n + 3 < N) {
          *reinterpret_cast<f32x4_t*>(o) = v;
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r < N) o[r] = v[r];
        }
      } else {
        uint16_t* o = reinterpret_cast<uint16_t*>(C) + (int64_t)m * N + n;
        if (vec && n + 3 < N) {
          const uint32_t lo = (uint32_t)f32_bf16(v[0]) | ((uint32_t)f32_bf16(v[1]) << 16);
          const uint32_t hi = (uint32_t)f32_bf16(v[2]) | ((uint32_t)f32_bf16(v[3]) << 16);
          *reinterpret_cast<uint2*>(o) = make_uint2(lo, hi);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r < N) o[r] = f32_bf16(v[r]);
        }
      }
    }
  }
}

// C = sum over the S slices of part, in slice order; 4 elements per thread
__global__ void __launch_bounds__(256) fp8_splitk_reduce_kernel(const float* __restrict__ part, int S, int64_t mn,
                                                                void* __restrict__ C, int out_f32) {
  const int64_t i0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t i = i0 + j;
    if (i >= mn) break;
    float v = part[i];
    for (int sl = 1; sl < S; ++sl) v += part[(int64_t)sl * mn + i];
    if (out_f32)
      reinterpret_cast<float*>(C)[i] = v;
    else
      reinterpret_cast<uint16_t*>(C)[i] = f32_bf16(v);
  }
}

template <int BM>
static void launch_fp8_tiled(const uint8_t* a, const float* as, const uint8_t* b, const float* bs, void* c,
                             int64_t m, int64_t n, int64_t k, int out_f32, hipStream_t st, int S = 1,
                             float* part = nullptr) {
  const int64_t tiles = ((m + BM - 1) / BM) * ((n + kTileN - 1) / kTileN);
  const int nkb = (int)(k / 128), kps = (nkb + S - 1) / S;
  // slices of kps blocks: only the non-empty ones are launched (K = 33 blocks
  // in 8 slices of 5 would leave slice 7 starting past K)
  S = (nkb + kps - 1) / kps;
  MOSAIC_LAUNCH((fp8_gemm_tiled_kernel<BM>), dim3((unsigned)tiles, (unsigned)S), dim3(BM * 2), 0, st, a, as, b,
                     bs, c, (int)m, (int)n, (int)k, out_f32, kps, S > 1 ? part : nullptr);
  if (S > 1) {
    const int64_t mn = m * n;
    MOSAIC_LAUNCH(fp8_splitk_reduce_kernel, dim3((unsigned)((mn + 1023) / 1024)), dim3(256), 0, st, part, S, mn,
                       c, out_f32);
  }
}

// Mid-size kernel (16 < M <= 64): the decode ring's weight stream with G
// groups of 16 rows of A.  A workgroup owns 16 W columns of C and one K slice
// (blockIdx.y): W compute waves, a 16-column tile each, and a copier wave.
// Every compute wave streams its tile's weight blocks through a register ring
// LB blocks ahead with buffer loads (L = 2: the T16 prepack, 1 KB contiguous
// per load; L = 0: the checkpoint rows), and waits for them only where the
// compiler's own count places the wait.  The copier wave alone copies the A
// blocks (G x 16 rows x 128 bytes, XOR-swizzled 16-byte chunks as the tiled
// kernel stages them) and their a_s values into an LDS ring LA blocks ahead
// with global -> LDS copies, so its copy wait is exact and no compute wave
// waits behind a copy: each A block is read once per workgroup and used by
// its W compute waves.  One barrier per block hands a stage over.  Per
// block a compute wave runs G unit-scale MFMAs (roles transposed: lane (c, q)
// holds C[16 g + c][n .. n + 3]) and rescales them by a_s x b_s into separate
// fp32 accumulators.  The loop runs whole chunks of LB blocks; blocks past the
// slice reload its last block and are scaled by 0.  With `part` the slice
// writes its fp32 partials to part[slice][M][N].
constexpr int kMidLA = 3, kMidDA = kMidLA + 1, kMidLB = 8;

template <int G>
struct Fp8Mid {
  static constexpr int RUNS = 2 * G;                        // 1 KB A runs per block (copier wave)
  static constexpr int SLOTS = G * 16 < 64 ? 64 : G * 16;   // a_s slots of a stage
  static constexpr int SCOPIES = SLOTS / 64;                // 64-slot a_s copies per block
  static constexpr int SA = G * 2048;                       // a_s offset in a stage
  static constexpr int STAGE = SA + SLOTS * 4;
  static constexpr int OPA = RUNS + SCOPIES;                // copies per block
  static_assert((kMidLA - 1) * OPA <= 63, "the copy wait count fits vmcnt");
};

template <int G, int L, int W>
__global__ void __launch_bounds__((W + 1) * 64) fp8_gemm_mid_kernel(const uint8_t* __restrict__ A, const float* __restrict__ As,
                                                           const uint8_t* __restrict__ B,
                                                           const float* __restrict__ Bs, void* __restrict__ C, int M,
                                                           int N, int K, int out_f32, float* __restrict__ part) {
  using TT = Fp8Mid<G>;
  constexpr int LA = kMidLA, DA = kMidDA, LB = kMidLB;
  __shared__ __attribute__((aligned(16))) uint8_t lds[DA][TT::STAGE];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, q = lane >> 4;
  const int nkb = K / 128, ntile = N / 16;
  const int S = gridDim.y;
  const int kb0 = nkb * (int)blockIdx.y / S, nb = nkb * ((int)blockIdx.y + 1) / S - kb0;
  const int nchunks = (nb + LB - 1) / LB;
  if (wv == W) {
    // copier wave: run r is rows 8 r .. 8 r + 7 of the A block; the a_s copy j
    // takes slots 64 j .. 64 j + 63
    if (nb <= 0) return;
    const uint8_t* gsrc[TT::RUNS];
#pragma unroll
    for (int r = 0; r < TT::RUNS; ++r) {
      const int row = 8 * r + (lane >> 3);
      const int logical = (lane & 7) ^ ((row >> 1) & 7);
      gsrc[r] = A + (int64_t)min(row, M - 1) * K + logical * 16;
    }
    const float* ssrc[TT::SCOPIES];
#pragma unroll
    for (int j = 0; j < TT::SCOPIES; ++j) ssrc[j] = As + (int64_t)min(64 * j + lane, M - 1) * nkb;
    auto issue = [&](int st, int kb) {
      const uint32_t base = fp8_lds_addr(lds[st]);
#pragma unroll
      for (int r = 0; r < TT::RUNS; ++r) fp8_copy16(gsrc[r] + (int64_t)kb * 128, base + (uint32_t)(r * 1024));
#pragma unroll
      for (int j = 0; j < TT::SCOPIES; ++j) fp8_copy4(ssrc[j] + kb, base + (uint32_t)(TT::SA + 256 * j));
    };
#pragma unroll
    for (int j = 0; j < LA; ++j) issue(j, kb0 + (j < nb ? j : nb - 1));
    for (int ch = 0; ch < nchunks; ++ch) {
#pragma unroll
      for (int u = 0; u < LB; ++u) {
        const int i = ch * LB + u;
        // block i has landed: after its copies only those of the LA - 1 next blocks were issued
        asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((LA - 1) * TT::OPA) : "memory");
        issue((u + LA) % DA, kb0 + (i + LA < nb ? i + LA : nb - 1));
      }
    }
    // the copies issued past the slice land before the LDS is released
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return;
  }
  const int tile = __builtin_amdgcn_readfirstlane((int)blockIdx.x * W + wv), tile_c = min(tile, ntile - 1);
  // this wave's weight tile and its 128-row scale row
  const __amdgpu_buffer_rsrc_t rb = fp8_rsrc(B + (int64_t)tile_c * 16 * K, (int64_t)16 * K);
  const float* bs_row = Bs + (int64_t)(tile_c * 16 / 128) * nkb;
  u32x4_t rbv[LB][2];
  float rsb[LB];
  auto load_b = [&](int s, int i) {
    const int kb = kb0 + (i < nb ? i : nb - 1);
    const uint32_t off = L == 2 ? (uint32_t)(kb * 2048 + 16 * (4 * c + q)) : (uint32_t)(c * K + kb * 128 + 16 * q);
    rbv[s][0] = __builtin_amdgcn_raw_buffer_load_b128(rb, (int)off, 0, 0);
    rbv[s][1] = __builtin_amdgcn_raw_buffer_load_b128(rb, (int)(off + (L == 2 ? 1024 : 64)), 0, 0);
    rsb[s] = bs_row[kb];
  };
  f32x4_t acc[G];
#pragma unroll
  for (int g = 0; g < G; ++g) acc[g] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  if (nb > 0) {
    // in slot order (the compiler's wait for slot u counts the loads issued after it)
#pragma unroll
    for (int j = 0; j < LB; ++j) {
      load_b(j, j);
      asm volatile("" ::: "memory");
    }
    for (int ch = 0; ch < nchunks; ++ch) {
#pragma unroll
      for (int u = 0; u < LB; ++u) {
        const int i = ch * LB + u;
        // this wave's reads of the stage the copier refills next are done
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const uint8_t* stg = lds[u % DA];
        const float* sas = reinterpret_cast<const float*>(stg + TT::SA);
        const i32x8_t bo = {(int)rbv[u][0][0], (int)rbv[u][0][1], (int)rbv[u][0][2], (int)rbv[u][0][3],
                            (int)rbv[u][1][0], (int)rbv[u][1][1], (int)rbv[u][1][2], (int)rbv[u][1][3]};
        const float sb = i < nb ? rsb[u] : 0.f;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const f32x4_t d = mfma_fp8_block(bo, lds_fp8_operand(stg, 16 * g + c, q));
          const float sc = sas[16 * g + c] * sb;
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[g][r] = __builtin_fmaf(d[r], sc, acc[g][r]);
        }
        load_b(u, i + LB);
      }
    }
  }
  if (tile >= ntile) return;
  const int n = tile * 16 + 4 * q;
  // 4-column vector stores where the output base allows them (N % 16 == 0)
  const bool vec = (reinterpret_cast<uintptr_t>(part ? (const void*)part : C) & 15) == 0;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int m = 16 * g + c;
    if (m >= M) continue;
    const f32x4_t v = acc[g];
    if (part || out_f32) {
      float* o = part ? part + ((int64_t)blockIdx.y * M + m) * N + n : reinterpret_cast<float*>(C) + (int64_t)m * N + n;
      if (vec) {
        *reinterpret_cast<f32x4_t*>(o) = v;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = v[r];
      }
    } else {
      uint16_t* o = reinterpret_cast<uint16_t*>(C) + (int64_t)m * N + n;
      if (vec) {
        const uint32_t lo = (uint32_t)f32_bf16(v[0]) | ((uint32_t)f32_bf16(v[1]) << 16);
        const uint32_t hi = (uint32_t)f32_bf16(v[2]) | ((uint32_t)f32_bf16(v[3]) << 16);
        *reinterpret_cast<uint2*>(o) = make_uint2(lo, hi);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = f32_bf16(v[r]);
      }
    }
  }
}

// Mid-kernel plan: G groups of 16 rows (2 or 4), W compute waves (16-column
// tiles) per workgroup and S K slices of at least 8 blocks each (the slices'
// fp32 partials are summed by fp8_splitk_reduce_kernel).  Every workgroup
// copies the whole A block stream of its slice, so wider workgroups copy A
// fewer times; the (W, S) with 4 <= W <= 8 whose grid comes closest to one
// workgroup per CU without passing 256 is taken, the fewest slices and then
// the fewest waves on ties.  Measured with the weights cold at M = 32 / 64
// against the earlier 4 waves and up to 512 workgroups: 18432 x 7168 (5, 1)
// 38.5 -> 32.4 / 50.0 -> 42.0 us, 7168 x 16384 (7, 4) 34-35 -> 30.7 / 41-43 ->
// 36.6 us, 24576 x 1536 (6, 1) 13.9 -> 12.3 / 16.9 -> 15.3 us; narrow N
// keeps 4 waves.
struct Fp8MidPlan {
  int G, S, W;  // row groups, K slices, compute waves per workgroup
};
static Fp8MidPlan fp8_mid_plan(int64_t m, int64_t n, int64_t k) {
  const int G = m <= 16 ? 1 : m <= 32 ? 2 : 4;
  const int64_t tiles = n / 16, nkb = k / 128;
  const int64_t smax = std::max<int64_t>(1, std::min<int64_t>(8, nkb / 8));
  Fp8MidPlan plan{G, 1, 8};  // more than 2048 tiles: the widest workgroups, unsplit
  int64_t best = 0;
  for (int64_t sl = 1; sl <= smax; ++sl)
    for (int w = 4; w <= 8; ++w) {
      const int64_t wgs = (tiles + w - 1) / w * sl;
      if (wgs <= 256 && wgs > best) {
        best = wgs;
        plan = {G, (int)sl, w};
      }
    }
  return plan;
}

// 12..16 rows: the mid kernel with one row group replaces the decode ring where
// its plan needs no K split (a very wide N) and K has at least 48 blocks; the
// ring's two-tile workgroups read A once per 32 columns, the mid kernel once
// per 16 W.  Interleaved A/B, weights cold, M = 12 / 16, T16 and checkpoint
// rows: 18432 x 7168 30.0 / 32.1 -> 26.4 / 26.6 us and 34.8 / 37.4 -> 29.3 /
// 29.6 us; 32768 x 7168 46.2 / 48.5 -> 45.7 / 45.7 us and 50.2 / 55.4 -> 48.5 /
// 48.8 us.  Not taken: 8 rows (32768 x 7168 over the checkpoint rows 46.4 ->
// 48.4 us), K = 4096 (16384 x 4096: 15.3-18.6 -> 16.7-20.2 us), and the
// narrower or shorter config shapes, which stay faster on the ring.
static bool fp8_mid_small(int64_t m, int64_t n, int64_t k) {
  return m >= 12 && m <= 16 && n % 16 == 0 && k / 128 >= 48 && fp8_mid_plan(m, n, k).S == 1;
}

template <int L>
static void launch_fp8_mid(const uint8_t* a, const float* as, const uint8_t* b, const float* bs, void* c, int64_t m,
                           int64_t n, int64_t k, int out_f32, hipStream_t st, Fp8MidPlan plan, float* part) {
  const int S = part ? plan.S : 1;
  const dim3 grid((unsigned)((n / 16 + plan.W - 1) / plan.W), (unsigned)S);
  float* pp = S > 1 ? part : nullptr;
#define FP8_MID(GV, WV)                                                                                           \
  MOSAIC_LAUNCH((fp8_gemm_mid_kernel<GV, L, WV>), grid, dim3((WV + 1) * 64), 0, st, a, as, b, bs, c, (int)m, (int)n, \
                (int)k, out_f32, pp)
#define FP8_MID_W(GV)  \
  switch (plan.W) {    \
    case 5: FP8_MID(GV, 5); break; \
    case 6: FP8_MID(GV, 6); break; \
    case 7: FP8_MID(GV, 7); break; \
    case 8: FP8_MID(GV, 8); break; \
    default: FP8_MID(GV, 4); break; \
  }
  if (plan.G == 1) {
    FP8_MID_W(1)
  } else if (plan.G == 2) {
    FP8_MID_W(2)
  } else {
    FP8_MID_W(4)
  }
#undef FP8_MID_W
#undef FP8_MID
  if (S > 1) {
    const int64_t mn = m * n;
    MOSAIC_LAUNCH(fp8_splitk_reduce_kernel, dim3((unsigned)((mn + 1023) / 1024)), dim3(256), 0, st, part, S, mn, c,
                  out_f32);
  }
}

// Large tiled kernel (enough 256 x 256 tiles to fill the chip): a workgroup
// of 8 waves owns a 256 x 256 block of C; wave w owns rows 128 (w >> 2) and
// columns 64 (w & 3) of it.  Twice the columns of the 256 x 128 kernel for
// the same A block: 256 instead of 171 flops per byte copied into LDS.  A
// stage (A and B blocks of one K-block) is 64 KB, so the ring holds two
// stages, one K-block ahead.  Copies use a wave-uniform base (SGPR pair) plus
// per-lane 32-bit offsets.
//
// Scales: a stage copy waits for its slowest load, and a per-block gather of
// 256 a_s values (one per A row, 256 cache lines) was the slowest.  a_s and
// b_s are instead staged for 8 K-blocks at a time ([8 blocks][256 rows] and
// [8][2] floats, two chunk buffers): one 16-byte load per thread (a row's 8
// consecutive a_s values are 32 contiguous bytes), issued one block after a
// chunk starts and written to LDS after the next barrier, 6 blocks before use.
//
// MFMA roles are transposed (B rows are the MFMA rows, A rows the columns):
// a lane's 16 x 16 tile entries then share one A row, hence one a_s value per
// tile, and 4 consecutive C columns, stored as one 8- or 16-byte write.  The
// a_s values of a block are laid out so that lane c reads its 8 tiles' values
// as two 16-byte words.  A tile's fp32 rescale (acc += d * a_s * b_s) is
// issued after the next tile's MFMAs, so the MFMA results are not waited on;
// the next A fragment is read from LDS while the current MFMAs run.
struct Fp8Big {
  static constexpr int BM = 256, BN = 256, NT = 512, NW = 8;
  static constexpr int STAGE = (BM + BN) * 128;  // A and B bytes of a stage
  static constexpr int RUNS = STAGE / 1024 / NW;  // 8 one-KB A/B runs per wave per stage
  static constexpr int CHUNK = 8;                 // K-blocks per scale chunk
};

// a_s slot of tile row m (0..255): (m / 128) * 128 + (m % 16) * 8 + (m % 128) / 16,
// so that rows wm + 16 mt + c (mt = 0..7) of one wave sit at slots wm + 8 c + mt
__device__ __forceinline__ int fp8_big_slot_row(int s) {
  const int t = s & 127;
  return (s & ~127) + (t & 7) * 16 + (t >> 3);
}

__device__ __forceinline__ void fp8_copy16_so(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(__builtin_amdgcn_readfirstlane(lds)),
               "v"(off), "s"(base) : "memory", "m0");
}
__device__ __forceinline__ void fp8_copy4_so(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2" ::"s"(__builtin_amdgcn_readfirstlane(lds)),
               "v"(off), "s"(base) : "memory", "m0");
}

__global__ void __launch_bounds__(512, 1) fp8_gemm_big_kernel(const uint8_t* __restrict__ A,
                                                              const float* __restrict__ As,
                                                              const uint8_t* __restrict__ B,
                                                              const float* __restrict__ Bs, void* __restrict__ C,
                                                              int M, int N, int K, int out_f32) {
  using TT = Fp8Big;
  __shared__ __attribute__((aligned(16))) uint8_t lds[2][TT::STAGE];
  __shared__ __attribute__((aligned(16))) float sc_a[2][TT::CHUNK][TT::BM];  // [chunk buf][block][a_s slot]
  __shared__ float sc_b[2][TT::CHUNK][2];                                    // [chunk buf][block][column half]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, q = lane >> 4;
  int tm, tn;
  tile_coords(blockIdx.x, (M + TT::BM - 1) / TT::BM, (N + TT::BN - 1) / TT::BN, tm, tn);
  const int m0 = tm * TT::BM, n0 = tn * TT::BN;
  const int wm = (wv >> 2) * 128, wn = (wv & 3) * 64;
  const int nkb = K / 128;
  // waves 0..3 copy A rows 64 w .. 64 w + 63 of the tile, waves 4..7 B rows
  // 64 (w - 4) ..; run ii is 8 rows (1 KB, its 16-byte chunks XOR-swizzled)
  const bool is_a = wv < 4;
  const uint8_t* obase = is_a ? A : B;
  const int r0 = is_a ? m0 : n0, lim = (is_a ? M : N) - 1, rb = 64 * (wv & 3);
  uint32_t voff[TT::RUNS];
#pragma unroll
  for (int ii = 0; ii < TT::RUNS; ++ii) {
    const int row = rb + 8 * ii + (lane >> 3);
    const int logical = (lane & 7) ^ ((row >> 1) & 7);
    voff[ii] = (uint32_t)min(r0 + row, lim) * (uint32_t)K + (uint32_t)(logical * 16);
  }
  // Copy issue: a wave stalls at a copy until the address unit takes it, and
  // 64 one-KB copies per stage keep it busy for ~1000 cycles.  In interior
  // tiles one half of the waves (0..3 on even blocks, 4..7 on odd) issues the
  // whole stage, A and B rows through the same lane offsets (the base moved by
  // n0 - m0 rows), so the other wave of each SIMD keeps its MFMAs going; edge
  // tiles, whose clamped rows differ between A and B, copy their own operand.
  const bool interior = m0 + TT::BM <= M && n0 + TT::BN <= N;
  const uint8_t* base_a = is_a ? A : A + (int64_t)(m0 - n0) * K;
  const uint8_t* base_b = is_a ? B + (int64_t)(n0 - m0) * K : B;
  auto issue = [&](int st, int kb) {
    const uint32_t base = fp8_lds_addr(lds[st]);
    if (interior) {
      if ((wv >> 2) == (kb & 1)) {
        const int wq = wv & 3;
#pragma unroll
        for (int ii = 0; ii < TT::RUNS; ++ii) {
          fp8_copy16_so(base_a + (int64_t)kb * 128, voff[ii], base + (uint32_t)((wq * TT::RUNS + ii) * 1024));
          fp8_copy16_so(base_b + (int64_t)kb * 128, voff[ii], base + (uint32_t)(((wq + 4) * TT::RUNS + ii) * 1024));
        }
      }
    } else {
      const uint8_t* ob = obase + (int64_t)kb * 128;
#pragma unroll
      for (int ii = 0; ii < TT::RUNS; ++ii) fp8_copy16_so(ob, voff[ii], base + (uint32_t)((wv * TT::RUNS + ii) * 1024));
    }
  };
  // scale chunk loads: thread t takes a_s slot t / 2, blocks 4 (t % 2) .. + 3 of
  // the chunk; threads 0..15 also take b_s (block t % 8, column half t / 8)
  const int slot = tid >> 1, half = tid & 1;
  const float* arow = As + (int64_t)min(m0 + fp8_big_slot_row(slot), M - 1) * nkb;
  const float* brow = Bs + (int64_t)min(n0 / 128 + ((tid >> 3) & 1), (N - 1) / 128) * nkb;
  const bool vec_as = (nkb & 3) == 0 && (reinterpret_cast<uintptr_t>(As) & 15) == 0;  // 16-byte aligned a_s rows
  auto load_chunk = [&](int ch, f32x4_t& va, float& vb) {
    const int k0 = ch * TT::CHUNK + 4 * half;
    if (vec_as && k0 + 3 < nkb) {
      va = *reinterpret_cast<const f32x4_t*>(arow + k0);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) va[i] = arow[min(k0 + i, nkb - 1)];
    }
    vb = tid < 16 ? brow[min(ch * TT::CHUNK + (tid & 7), nkb - 1)] : 0.f;
  };
  auto store_chunk = [&](int ch, const f32x4_t& va, float vb) {
    const int bf = ch & 1;
#pragma unroll
    for (int i = 0; i < 4; ++i) sc_a[bf][4 * half + i][slot] = va[i];
    if (tid < 16) sc_b[bf][tid & 7][tid >> 3] = vb;
  };
  f32x4_t acc[8][4];
#pragma unroll
  for (int mt = 0; mt < 8; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  f32x4_t dp[4];  // product of the previous tile, rescaled one tile later
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) dp[nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float sp = 0.f;
  f32x4_t pend_a;  // the next scale chunk, between its load and its LDS write
  float pend_b;
  load_chunk(0, pend_a, pend_b);
  store_chunk(0, pend_a, pend_b);
  issue(0, 0);
  for (int kb = 0; kb < nkb; ++kb) {
    // block kb landed for every wave, and every wave is done with block kb - 1
    asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const int ch = kb / TT::CHUNK, kc = kb % TT::CHUNK;
    const bool next_chunk = (ch + 1) * TT::CHUNK < nkb;
    if (kc == 2 && next_chunk) store_chunk(ch + 1, pend_a, pend_b);  // its loads completed at the wait above
    if (kc == 1 && next_chunk) load_chunk(ch + 1, pend_a, pend_b);
    const uint8_t* stg = lds[kb & 1];
    const uint8_t* ta = stg;
    const uint8_t* tb = stg + TT::BM * 128;
    const float sb = sc_b[ch & 1][kc][wn >= 128 ? 1 : 0];
    const f32x4_t s0 = *reinterpret_cast<const f32x4_t*>(&sc_a[ch & 1][kc][wm + 8 * c]);
    const f32x4_t s1 = *reinterpret_cast<const f32x4_t*>(&sc_a[ch & 1][kc][wm + 8 * c + 4]);
    i32x8_t bop[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) bop[nt] = lds_fp8_operand(tb, wn + 16 * nt + c, q);
    i32x8_t aop[2];
    aop[0] = lds_fp8_operand(ta, wm + c, q);
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
      // block kb + 1's copies, once the first tile's MFMAs are issued
      if (mt == 1 && kb + 1 < nkb) issue((kb + 1) & 1, kb + 1);
      if (mt + 1 < 8) aop[(mt + 1) & 1] = lds_fp8_operand(ta, wm + 16 * (mt + 1) + c, q);
      f32x4_t d[4];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) d[nt] = mfma_fp8_block(bop[nt], aop[mt & 1]);
      const int pm = mt == 0 ? 7 : mt - 1;  // the previous tile (tile 7 of block kb - 1 at mt == 0)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[pm][nt][r] = __builtin_fmaf(dp[nt][r], sp, acc[pm][nt][r]);
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) dp[nt] = d[nt];
      sp = (mt < 4 ? s0[mt & 3] : s1[mt & 3]) * sb;
    }
  }
#pragma unroll
  for (int nt = 0; nt < 4; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[7][nt][r] = __builtin_fmaf(dp[nt][r], sp, acc[7][nt][r]);
  // lane (c, q) of tile (mt, nt) holds C[m0 + wm + 16 mt + c][n .. n + 3], n = n0 + wn + 16 nt + 4 q
  // 4-column vector stores: N % 4 == 0 and an output base aligned for them (16 B covers both widths)
  const bool vec = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(C) & 15) == 0;
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) {
    const int m = m0 + wm + 16 * mt + c;
    if (m >= M) continue;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int n = n0 + wn + 16 * nt + 4 * q;
      const f32x4_t v = acc[mt][nt];
      if (out_f32) {
        float* o = reinterpret_cast<float*>(C) + (int64_t)m * N + n;
        if (vec && n + 3 < N) {
          *reinterpret_cast<f32x4_t*>(o) = v;
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r < N) o[r] = v[r];
        }
      } else {
        uint16_t* o = reinterpret_cast<uint16_t*>(C) + (int64_t)m * N + n;
        if (vec && n + 3 < N) {
          const uint32_t lo = (uint32_t)f32_bf16(v[0]) | ((uint32_t)f32_bf16(v[1]) << 16);
          const uint32_t hi = (uint32_t)f32_bf16(v[2]) | ((uint32_t)f32_bf16(v[3]) << 16);
          *reinterpret_cast<uint2*>(o) = make_uint2(lo, hi);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r < N) o[r] = f32_bf16(v[r]);
        }
      }
    }
  }
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

// T16 prepack of e4m3 weights for the ring kernel: [N, K] (N % 16 == 0,
// K % 128 == 0) -> blocks of 2048 bytes, block (g, kb) at (g * K/128 + kb) *
// 2048 holding rows 16g..16g+15, K bytes 128kb..128kb+127, in lane order:
// byte 1024h + 16(4c + q) + j = W[16g + c][128kb + 64h + 16q + j].  One
// thread moves one 16-byte chunk; PACK false is the exact inverse.
template <bool PACK>
__global__ void __launch_bounds__(256) fp8_t16_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                      int64_t chunks, int64_t k) {
  const int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= chunks) return;
  const int64_t nkb = k / 128, blk = o >> 7;
  const int w = (int)(o & 127), h = w >> 6, c = (w >> 2) & 15, q = w & 3;
  const int64_t row = (blk / nkb) * 16 + c, col = (blk % nkb) * 128 + 64 * h + 16 * q;
  const int64_t raw = row * k + col, t16 = o * 16;
  const int64_t from = PACK ? raw : t16, to = PACK ? t16 : raw;
  *reinterpret_cast<u32x4_t*>(dst + to) = *reinterpret_cast<const u32x4_t*>(src + from);
}

extern "C" int mosaic_fp8_block_dequant(const uint8_t* w, const float* s, uint16_t* out, int64_t n, int64_t k,
                                        int block_n, int block_k, void* stream) {
  MOSAIC_CHECK_ARG(w && s && out, "fp8_block_dequant: null pointer");
  MOSAIC_CHECK_ARG(n >= 0 && k > 0 && k % 4 == 0 && block_n > 0 && block_k > 0 && block_k % 4 == 0,
                   "fp8_block_dequant: K=%lld, block %dx%d", (long long)k, block_n, block_k);
  if (n == 0) return kOk;
  const int64_t total = n * k / 4;
  MOSAIC_LAUNCH(fp8_block_dequant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, w, s, out, n, k, block_n, block_k, (k + block_k - 1) / block_k);
  MOSAIC_RETURN_LAUNCH("fp8_block_dequant");
}

// Kernel choice of the block GEMM.  kind 0: skinny, 1: tiled<128>, 2: tiled<256>,
// 3: big tiles, 4: decode ring (M <= 16 with N >= 4096, or narrower N when K has
// at least 32 blocks), 5: mid kernel (17..64 rows, N % 16 == 0, its own K split;
// and 12..16 rows where fp8_mid_small holds).  The tiled kernels split K into S slices (S > 1 needs the
// S * M * N * 4-byte partials workspace) when their tiles cover fewer than
// half of the 256 CUs: S = min(8, 256 / tiles, K-blocks / 4).
struct Fp8Plan {
  int kind, S;
};
static Fp8Plan fp8_plan(int64_t m, int64_t n, int64_t k) {
  const int64_t nkb = k / 128;
  auto split = [&](int64_t tiles) {
    int64_t s = std::min<int64_t>(8, std::min<int64_t>(256 / std::max<int64_t>(tiles, 1), nkb / 4));
    return tiles * 2 <= 256 && s >= 2 ? (int)s : 1;
  };
  if (m >= 256) {
    const int64_t big_tiles = ((m + 255) / 256) * ((n + 255) / 256);
    // the big kernel addresses A and B with 32-bit offsets
    if (big_tiles >= 256 && m * k < (1ll << 32) && n * k < (1ll << 32)) return {3, 1};
    return {2, split(((m + 255) / 256) * ((n + 127) / 128))};
  }
  // 65..95 rows: the tiled kernel for weights of 8 MB and more (18432 x 7168:
  // 180 -> 55 us), the skinny kernel below (576 x 7168: 11.7 against 16.9 us)
  if (m >= 96 || (m > 64 && n * k >= (8ll << 20))) {
    const int64_t tiles = ((m + 127) / 128) * ((n + 127) / 128);
    const int s = split(tiles);
    if (tiles * s >= 32) return {1, s};
  }
  // decode shapes: the ring kernel for wide N, and for narrower N when K is deep
  // enough for its 8-wave split to leave each wave >= 4 blocks (M = 1 / 16,
  // N = 576..2048, K = 7168: 9.2-9.6 -> 7.2-8.1 us and 11.8-12.3 -> 10.6-10.7 us
  // against the skinny kernel; at K = 1536 the skinny kernel stays faster)
  if (fp8_mid_small(m, n, k) && n * k < (1ll << 31)) return {5, 1};
  if (m <= 16 && nkb >= 8 && (n >= 4096 || nkb >= 32) && (int64_t)n * k < (1ll << 31)) return {4, 1};
  // 17..64 rows over the checkpoint layout: the mid kernel, its weight read once,
  // for weights of 8 MB and more (18432 x 7168, M = 64: 147 -> 61 us); below, the
  // skinny kernel's latency is lower (576 x 7168, M = 64: 12.1 against 13.6 us)
  if (m > 16 && m <= 64 && n % 16 == 0 && n * k >= (8ll << 20) && n * k < (1ll << 31))
    return {5, fp8_mid_plan(m, n, k).S};
  return {0, 1};
}

}  // namespace mosaic

using namespace mosaic;

static int fp8_block_gemm_impl(const uint8_t* a, const float* a_s, const uint8_t* b, const float* b_s, void* c,
                               int out_dtype, int64_t m, int64_t n, int64_t k, void* workspace,
                               size_t workspace_bytes, void* stream) {
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
  Fp8Plan plan = fp8_plan(m, n, k);
  if (plan.S > 1 && (!workspace || workspace_bytes < (size_t)plan.S * m * n * 4)) {
    // no partials workspace: the whole K in one slice (the kernels of the plan without split)
    plan = plan.kind == 1 && ((m + 127) / 128) * ((n + 127) / 128) < 32 ? Fp8Plan{0, 1} : Fp8Plan{plan.kind, 1};
  }
  float* part = reinterpret_cast<float*>(workspace);
  const int64_t mt = (m + 15) / 16;
  switch (plan.kind) {
    case 3: {
      const int64_t big_tiles = ((m + 255) / 256) * ((n + 255) / 256);
      MOSAIC_LAUNCH(fp8_gemm_big_kernel, dim3((unsigned)big_tiles), dim3(512), 0, st, a, a_s, b, b_s, c, (int)m,
                         (int)n, (int)k, f32);
      break;
    }
    case 4:
      // whole-line loads pay where a workgroup has more than 4 rows of work
      if (m <= 4)
        dispatch_fp8_gemv<0>(a, a_s, b, b_s, c, m, n, k, f32, st);
      else
        dispatch_fp8_gemv<1>(a, a_s, b, b_s, c, m, n, k, f32, st);
      break;
    case 5: launch_fp8_mid<0>(a, a_s, b, b_s, c, m, n, k, f32, st, fp8_mid_plan(m, n, k), plan.S > 1 ? part : nullptr);
      break;
    case 2: launch_fp8_tiled<256>(a, a_s, b, b_s, c, m, n, k, f32, st, plan.S, part); break;
    case 1: launch_fp8_tiled<128>(a, a_s, b, b_s, c, m, n, k, f32, st, plan.S, part); break;
    default:
      // columns per wave chosen so the grid covers the chip (>= ~2048 waves)
      if (((n + 63) / 64) * mt * 8 >= 4096)
        launch_fp8_skinny<4, 8>(a, a_s, b, b_s, c, m, n, k, f32, st);
      else if (((n + 31) / 32) * mt * 8 >= 4096)
        launch_fp8_skinny<2, 8>(a, a_s, b, b_s, c, m, n, k, f32, st);
      else
        launch_fp8_skinny<1, 8>(a, a_s, b, b_s, c, m, n, k, f32, st);
  }
  MOSAIC_RETURN_LAUNCH("fp8_block_gemm");
}

extern "C" int mosaic_fp8_block_gemm(const uint8_t* a, const float* a_s, const uint8_t* b, const float* b_s, void* c,
                                     int out_dtype, int64_t m, int64_t n, int64_t k, void* stream) {
  return fp8_block_gemm_impl(a, a_s, b, b_s, c, out_dtype, m, n, k, nullptr, 0, stream);
}

extern "C" size_t mosaic_fp8_block_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0 || k % 128) return 0;
  const Fp8Plan plan = fp8_plan(m, n, k);
  return plan.S > 1 ? (size_t)plan.S * (size_t)m * (size_t)n * 4 : 0;
}

extern "C" int mosaic_fp8_block_gemm_ws(const uint8_t* a, const float* a_s, const uint8_t* b, const float* b_s,
                                        void* c, int out_dtype, int64_t m, int64_t n, int64_t k, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  return fp8_block_gemm_impl(a, a_s, b, b_s, c, out_dtype, m, n, k, workspace, workspace_bytes, stream);
}

static int fp8_t16_convert(bool pack, const uint8_t* src, uint8_t* dst, int64_t n, int64_t k, void* stream) {
  MOSAIC_CHECK_ARG(src && dst, "fp8_t16: null pointer");
  MOSAIC_CHECK_ARG(n >= 0 && n % 16 == 0 && k > 0 && k % 128 == 0,
                   "fp8_t16: N=%lld must be a multiple of 16 and K=%lld a positive multiple of 128", (long long)n,
                   (long long)k);
  if (n == 0) return kOk;
  const int64_t chunks = n * k / 16;
  const dim3 grid((unsigned)((chunks + 255) / 256));
  if (pack)
    MOSAIC_LAUNCH(fp8_t16_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream, src, dst, chunks, k);
  else
    MOSAIC_LAUNCH(fp8_t16_kernel<false>, grid, dim3(256), 0, (hipStream_t)stream, src, dst, chunks, k);
  MOSAIC_RETURN_LAUNCH("fp8_t16");
}

extern "C" int mosaic_fp8_t16_prepack(const uint8_t* w, uint8_t* out, int64_t n, int64_t k, void* stream) {
  return fp8_t16_convert(true, w, out, n, k, stream);
}

extern "C" int mosaic_fp8_t16_unpack(const uint8_t* t16, uint8_t* w, int64_t n, int64_t k, void* stream) {
  return fp8_t16_convert(false, t16, w, n, k, stream);
}

extern "C" size_t mosaic_fp8_block_gemm_t16_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || m > 64 || n <= 0 || k <= 0 || k % 128 || n % 16 || (m <= 16 && !fp8_mid_small(m, n, k))) return 0;
  const Fp8MidPlan plan = fp8_mid_plan(m, n, k);
  return plan.S > 1 ? (size_t)plan.S * (size_t)m * (size_t)n * 4 : 0;
}

extern "C" int mosaic_fp8_block_gemm_t16(const uint8_t* a, const float* a_s, const uint8_t* bt, const float* b_s,
                                         void* c, int out_dtype, int64_t m, int64_t n, int64_t k, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  MOSAIC_CHECK_ARG(a && a_s && bt && b_s && c, "fp8_block_gemm_t16: null pointer");
  MOSAIC_CHECK_ARG(m >= 0 && m <= 64, "fp8_block_gemm_t16: M=%lld; the T16 layout serves M <= 64", (long long)m);
  MOSAIC_CHECK_ARG(n >= 0 && n % 16 == 0 && k > 0 && k % 128 == 0 && (int64_t)n * k < (1ll << 31),
                   "fp8_block_gemm_t16: N=%lld (multiple of 16), K=%lld (multiple of 128), N*K < 2^31", (long long)n,
                   (long long)k);
  MOSAIC_CHECK_ARG(out_dtype == MOSAIC_DTYPE_F32 || out_dtype == MOSAIC_DTYPE_BF16,
                   "fp8_block_gemm_t16: out dtype %d", out_dtype);
  if (m == 0 || n == 0) return kOk;
  const int f32 = out_dtype == MOSAIC_DTYPE_F32;
  hipStream_t st = (hipStream_t)stream;
  if (m <= 16 && !fp8_mid_small(m, n, k)) {
    dispatch_fp8_gemv<2>(a, a_s, bt, b_s, c, m, n, k, f32, st);
  } else {
    const Fp8MidPlan plan = fp8_mid_plan(m, n, k);
    const bool split = plan.S > 1 && workspace && workspace_bytes >= (size_t)plan.S * m * n * 4;
    launch_fp8_mid<2>(a, a_s, bt, b_s, c, m, n, k, f32, st, plan, split ? (float*)workspace : nullptr);
  }
  MOSAIC_RETURN_LAUNCH("fp8_block_gemm_t16");
}
