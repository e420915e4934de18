// DSA decode on gfx950: the FP8 lightning indexer with an exact top-k, and
// MLA decode over the selected KV entries.
//
// Indexer (Indexer.forward, .mosaicvm/source/inference_model.py:408-439):
//   score[t] = sum_h w_h * ReLU(q_h . k_t * q_scale[h] * k_scale[t]),  top-k over t.
// The canonical score (the one the indices are defined on) is fixed step by step:
//   d = exact dot of the decoded e4m3 values rounded once to fp32;
//   a = fp32(fp32(d * q_scale[h]) * k_scale[t]); r = a > 0 ? a : +0;
//   s = sequential fp32 sum over h ascending, from +0, of fp32(r * w_h);
// top-k lists descending s, ties to the lower index, NaN lowest.
//
// The exact dot is cheap per token but not for every token, so selection is
// certified in two stages:
//   1. dsa_index_bound_kernel streams k once through the fp8 MFMA and writes,
//      per token, an interval [lo, hi] that contains the canonical score.  The
//      width is 2^-12 * 448 * |k_scale[t]| * sum_h |w_h| |q_scale[h]| ||q_h||_1,
//      at least 16x the worst-case error of any fp32 accumulation order of the
//      128 products (|products| summed <= 448 ||q_h||_1 in code units) plus the
//      rounding of the remaining steps.
//   2. tau = a lower bound of the k-th largest lo (radix digits of its order key).
//      Any token with hi < tau is beaten by k tokens whose lo >= tau, so the
//      true top-k lies inside {t : hi >= tau}.  Those candidates (typically
//      k + a few percent) get the exact score (fp64 accumulation is exact:
//      products are multiples of 2^-18 below 2^17.6, 128 of them stay below
//      2^25) and are sorted by (score, -index).
//
// MLA decode (sparse_attn_kernel, .mosaicvm/source/inference_kernel.py:276-352;
// sparse_attn_ref, mosaicvm/model/dsa.py:214-242): per (row, head)
//   o = sum_t bf16(p_t) * v_t / (sum_t p_t + exp(sink - m)),  p_t = exp(s_t - m),
//   s_t = q . kv_t * scale over the selected t (index -1 masked), kv_t = [latent
//   e4m3 * scale -> bf16, rope bf16], v_t = latent.  Online softmax over 64-token
//   blocks (the reference's block size) in each of several token splits, then a
//   combine over splits.
#include <algorithm>

#include "common.h"
#include "../../include/mosaic_amd.h"

namespace mosaic {

// ===================================================================== indexer
constexpr int kIdxD = 128;
constexpr int kHistBins = 2048;     // 11-bit radix digits
constexpr int kSortCap = 4096;      // candidates sorted in LDS
constexpr int kMaxTopk = 4096;
constexpr float kBoundFactor = 448.0f / 4096.0f * (1.0f + 1.0f / 512.0f);

// order-preserving keys of fp32 values: NaN lowest (exact scores, lower bounds)
// or highest (upper bounds)
__device__ __forceinline__ uint32_t f32_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ uint32_t key_low_nan(float f) { return (f != f) ? 0u : f32_key(f); }
__device__ __forceinline__ uint32_t key_high_nan(float f) { return (f != f) ? 0xFFFFFFFFu : f32_key(f); }

__device__ __forceinline__ int64_t row_length(const int32_t* lengths, int b, int64_t L) {
  if (!lengths) return L;
  const int64_t n = lengths[b];
  return n < 0 ? 0 : (n > L ? L : n);
}

__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Sum of |decoded e4m3| over the 32 code bytes of one MFMA operand lane.
__device__ __forceinline__ float abs_sum_fp8(const i32x8_t v) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const f32x2_t a = __builtin_amdgcn_cvt_pk_f32_fp8(v[i], false);
    const f32x2_t b = __builtin_amdgcn_cvt_pk_f32_fp8(v[i], true);
    s += fabsf(a[0]) + fabsf(a[1]) + fabsf(b[0]) + fabsf(b[1]);
  }
  return s;
}

__global__ void dsa_zero_kernel(uint32_t* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// Stage 1: fp8 MFMA scores with a rigorous interval; optional histogram of the
// top 11 bits of the lower-bound keys (per row, global atomics per workgroup).
template <int HT, int U>
__global__ void __launch_bounds__(256) dsa_index_bound_kernel(
    const uint8_t* __restrict__ q, const float* __restrict__ qs, const uint8_t* __restrict__ k,
    const float* __restrict__ ks, const float* __restrict__ w, const int32_t* __restrict__ lengths,
    float* __restrict__ lo, float* __restrict__ hi, uint32_t* __restrict__ hist1, int64_t L) {
  constexpr int H = HT * 16;
  __shared__ uint32_t lh[kHistBins];
  const int b = blockIdx.y;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int c = lane & 15, qq = lane >> 4;
  const int64_t n = row_length(lengths, b, L);
  if (hist1) {
    for (int i = threadIdx.x; i < kHistBins; i += 256) lh[i] = 0u;
    __syncthreads();
  }
  const uint8_t* qb = q + (int64_t)b * H * kIdxD;
  const float* qsb = qs + (int64_t)b * H;
  const float* wb = w + (int64_t)b * H;
  i32x8_t qa[HT];
  float qsv[HT][4], wvv[HT][4];
  float bound = 0.f;
#pragma unroll
  for (int j = 0; j < HT; ++j) {
    qa[j] = load_fp8_operand(qb + (int64_t)(16 * j + c) * kIdxD, 0, qq);
    float l1 = abs_sum_fp8(qa[j]);
    l1 += __shfl_xor(l1, 16, 64);
    l1 += __shfl_xor(l1, 32, 64);
    if (qq == 0) bound += fabsf(wb[16 * j + c]) * fabsf(qsb[16 * j + c]) * l1;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      qsv[j][r] = qsb[16 * j + 4 * qq + r];
      wvv[j][r] = wb[16 * j + 4 * qq + r];
    }
  }
  const float qbound = wave_sum_f32(bound) * kBoundFactor;
  const int64_t n_tiles = (n + 15) / 16;
  const int64_t wave_id = (int64_t)blockIdx.x * 4 + wv, n_waves = (int64_t)gridDim.x * 4;
  const uint8_t* kb = k + (int64_t)b * L * kIdxD;
  const float* ksb = ks + (int64_t)b * L;
  for (int64_t tile0 = wave_id * U; tile0 < n_tiles; tile0 += n_waves * U) {
    i32x8_t kv[U];
    float ksv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t t = (tile0 + u) * 16 + c;
      const bool ok = t < n;
      kv[u] = ok ? load_fp8_operand_nt(kb + t * kIdxD, 0, qq) : i32x8_t{0, 0, 0, 0, 0, 0, 0, 0};
      ksv[u] = ok ? ksb[t] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float part = 0.f;
#pragma unroll
      for (int j = 0; j < HT; ++j) {
        const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
        const f32x4_t d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(qa[j], kv[u], z, 0, 0, 0, 127, 0, 127);
#pragma unroll
        for (int r = 0; r < 4; ++r) part = fmaf(fmaxf((d[r] * qsv[j][r]) * ksv[u], 0.f), wvv[j][r], part);
      }
      part += __shfl_xor(part, 16, 64);
      part += __shfl_xor(part, 32, 64);
      const int64_t t = (tile0 + u) * 16 + c;
      if (qq == 0 && t < n) {
        const float e = fabsf(ksv[u]) * qbound;
        const float l = part - e, h = part + e;
        lo[(int64_t)b * L + t] = l;
        hi[(int64_t)b * L + t] = h;
        if (hist1) atomicAdd(&lh[key_low_nan(l) >> 21], 1u);
      }
    }
  }
  if (hist1) {
    __syncthreads();
    for (int i = threadIdx.x; i < kHistBins; i += 256) {
      const uint32_t v = lh[i];
      if (v) atomicAdd(&hist1[(int64_t)b * kHistBins + i], v);
    }
  }
}

// Within a histogram of kHistBins digits (in `h`, LDS), find the digit that
// holds the rem-th largest element: the largest d with count(> d) < rem.
// Block of NT threads; returns digit and count(> digit) to every thread.
template <int NT>
__device__ void find_digit(const uint32_t* h, uint32_t rem, uint32_t* sh_out, uint32_t& digit, uint32_t& above) {
  constexpr int PER = kHistBins / NT;
  constexpr int NW = NT / 64;
  __shared__ uint32_t wtot[NW];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  // thread tid owns digits (top down) kHistBins-1-PER*tid ... kHistBins-PER*(tid+1)
  uint32_t local = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) local += h[kHistBins - 1 - (PER * tid + i)];
  const uint32_t incl = wave_incl_scan_u32(local);
  if (lane == 63) wtot[wv] = incl;
  __syncthreads();
  uint32_t base = 0;
  for (int i = 0; i < wv; ++i) base += wtot[i];
  uint32_t acc = base + incl - local;
  for (int i = 0; i < PER; ++i) {
    const uint32_t d = kHistBins - 1 - (PER * tid + i);
    const uint32_t cnt = h[d];
    if (acc < rem && rem <= acc + cnt) {
      sh_out[0] = d;
      sh_out[1] = acc;
    }
    acc += cnt;
  }
  __syncthreads();
  digit = sh_out[0];
  above = sh_out[1];
}

// Stage 2a: histogram of bits 20..10 of the lower-bound keys inside the top
// digit that holds the k-th largest.
__global__ void __launch_bounds__(256) dsa_hist2_kernel(const float* __restrict__ lo, const int32_t* __restrict__ lengths,
                                                        const uint32_t* __restrict__ hist1,
                                                        uint32_t* __restrict__ hist2, int64_t L, int topk) {
  __shared__ uint32_t lh[kHistBins];
  __shared__ uint32_t sh[2];
  const int b = blockIdx.y;
  const int64_t n = row_length(lengths, b, L);
  if (n <= topk) return;
  for (int i = threadIdx.x; i < kHistBins; i += 256) lh[i] = hist1[(int64_t)b * kHistBins + i];
  __syncthreads();
  uint32_t d1, above1;
  find_digit<256>(lh, (uint32_t)topk, sh, d1, above1);
  for (int i = threadIdx.x; i < kHistBins; i += 256) lh[i] = 0u;
  __syncthreads();
  const float* lob = lo + (int64_t)b * L;
  for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < n; t += (int64_t)gridDim.x * 256) {
    const uint32_t key = key_low_nan(lob[t]);
    if ((key >> 21) == d1) atomicAdd(&lh[(key >> 10) & (kHistBins - 1)], 1u);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < kHistBins; i += 256) {
    const uint32_t v = lh[i];
    if (v) atomicAdd(&hist2[(int64_t)b * kHistBins + i], v);
  }
}

// Exact canonical score of token t for one row; lanes are heads (lane < H).
// qw: this lane's 128 q code bytes; returns the score in every lane.
__device__ __forceinline__ float exact_score(const uint32_t (&qw)[32], const uint8_t* __restrict__ krow, float qs_h,
                                             float w_h, float ks_t, int H) {
  const u32x4_t* kp = reinterpret_cast<const u32x4_t*>(krow);
  double acc = 0.0;
#pragma unroll 1
  for (int v = 0; v < 8; ++v) {
    const u32x4_t kw = kp[v];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const f32x2_t q01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)qw[4 * v + e], false);
      const f32x2_t q23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)qw[4 * v + e], true);
      const f32x2_t k01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)kw[e], false);
      const f32x2_t k23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)kw[e], true);
      acc = fma((double)q01[0], (double)k01[0], acc);
      acc = fma((double)q01[1], (double)k01[1], acc);
      acc = fma((double)q23[0], (double)k23[0], acc);
      acc = fma((double)q23[1], (double)k23[1], acc);
    }
  }
  const float d = (float)acc;
  const float a = (d * qs_h) * ks_t;
  const float r = a > 0.f ? a : 0.f;
  const float term = r * w_h;
  float s = 0.f;
  for (int h = 0; h < H; ++h) s = s + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(term), h));
  return s;
}

// Stage 2b: exact scores.  With `hi` set, only tokens whose upper bound reaches
// tau are scored and appended as 64-bit keys (score key << 32 | ~index) to the
// row's candidate list; without it every token's score goes to `scores`.
__global__ void __launch_bounds__(256) dsa_rescore_kernel(
    const uint8_t* __restrict__ q, const float* __restrict__ qs, const uint8_t* __restrict__ k,
    const float* __restrict__ ks, const float* __restrict__ w, const int32_t* __restrict__ lengths,
    const float* __restrict__ hi, const uint32_t* __restrict__ hist1, const uint32_t* __restrict__ hist2,
    uint64_t* __restrict__ keys, uint32_t* __restrict__ counts, float* __restrict__ scores, int64_t L, int H,
    int topk) {
  __shared__ uint32_t lh[kHistBins];
  __shared__ uint32_t sh[2];
  const int b = blockIdx.y;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t n = row_length(lengths, b, L);
  uint32_t tau = 0u;
  if (hi && n > topk) {
    for (int i = threadIdx.x; i < kHistBins; i += 256) lh[i] = hist1[(int64_t)b * kHistBins + i];
    __syncthreads();
    uint32_t d1, above1, d2, above2;
    find_digit<256>(lh, (uint32_t)topk, sh, d1, above1);
    for (int i = threadIdx.x; i < kHistBins; i += 256) lh[i] = hist2[(int64_t)b * kHistBins + i];
    __syncthreads();
    find_digit<256>(lh, (uint32_t)topk - above1, sh, d2, above2);
    tau = (d1 << 21) | (d2 << 10);
  }
  const int hl = lane < H ? lane : 0;
  uint32_t qw[32];
  const u32x4_t* qrow = reinterpret_cast<const u32x4_t*>(q + ((int64_t)b * H + hl) * kIdxD);
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    const u32x4_t x = qrow[v];
    qw[4 * v] = x[0];
    qw[4 * v + 1] = x[1];
    qw[4 * v + 2] = x[2];
    qw[4 * v + 3] = x[3];
  }
  const float qs_h = qs[(int64_t)b * H + hl];
  const float w_h = lane < H ? w[(int64_t)b * H + hl] : 0.f;
  const uint8_t* kb = k + (int64_t)b * L * kIdxD;
  const float* ksb = ks + (int64_t)b * L;
  const int64_t wave_id = (int64_t)blockIdx.x * 4 + wv, n_waves = (int64_t)gridDim.x * 4;
  for (int64_t c0 = wave_id * 64; c0 < n; c0 += n_waves * 64) {
    const int64_t t = c0 + lane;
    bool cand = t < n;
    if (hi && cand) cand = key_high_nan(hi[(int64_t)b * L + t]) >= tau;
    uint64_t mask = __ballot(cand);
    while (mask) {
      const int bit = __builtin_ctzll(mask);
      mask &= mask - 1;
      const int64_t tc = c0 + bit;
      const float s = exact_score(qw, kb + tc * kIdxD, qs_h, w_h, ksb[tc], H);
      if (lane == 0) {
        if (hi) {
          const uint32_t pos = atomicAdd(&counts[b], 1u);
          keys[(int64_t)b * L + pos] = ((uint64_t)key_low_nan(s) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)tc);
        } else {
          scores[(int64_t)b * L + tc] = s;
        }
      }
    }
  }
}

// Stage 3: sort the candidates of one row by key (descending) and write the
// top-k indices (+offset), -1 past the row's valid count.
__global__ void __launch_bounds__(1024) dsa_topk_sort_kernel(const uint64_t* __restrict__ keys,
                                                             const uint32_t* __restrict__ counts,
                                                             const int32_t* __restrict__ lengths, int64_t L, int topk,
                                                             int offset, int32_t* __restrict__ idx_out) {
  __shared__ uint64_t sk[kSortCap];
  __shared__ uint32_t lh[256];
  __shared__ uint32_t sh[4];
  const int b = blockIdx.x, tid = threadIdx.x;
  const int64_t n = row_length(lengths, b, L);
  const int64_t cnt = min((int64_t)counts[b], n);
  const int kk = (int)min((int64_t)topk, cnt);
  const uint64_t* kb = keys + (int64_t)b * L;
  int m;  // number of keys placed in sk
  if (cnt <= kSortCap) {
    m = (int)cnt;
    for (int i = tid; i < kSortCap; i += 1024) sk[i] = i < m ? kb[i] : 0ull;
  } else {
    // radix select of the kk-th largest 64-bit key (keys are unique), 8 bits a pass
    uint64_t prefix = 0, pmask = 0;
    uint32_t rem = (uint32_t)kk;
    for (int shift = 56; shift >= 0; shift -= 8) {
      if (tid < 256) lh[tid] = 0u;
      __syncthreads();
      for (int64_t i = tid; i < cnt; i += 1024) {
        const uint64_t key = kb[i];
        if ((key & pmask) == prefix) atomicAdd(&lh[(key >> shift) & 255u], 1u);
      }
      __syncthreads();
      if (tid == 0) {
        uint32_t acc = 0;
        for (int d = 255; d >= 0; --d) {
          if (acc + lh[d] >= rem) {
            sh[0] = (uint32_t)d;
            sh[1] = acc;
            break;
          }
          acc += lh[d];
        }
      }
      __syncthreads();
      prefix |= (uint64_t)sh[0] << shift;
      pmask |= 255ull << shift;
      rem -= sh[1];
      __syncthreads();
    }
    if (tid == 0) sh[2] = 0u;
    for (int i = tid; i < kSortCap; i += 1024) sk[i] = 0ull;
    __syncthreads();
    for (int64_t i = tid; i < cnt; i += 1024) {
      const uint64_t key = kb[i];
      if (key >= prefix) {
        const uint32_t pos = atomicAdd(&sh[2], 1u);
        if (pos < (uint32_t)kSortCap) sk[pos] = key;
      }
    }
    __syncthreads();
    m = (int)min(sh[2], (uint32_t)kSortCap);
  }
  __syncthreads();
  int P = 64;
  while (P < m) P <<= 1;
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = tid; i < P / 2; i += 1024) {
        const int a = 2 * i - (i & (stride - 1));
        const int c2 = a + stride;
        const bool desc = (a & size) == 0;
        const uint64_t x = sk[a], y = sk[c2];
        if ((x < y) == desc) {
          sk[a] = y;
          sk[c2] = x;
        }
      }
      __syncthreads();
    }
  }
  for (int j = tid; j < topk; j += 1024) {
    int32_t v = -1;
    if (j < kk && j < m) v = (int32_t)(0xFFFFFFFFu - (uint32_t)sk[j]) + offset;
    idx_out[(int64_t)b * topk + j] = v;
  }
}

// ===================================================================== MLA
constexpr int kMlaBT = 64;        // tokens per online-softmax block
constexpr int kMlaDl = 512;       // latent (value) width
constexpr int kVtStride = 72;     // bf16 per V^T row (64 tokens + 8)

__device__ __forceinline__ f32x4_t mfma_bf16(const bf16x8_t a, const bf16x8_t b, const f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Where the KV of a row lives.  FP8: latent e4m3 [rows, 512] + f32 scales
// [rows, 512 >> sb_shift] + rope bf16 [rows, DR].  BF16: one bf16 tensor
// [rows, 512 + DR] (latent first).  Row r of the queries reads KV batch
// r / rows_per_kv.
struct MlaKv {
  const void* lat;
  const float* lat_s;
  const uint16_t* rope;
  int64_t n;
  int rows_per_kv;
  int sb_shift;
};

// One split (a contiguous slice of the selected tokens) of one query row and
// one group of 16*NW heads: partial (m, l, O) per head.  Waves own 16 heads;
// with at most 4 waves a workgroup runs one wave per SIMD, which leaves room
// for each wave's 16x512 fp32 O tile in accumulation registers.
template <int NW, bool FP8, int DR>
__global__ void __launch_bounds__(NW * 64) mla_decode_split_kernel(
    const uint16_t* __restrict__ q, const MlaKv kv, const int32_t* __restrict__ idx, float* __restrict__ part_o,
    float* __restrict__ part_ml, int topk, float scale, int chunk) {
  constexpr int DQK = kMlaDl + DR;
  constexpr int KS = DQK + 8;  // bf16 per K row in LDS: 16-byte reads of 16 rows hit distinct banks
  __shared__ __attribute__((aligned(16))) uint16_t Kt[kMlaBT * KS];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[kMlaDl * kVtStride];
  __shared__ int tok_ok[kMlaBT];
  const int H = NW * 16 * gridDim.z;
  const int split = blockIdx.x, b = blockIdx.y, S = gridDim.x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = tid >> 6, hw = (int)blockIdx.z * NW + wv;  // wave's 16-head group in the row
  const int c = lane & 15, qd = lane >> 4;
  const int head = 16 * hw + c;
  const int64_t n = kv.n;
  const int64_t kvb = b / kv.rows_per_kv;
  // q as the B operand of S^T = K Q^T: lane (c, qd) holds q[head][32 s + 8 qd .. +8]
  bf16x8_t qb[DQK / 32];
  {
    const uint16_t* qrow = q + ((int64_t)b * H + head) * DQK;
#pragma unroll
    for (int s = 0; s < DQK / 32; ++s) qb[s] = *reinterpret_cast<const bf16x8_t*>(qrow + 32 * s + 8 * qd);
  }
  f32x4_t o[kMlaDl / 16];
#pragma unroll
  for (int i = 0; i < kMlaDl / 16; ++i) o[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  const int t_begin = split * chunk;
  const int t_end = min(topk, t_begin + chunk);
  for (int t0 = t_begin; t0 < t_end; t0 += kMlaBT) {
    __syncthreads();
    // gather: (token, 64-wide latent segment) items -> bf16 rows of Kt and columns of Vt
    for (int item = tid; item < kMlaBT * 8; item += NW * 64) {
      const int tk = item >> 3, seg = item & 7;
      const int ti = t0 + tk;
      const int id = ti < t_end ? idx[(int64_t)b * topk + ti] : -1;
      const bool ok = id >= 0 && (int64_t)id < n;
      if (seg == 0) tok_ok[tk] = ok ? 1 : 0;
      uint32_t outw[32];
      if (ok) {
        const int64_t row = kvb * n + id;
        if constexpr (FP8) {
          const uint8_t* src = reinterpret_cast<const uint8_t*>(kv.lat) + row * kMlaDl + seg * 64;
          const float* ssrc = kv.lat_s + row * (kMlaDl >> kv.sb_shift);
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const u32x4_t x = *reinterpret_cast<const u32x4_t*>(src + 16 * v);
            const float sc = ssrc[(seg * 64 + 16 * v) >> kv.sb_shift];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const f32x2_t a = __builtin_amdgcn_cvt_pk_f32_fp8((int)x[e], false);
              const f32x2_t bb = __builtin_amdgcn_cvt_pk_f32_fp8((int)x[e], true);
              outw[8 * v + 2 * e] = (uint32_t)f32_bf16(a[0] * sc) | ((uint32_t)f32_bf16(a[1] * sc) << 16);
              outw[8 * v + 2 * e + 1] = (uint32_t)f32_bf16(bb[0] * sc) | ((uint32_t)f32_bf16(bb[1] * sc) << 16);
            }
          }
        } else {
          const uint16_t* src = reinterpret_cast<const uint16_t*>(kv.lat) + row * DQK + seg * 64;
#pragma unroll
          for (int v = 0; v < 8; ++v) {
            const u32x4_t x = *reinterpret_cast<const u32x4_t*>(src + 8 * v);
            outw[4 * v] = x[0];
            outw[4 * v + 1] = x[1];
            outw[4 * v + 2] = x[2];
            outw[4 * v + 3] = x[3];
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) outw[i] = 0u;
      }
      u32x4_t* kdst = reinterpret_cast<u32x4_t*>(Kt + tk * KS + seg * 64);
#pragma unroll
      for (int v = 0; v < 8; ++v) kdst[v] = u32x4_t{outw[4 * v], outw[4 * v + 1], outw[4 * v + 2], outw[4 * v + 3]};
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        Vt[(seg * 64 + 2 * i) * kVtStride + tk] = (uint16_t)(outw[i] & 0xFFFFu);
        Vt[(seg * 64 + 2 * i + 1) * kVtStride + tk] = (uint16_t)(outw[i] >> 16);
      }
    }
    if constexpr (DR > 0) {
      for (int item = tid; item < kMlaBT * (DR / 8); item += NW * 64) {
        const int tk = item / (DR / 8), pc = item % (DR / 8);
        const int ti = t0 + tk;
        const int id = ti < t_end ? idx[(int64_t)b * topk + ti] : -1;
        const bool ok = id >= 0 && (int64_t)id < n;
        u32x4_t v = {0u, 0u, 0u, 0u};
        if (ok) {
          const int64_t row = kvb * n + id;
          const uint16_t* src = FP8 ? kv.rope + row * DR : reinterpret_cast<const uint16_t*>(kv.lat) + row * DQK + kMlaDl;
          v = *reinterpret_cast<const u32x4_t*>(src + 8 * pc);
        }
        *reinterpret_cast<u32x4_t*>(Kt + tk * KS + kMlaDl + 8 * pc) = v;
      }
    }
    __syncthreads();
    // S^T tiles (rows = tokens 16 j + 4 qd + r, column = head c)
    f32x4_t st[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      st[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      const uint16_t* krow = Kt + (16 * j + c) * KS + 8 * qd;
#pragma unroll
      for (int s = 0; s < DQK / 32; ++s) st[j] = mfma_bf16(*reinterpret_cast<const bf16x8_t*>(krow + 32 * s), qb[s], st[j]);
    }
    float sc[4][4];
    float bm = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sc[j][r] = tok_ok[16 * j + 4 * qd + r] ? st[j][r] * scale : -INFINITY;
        bm = fmaxf(bm, sc[j][r]);
      }
    bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
    bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
    const float m_new = fmaxf(m_run, bm);
    const bool none = m_new == -INFINITY;
    const float alpha = none ? 1.f : __expf(m_run - m_new);
    float psum = 0.f;
    float p[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[j][r] = none ? 0.f : __expf(sc[j][r] - m_new);
        psum += p[j][r];
      }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;
    // rescale O rows (heads 4 qd + r of this wave) by their alpha
    float al[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) al[r] = __shfl(alpha, 4 * qd + r, 64);
#pragma unroll
    for (int dt = 0; dt < kMlaDl / 16; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) o[dt][r] *= al[r];
    // O += P V: k index 8 qd + j <-> token 32 s2 + 4 qd + j (j < 4), 32 s2 + 16 + 4 qd + j - 4 (j >= 4)
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      bf16x8_t pa;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pa[r] = __builtin_bit_cast(__bf16, f32_bf16(p[2 * s2][r]));
        pa[4 + r] = __builtin_bit_cast(__bf16, f32_bf16(p[2 * s2 + 1][r]));
      }
#pragma unroll
      for (int dt = 0; dt < kMlaDl / 16; ++dt) {
        const uint16_t* vrow = Vt + (16 * dt + c) * kVtStride + 32 * s2 + 4 * qd;
        const uint2 v0 = *reinterpret_cast<const uint2*>(vrow);
        const uint2 v1 = *reinterpret_cast<const uint2*>(vrow + 16);
        const u32x4_t vv = {v0.x, v0.y, v1.x, v1.y};
        o[dt] = mfma_bf16(pa, __builtin_bit_cast(bf16x8_t, vv), o[dt]);
      }
    }
  }
  // partials: O rows are heads 16 hw + 4 qd + r, columns 16 dt + c
  float* po = part_o + (((int64_t)b * S + split) * H) * kMlaDl;
#pragma unroll
  for (int dt = 0; dt < kMlaDl / 16; ++dt)
#pragma unroll
    for (int r = 0; r < 4; ++r) po[(int64_t)(16 * hw + 4 * qd + r) * kMlaDl + 16 * dt + c] = o[dt][r];
  if (qd == 0) {
    float* pml = part_ml + (((int64_t)b * S + split) * H + head) * 2;
    pml[0] = m_run;
    pml[1] = l_run;
  }
}

// Merge the splits of one (row, head) with the sink term and normalize.
__global__ void __launch_bounds__(128) mla_combine_kernel(const float* __restrict__ part_o,
                                                          const float* __restrict__ part_ml,
                                                          const float* __restrict__ sink, uint16_t* __restrict__ out,
                                                          int H, int S) {
  const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  float M = -INFINITY;
  for (int s = 0; s < S; ++s) M = fmaxf(M, part_ml[(((int64_t)b * S + s) * H + h) * 2]);
  uint16_t* dst = out + ((int64_t)b * H + h) * kMlaDl;
  if (M == -INFINITY) {
    for (int d = tid; d < kMlaDl; d += 128) dst[d] = 0;
    return;
  }
  float lsum = sink ? __expf(sink[h] - M) : 0.f;
  for (int s = 0; s < S; ++s) {
    const float* ml = part_ml + (((int64_t)b * S + s) * H + h) * 2;
    if (ml[0] != -INFINITY) lsum += ml[1] * __expf(ml[0] - M);
  }
  const float inv = 1.0f / lsum;
  for (int d = tid; d < kMlaDl; d += 128) {
    float acc = 0.f;
    for (int s = 0; s < S; ++s) {
      const float ms = part_ml[(((int64_t)b * S + s) * H + h) * 2];
      if (ms != -INFINITY) acc += part_o[(((int64_t)b * S + s) * H + h) * kMlaDl + d] * __expf(ms - M);
    }
    dst[d] = f32_bf16(acc * inv);
  }
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct IndexerWs {
  float *lo, *hi;
  uint64_t* keys;
  uint32_t *hist1, *hist2, *counts;
  size_t zero_words;  // hist1 .. counts, contiguous
};

static size_t indexer_ws(int64_t b, int64_t l, char* base, IndexerWs* w) {
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? base + off : nullptr;
    off += align256(bytes);
    return p;
  };
  float* lo = (float*)take((size_t)b * l * 4);
  float* hi = (float*)take((size_t)b * l * 4);
  uint64_t* keys = (uint64_t*)take((size_t)b * l * 8);
  const size_t zbytes = (size_t)b * kHistBins * 4 * 2 + (size_t)b * 4;
  uint32_t* z = (uint32_t*)take(zbytes);
  if (w) {
    w->lo = lo;
    w->hi = hi;
    w->keys = keys;
    w->hist1 = z;
    w->hist2 = z ? z + (size_t)b * kHistBins : nullptr;
    w->counts = z ? z + (size_t)b * kHistBins * 2 : nullptr;
    w->zero_words = zbytes / 4;
  }
  return off;
}

static int bound_grid(int64_t b, int64_t l) {
  // ~8 waves per CU over the chip, at least one 16-token tile per wave
  int64_t gx = (2048 + b - 1) / b;
  const int64_t tiles = (l + 15) / 16;
  gx = std::min<int64_t>(gx, (tiles + 3) / 4);
  return (int)std::max<int64_t>(gx, 1);
}

template <int HT>
static void launch_bound(const uint8_t* q, const float* qs, const uint8_t* k, const float* ks, const float* w,
                         const int32_t* lengths, float* lo, float* hi, uint32_t* hist1, int64_t b, int64_t l,
                         hipStream_t st) {
  dim3 grid((unsigned)bound_grid(b, l), (unsigned)b);
  hipLaunchKernelGGL((dsa_index_bound_kernel<HT, 4>), grid, dim3(256), 0, st, q, qs, k, ks, w, lengths, lo, hi, hist1,
                     l);
}

static int check_indexer(const void* q, const void* qs, const void* k, const void* ks, const void* w, int64_t b,
                         int64_t h, int64_t d, int64_t l) {
  MOSAIC_CHECK_ARG(q && qs && k && ks && w, "dsa_indexer: null pointer");
  MOSAIC_CHECK_ARG(d == kIdxD, "dsa_indexer: head dim %lld (128 supported)", (long long)d);
  MOSAIC_CHECK_ARG(h >= 16 && h <= 64 && h % 16 == 0, "dsa_indexer: heads %lld (16, 32, 48 or 64)", (long long)h);
  MOSAIC_CHECK_ARG(b >= 0 && b <= 65535 && l >= 0 && l < (1ll << 31), "dsa_indexer: shape out of range");
  return kOk;
}

static void dispatch_bound(const uint8_t* q, const float* qs, const uint8_t* k, const float* ks, const float* w,
                           const int32_t* lengths, float* lo, float* hi, uint32_t* hist1, int64_t b, int64_t h,
                           int64_t l, hipStream_t st) {
  switch (h / 16) {
    case 1: launch_bound<1>(q, qs, k, ks, w, lengths, lo, hi, hist1, b, l, st); break;
    case 2: launch_bound<2>(q, qs, k, ks, w, lengths, lo, hi, hist1, b, l, st); break;
    case 3: launch_bound<3>(q, qs, k, ks, w, lengths, lo, hi, hist1, b, l, st); break;
    default: launch_bound<4>(q, qs, k, ks, w, lengths, lo, hi, hist1, b, l, st); break;
  }
}

static int rescore_grid(int64_t b, int64_t l) {
  int64_t gx = (1024 + b - 1) / b;
  gx = std::min<int64_t>(gx, (l + 255) / 256);
  return (int)std::max<int64_t>(gx, 1);
}

struct MlaWs {
  float *part_o, *part_ml;
};

static int mla_splits(int64_t b, int64_t topk) {
  const int64_t blocks = (topk + kMlaBT - 1) / kMlaBT;
  int64_t s = (256 + b - 1) / b;
  s = std::min<int64_t>(s, blocks);
  s = std::min<int64_t>(s, 32);
  return (int)std::max<int64_t>(s, 1);
}

static size_t mla_ws(int64_t b, int64_t h, int64_t topk, char* base, MlaWs* w) {
  const int64_t S = mla_splits(b, topk);
  const size_t ob = align256((size_t)b * S * h * kMlaDl * 4);
  const size_t mb = align256((size_t)b * S * h * 2 * 4);
  if (w) {
    w->part_o = (float*)base;
    w->part_ml = (float*)(base + ob);
  }
  return ob + mb;
}

}  // namespace mosaic

using namespace mosaic;

extern "C" size_t mosaic_dsa_indexer_workspace_bytes(int64_t b, int64_t l) {
  if (b < 0 || l < 0) return 0;
  return indexer_ws(b, l, nullptr, nullptr);
}

extern "C" int mosaic_dsa_indexer_topk(const uint8_t* q, const float* q_s, const uint8_t* k, const float* k_s,
                                       const float* w, const int32_t* lengths, int32_t* idx_out, int64_t b, int64_t h,
                                       int64_t d, int64_t l, int64_t topk, int32_t offset, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  int rc = check_indexer(q, q_s, k, k_s, w, b, h, d, l);
  if (rc) return rc;
  MOSAIC_CHECK_ARG(idx_out, "dsa_indexer_topk: null output");
  MOSAIC_CHECK_ARG(topk >= 1 && topk <= kMaxTopk, "dsa_indexer_topk: topk %lld (1..%d)", (long long)topk, kMaxTopk);
  const size_t need = indexer_ws(b, l, nullptr, nullptr);
  MOSAIC_CHECK_ARG(workspace && workspace_bytes >= need, "dsa_indexer_topk: workspace %zu bytes < %zu",
                   workspace_bytes, need);
  if (b == 0) return kOk;
  hipStream_t st = (hipStream_t)stream;
  IndexerWs ws;
  indexer_ws(b, l, (char*)workspace, &ws);
  hipLaunchKernelGGL(dsa_zero_kernel, dim3((unsigned)((ws.zero_words + 255) / 256)), dim3(256), 0, st, ws.hist1,
                     (int64_t)ws.zero_words);
  if (l > 0) {
    dispatch_bound(q, q_s, k, k_s, w, lengths, ws.lo, ws.hi, ws.hist1, b, h, l, st);
    const int g2 = std::max(1, std::min<int>((int)((l + 255) / 256), (int)((1024 + b - 1) / b)));
    hipLaunchKernelGGL(dsa_hist2_kernel, dim3((unsigned)g2, (unsigned)b), dim3(256), 0, st, ws.lo, lengths, ws.hist1,
                       ws.hist2, l, (int)topk);
    hipLaunchKernelGGL(dsa_rescore_kernel, dim3((unsigned)rescore_grid(b, l), (unsigned)b), dim3(256), 0, st, q, q_s,
                       k, k_s, w, lengths, ws.hi, ws.hist1, ws.hist2, ws.keys, ws.counts, (float*)nullptr, l, (int)h,
                       (int)topk);
  }
  hipLaunchKernelGGL(dsa_topk_sort_kernel, dim3((unsigned)b), dim3(1024), 0, st, ws.keys, ws.counts, lengths, l,
                     (int)topk, (int)offset, idx_out);
  MOSAIC_RETURN_LAUNCH("dsa_indexer_topk");
}

extern "C" int mosaic_dsa_indexer_scores(const uint8_t* q, const float* q_s, const uint8_t* k, const float* k_s,
                                         const float* w, float* scores, int64_t b, int64_t h, int64_t d, int64_t l,
                                         void* stream) {
  int rc = check_indexer(q, q_s, k, k_s, w, b, h, d, l);
  if (rc) return rc;
  MOSAIC_CHECK_ARG(scores, "dsa_indexer_scores: null output");
  if (b == 0 || l == 0) return kOk;
  hipLaunchKernelGGL(dsa_rescore_kernel, dim3((unsigned)rescore_grid(b, l), (unsigned)b), dim3(256), 0,
                     (hipStream_t)stream, q, q_s, k, k_s, w, (const int32_t*)nullptr, (const float*)nullptr,
                     (const uint32_t*)nullptr, (const uint32_t*)nullptr, (uint64_t*)nullptr, (uint32_t*)nullptr,
                     scores, l, (int)h, 0);
  MOSAIC_RETURN_LAUNCH("dsa_indexer_scores");
}

extern "C" int mosaic_dsa_indexer_bounds(const uint8_t* q, const float* q_s, const uint8_t* k, const float* k_s,
                                         const float* w, float* lo, float* hi, int64_t b, int64_t h, int64_t d,
                                         int64_t l, void* stream) {
  int rc = check_indexer(q, q_s, k, k_s, w, b, h, d, l);
  if (rc) return rc;
  MOSAIC_CHECK_ARG(lo && hi, "dsa_indexer_bounds: null output");
  if (b == 0 || l == 0) return kOk;
  dispatch_bound(q, q_s, k, k_s, w, nullptr, lo, hi, nullptr, b, h, l, (hipStream_t)stream);
  MOSAIC_RETURN_LAUNCH("dsa_indexer_bounds");
}

extern "C" size_t mosaic_mla_decode_workspace_bytes(int64_t b, int64_t h, int64_t topk) {
  if (b < 0 || h < 0 || topk < 0) return 0;
  return mla_ws(b, h, topk, nullptr, nullptr);
}

namespace mosaic {

template <bool FP8, int DR>
static int launch_mla(const uint16_t* q, const MlaKv& kv, const float* sink, const int32_t* idx, uint16_t* out,
                      int64_t rows, int64_t h, int64_t topk, float softmax_scale, void* workspace, hipStream_t st) {
  MlaWs ws;
  mla_ws(rows, h, topk, (char*)workspace, &ws);
  const int S = mla_splits(rows, topk);
  const int blocks = (int)((topk + kMlaBT - 1) / kMlaBT);
  const int chunk = ((blocks + S - 1) / S) * kMlaBT;
  const int nw = h >= 64 ? 4 : (int)(h / 16);
  dim3 grid((unsigned)S, (unsigned)rows, (unsigned)(h / (16 * nw)));
  switch (nw) {
#define MLA_CASE(NWV)                                                                                                  \
  case NWV:                                                                                                            \
    hipLaunchKernelGGL((mla_decode_split_kernel<NWV, FP8, DR>), grid, dim3(NWV * 64), 0, st, q, kv, idx, ws.part_o,  \
                       ws.part_ml, (int)topk, softmax_scale, chunk);                                                   \
    break;
    MLA_CASE(1) MLA_CASE(2) MLA_CASE(3) MLA_CASE(4)
#undef MLA_CASE
  }
  MOSAIC_LAUNCH_CHECK("mla_decode_split");
  hipLaunchKernelGGL(mla_combine_kernel, dim3((unsigned)h, (unsigned)rows), dim3(128), 0, st, ws.part_o, ws.part_ml,
                     sink, out, (int)h, S);
  MOSAIC_RETURN_LAUNCH("mla_sparse_decode");
}

static int check_mla_common(int64_t rows, int64_t h, int64_t n, int64_t topk, int64_t rows_per_kv, void* workspace,
                            size_t workspace_bytes) {
  MOSAIC_CHECK_ARG(h >= 16 && h <= 256 && h % 16 == 0 && (h <= 64 || h % 64 == 0),
                   "mla_sparse_decode: heads %lld (16, 32, 48, 64 or a multiple of 64 up to 256)", (long long)h);
  MOSAIC_CHECK_ARG(rows >= 0 && rows <= 65535 && n >= 0 && n < (1ll << 31) && topk >= 0 && topk < (1ll << 24),
                   "mla_sparse_decode: shape out of range");
  MOSAIC_CHECK_ARG(rows_per_kv >= 1 && rows % rows_per_kv == 0, "mla_sparse_decode: rows %lld, rows_per_kv %lld",
                   (long long)rows, (long long)rows_per_kv);
  const size_t need = mla_ws(rows, h, topk, nullptr, nullptr);
  MOSAIC_CHECK_ARG(workspace && workspace_bytes >= need, "mla_sparse_decode: workspace %zu bytes < %zu",
                   workspace_bytes, need);
  return kOk;
}

}  // namespace mosaic

extern "C" int mosaic_mla_sparse_decode(const uint16_t* q, const uint8_t* kv_latent, const float* kv_scale,
                                        const uint16_t* kv_rope, const float* sink, const int32_t* idx, uint16_t* out,
                                        int64_t b, int64_t h, int64_t n, int64_t topk, int64_t d_latent,
                                        int64_t d_rope, int64_t scale_block, float softmax_scale, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  MOSAIC_CHECK_ARG(q && kv_latent && kv_scale && kv_rope && idx && out, "mla_sparse_decode: null pointer");
  MOSAIC_CHECK_ARG(d_latent == kMlaDl && d_rope == 64, "mla_sparse_decode: dims %lld+%lld (512+64 supported)",
                   (long long)d_latent, (long long)d_rope);
  int sb_shift = -1;
  for (int s = 4; s <= 9; ++s)
    if (scale_block == (1ll << s)) sb_shift = s;
  MOSAIC_CHECK_ARG(sb_shift >= 0, "mla_sparse_decode: scale_block %lld (16..512, power of two)",
                   (long long)scale_block);
  int rc = check_mla_common(b, h, n, topk, 1, workspace, workspace_bytes);
  if (rc) return rc;
  if (b == 0) return kOk;
  const MlaKv kv{kv_latent, kv_scale, kv_rope, n, 1, sb_shift};
  return launch_mla<true, 64>(q, kv, sink, idx, out, b, h, topk, softmax_scale, workspace, (hipStream_t)stream);
}

extern "C" int mosaic_mla_sparse_decode_bf16(const uint16_t* q, const uint16_t* kv, const float* sink,
                                             const int32_t* idx, uint16_t* out, int64_t rows, int64_t h, int64_t n,
                                             int64_t topk, int64_t d, int64_t rows_per_kv, float softmax_scale,
                                             void* workspace, size_t workspace_bytes, void* stream) {
  MOSAIC_CHECK_ARG(q && kv && idx && out, "mla_sparse_decode_bf16: null pointer");
  MOSAIC_CHECK_ARG(d == 512 || d == 576, "mla_sparse_decode_bf16: head dim %lld (512 or 576)", (long long)d);
  int rc = check_mla_common(rows, h, n, topk, rows_per_kv, workspace, workspace_bytes);
  if (rc) return rc;
  if (rows == 0) return kOk;
  const MlaKv kvd{kv, nullptr, nullptr, n, (int)rows_per_kv, 0};
  if (d == 576)
    return launch_mla<false, 64>(q, kvd, sink, idx, out, rows, h, topk, softmax_scale, workspace, (hipStream_t)stream);
  return launch_mla<false, 0>(q, kvd, sink, idx, out, rows, h, topk, softmax_scale, workspace, (hipStream_t)stream);
}
