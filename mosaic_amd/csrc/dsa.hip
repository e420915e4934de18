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
//      k + a few tens of percent) get the exact score, then the k best are
//      selected (radix select on unique (score, -index) keys) and ranked.
// Exact dots on the integer MFMA: every e4m3 value times 512 is an integer X
// with |X| <= 229376, written X = L2*2^14 + L1*2^7 + L0 with L0, L1 in [0, 127]
// and L2 in [-14, 14] (three int8 limbs).  The nine limb products accumulate in
// int32 (v_mfma_i32_16x16x64_i8, exact), grouped by weight into five sums, and
// their weighted fp64 sum (< 2^43, integer) is 2^18 times the exact dot.  (The
// fp8 MFMA is not used here: its fp32 accumulation drops low-order bits once the
// operands span more than about four binades.)
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

// lanes with `active` add 1 to lh[bin]; lanes that share a bin are merged
// first, so a wave issues one LDS atomic per distinct bin
__device__ __forceinline__ void lds_hist_add(uint32_t* lh, uint32_t bin, bool active) {
  const int lane = threadIdx.x & 63;
  uint64_t pending = __ballot(active);
  while (pending) {
    const int leader = __builtin_ctzll(pending);
    const uint32_t lb = (uint32_t)__builtin_amdgcn_readlane((int)bin, leader);
    const uint64_t same = __ballot(bin == lb) & pending;
    if (lane == leader) atomicAdd(&lh[lb], (uint32_t)__builtin_popcountll(same));
    pending &= ~same;
  }
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
  auto load_group = [&](int64_t tile0, i32x8_t (&kv)[U], float (&ksv)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t t = (tile0 + u) * 16 + c;
      const bool ok = t < n;
      kv[u] = ok ? load_fp8_operand_nt(kb + t * kIdxD, 0, qq) : i32x8_t{0, 0, 0, 0, 0, 0, 0, 0};
      ksv[u] = ok ? ksb[t] : 0.f;
    }
  };
  const int64_t step = n_waves * U;
  auto compute_group = [&](int64_t tile0, const i32x8_t (&kv)[U], const float (&ksv)[U]) {
    f32x4_t d[U][HT];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < HT; ++j) {
        const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
        d[u][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(qa[j], kv[u], z, 0, 0, 0, 127, 0, 127);
      }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float part = 0.f;
#pragma unroll
      for (int j = 0; j < HT; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) part = fmaf(fmaxf((d[u][j][r] * qsv[j][r]) * ksv[u], 0.f), wvv[j][r], part);
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
  };
  // two register sets in ping-pong: the next group's loads are in flight while
  // the current one computes
  i32x8_t ka[U], kb2[U];
  float sa[U], sb[U];
  int64_t tile0 = wave_id * U;
  if (tile0 < n_tiles) load_group(tile0, ka, sa);
  for (; tile0 < n_tiles; tile0 += 2 * step) {
    const bool more = tile0 + step < n_tiles;
    if (more) load_group(tile0 + step, kb2, sb);
    compute_group(tile0, ka, sa);
    if (!more) break;
    if (tile0 + 2 * step < n_tiles) load_group(tile0 + 2 * step, ka, sa);
    compute_group(tile0 + step, kb2, sb);
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

typedef __attribute__((ext_vector_type(4))) int i32x4_v;

// 16 e4m3 codes -> three int8 limb vectors: 512 v = L2 2^14 + L1 2^7 + L0
__device__ __forceinline__ void e4m3_limbs(const u32x4_t x, i32x4_v (&o)[3]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f32x2_t a = __builtin_amdgcn_cvt_pk_f32_fp8((int)x[i], false);
    const f32x2_t c = __builtin_amdgcn_cvt_pk_f32_fp8((int)x[i], true);
    const int v0 = (int)(a[0] * 512.f), v1 = (int)(a[1] * 512.f);
    const int v2 = (int)(c[0] * 512.f), v3 = (int)(c[1] * 512.f);
    o[0][i] = (v0 & 127) | ((v1 & 127) << 8) | ((v2 & 127) << 16) | ((v3 & 127) << 24);
    o[1][i] = ((v0 >> 7) & 127) | (((v1 >> 7) & 127) << 8) | (((v2 >> 7) & 127) << 16) | (((v3 >> 7) & 127) << 24);
    o[2][i] = ((v0 >> 14) & 255) | (((v1 >> 14) & 255) << 8) | (((v2 >> 14) & 255) << 16) | ((v3 >> 14) << 24);
  }
}

__device__ __forceinline__ i32x4_v mfma_i8(const i32x4_v a, const i32x4_v b, const i32x4_v c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// Stage 2b: exact scores.  A workgroup owns `range` consecutive tokens of one
// row.  With `hi` set it keeps the tokens whose upper bound reaches tau (LDS
// list), scores them 16 at a time on the MFMA (lanes = 16 candidates x 4 head
// groups) and appends 64-bit keys (score key << 32 | ~index) to the row's list;
// without `hi` it scores every token into `scores`.
constexpr int kRsMaxRange = 4096;
__global__ void __launch_bounds__(256) dsa_rescore_kernel(
    const uint8_t* __restrict__ q, const float* __restrict__ qs, const uint8_t* __restrict__ k,
    const float* __restrict__ ks, const float* __restrict__ w, const int32_t* __restrict__ lengths,
    const float* __restrict__ hi, const uint32_t* __restrict__ hist1, const uint32_t* __restrict__ hist2,
    uint64_t* __restrict__ keys, uint32_t* __restrict__ counts, float* __restrict__ scores, int64_t L, int H,
    int topk, int range) {
  __shared__ uint32_t lh[kHistBins];
  __shared__ uint32_t lh2[kHistBins];
  __shared__ uint32_t sh[2];
  __shared__ int cand[kRsMaxRange];
  __shared__ uint32_t ncand;
  __shared__ float terms[4][16][65];
  const int b = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int c = lane & 15, qd = lane >> 4;
  const int64_t n = row_length(lengths, b, L);
  const int64_t t_begin = (int64_t)blockIdx.x * range;
  if (t_begin >= n) return;
  const int64_t t_end = min(n, t_begin + range);
  uint32_t tau = 0u;
  if (hi && n > topk) {
    for (int i = tid; i < kHistBins; i += 256) {
      lh[i] = hist1[(int64_t)b * kHistBins + i];
      lh2[i] = hist2[(int64_t)b * kHistBins + i];
    }
    __syncthreads();
    uint32_t d1, above1, d2, above2;
    find_digit<256>(lh, (uint32_t)topk, sh, d1, above1);
    find_digit<256>(lh2, (uint32_t)topk - above1, sh, d2, above2);
    tau = (d1 << 21) | (d2 << 10);
  }
  if (tid == 0) ncand = 0u;
  __syncthreads();
  for (int64_t c0 = t_begin + 64 * wv; c0 < t_end; c0 += 256) {
    const int64_t t = c0 + lane;
    bool ok = t < t_end;
    if (hi && ok) ok = key_high_nan(hi[(int64_t)b * L + t]) >= tau;
    const uint64_t mask = __ballot(ok);
    const int nc = __builtin_popcountll(mask);
    if (nc == 0) continue;
    uint32_t base = 0u;
    if (lane == 0) base = atomicAdd(&ncand, (uint32_t)nc);
    base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
    const int pos = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
    if (ok) cand[base + pos] = (int)t;
  }
  __syncthreads();
  const int C = (int)ncand;
  const int HT = H / 16;
  // A operands (rows = heads 16 j + c) as int8 limbs of dims 64 ch + 16 qd ..+16;
  // per-lane constants of the D layout (heads 16 j + 4 qd + r)
  i32x4_v ql[4][2][3];
  float qsv[4][4], wvv[4][4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int hr = j < HT ? 16 * j + c : 0;
    const uint8_t* qrow = q + ((int64_t)b * H + hr) * kIdxD + 16 * qd;
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) e4m3_limbs(*reinterpret_cast<const u32x4_t*>(qrow + 64 * ch), ql[j][ch]);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int hd = j < HT ? 16 * j + 4 * qd + r : 0;
      qsv[j][r] = qs[(int64_t)b * H + hd];
      wvv[j][r] = w[(int64_t)b * H + hd];
    }
  }
  const uint8_t* kb = k + (int64_t)b * L * kIdxD;
  const float* ksb = ks + (int64_t)b * L;
  struct Batch {
    u32x4_t x[2];
    float ks;
    int t;
  };
  auto load_batch = [&](int bt, Batch& o) {
    const int i = bt * 16 + c;
    const bool ok = i < C;
    o.t = ok ? cand[i] : -1;
    o.ks = ok ? ksb[o.t] : 0.f;
#pragma unroll
    for (int ch = 0; ch < 2; ++ch)
      o.x[ch] = ok ? *reinterpret_cast<const u32x4_t*>(kb + (int64_t)o.t * kIdxD + 64 * ch + 16 * qd)
                   : u32x4_t{0u, 0u, 0u, 0u};
  };
  auto score_batch = [&](int bt, const Batch& in) {
    i32x4_v kl[2][3];
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) e4m3_limbs(in.x[ch], kl[ch]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (j >= HT) break;
      i32x4_v g[5];
#pragma unroll
      for (int m = 0; m < 5; ++m) g[m] = i32x4_v{0, 0, 0, 0};
#pragma unroll
      for (int ch = 0; ch < 2; ++ch)
#pragma unroll
        for (int la = 0; la < 3; ++la)
#pragma unroll
          for (int lb = 0; lb < 3; ++lb) g[la + lb] = mfma_i8(ql[j][ch][la], kl[ch][lb], g[la + lb]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        double x = (double)g[4][r];
        x = fma(x, 128.0, (double)g[3][r]);
        x = fma(x, 128.0, (double)g[2][r]);
        x = fma(x, 128.0, (double)g[1][r]);
        x = fma(x, 128.0, (double)g[0][r]);
        const float d = (float)(x * 0x1p-18);
        const float a = (d * qsv[j][r]) * in.ks;
        const float rr = a > 0.f ? a : 0.f;
        terms[wv][c][16 * j + 4 * qd + r] = rr * wvv[j][r];
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    const int nvalid = min(16, C - bt * 16);
    uint32_t base = 0u;
    if (hi && lane == 0) base = atomicAdd(&counts[b], (uint32_t)nvalid);
    base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
    if (qd == 0 && in.t >= 0) {
      float sc = 0.f;
      for (int h = 0; h < H; ++h) sc = sc + terms[wv][c][h];
      if (hi)
        keys[(int64_t)b * L + base + c] =
            ((uint64_t)key_low_nan(sc) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)in.t);
      else
        scores[(int64_t)b * L + in.t] = sc;
    }
    __builtin_amdgcn_wave_barrier();
  };
  // ping-pong over this wave's batches (bt = wv, wv + 4, ...)
  Batch ba, bb;
  int bt = wv;
  if (bt * 16 < C) load_batch(bt, ba);
  for (; bt * 16 < C; bt += 8) {
    const bool more = (bt + 4) * 16 < C;
    if (more) load_batch(bt + 4, bb);
    score_batch(bt, ba);
    if (!more) break;
    if ((bt + 8) * 16 < C) load_batch(bt + 8, ba);
    score_batch(bt + 4, bb);
  }
}

// Stage 3a: radix-select the kk best keys of one row (keys are unique) and
// store them, unordered, in sel[b][0..kk).
__global__ void __launch_bounds__(1024) dsa_select_kernel(const uint64_t* __restrict__ keys,
                                                          const uint32_t* __restrict__ counts,
                                                          const int32_t* __restrict__ lengths, int64_t L, int topk,
                                                          uint64_t* __restrict__ sel) {
  __shared__ uint64_t sk[kSortCap];
  __shared__ uint32_t lh[256];
  __shared__ uint32_t sh[4];
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
  const int64_t n = row_length(lengths, b, L);
  const int64_t cnt = min((int64_t)counts[b], n);
  const int kk = (int)min((int64_t)topk, cnt);
  const uint64_t* kb = keys + (int64_t)b * L;
  uint64_t* out = sel + (int64_t)b * kSortCap;
  if (cnt <= kk) {
    for (int i = tid; i < cnt; i += 1024) out[i] = kb[i];
    return;
  }
  const bool in_lds = cnt <= kSortCap;
  if (in_lds)
    for (int i = tid; i < cnt; i += 1024) sk[i] = kb[i];
  uint64_t prefix = 0, pmask = 0;
  uint32_t rem = (uint32_t)kk;
  for (int shift = 56; shift >= 0; shift -= 8) {
    if (tid < 256) lh[tid] = 0u;
    __syncthreads();
    for (int64_t i = tid; i < cnt; i += 1024) {
      const uint64_t key = in_lds ? sk[i] : kb[i];
      if ((key & pmask) == prefix) atomicAdd(&lh[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid < 64) {  // one wave finds the digit: 4 bins per lane, scanned from the top
      uint32_t cnt4[4], local = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        cnt4[i] = lh[255 - (4 * lane + i)];
        local += cnt4[i];
      }
      uint32_t acc = wave_incl_scan_u32(local) - local;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (acc < rem && rem <= acc + cnt4[i]) {
          sh[0] = 255u - (uint32_t)(4 * lane + i);
          sh[1] = acc;
        }
        acc += cnt4[i];
      }
    }
    __syncthreads();
    prefix |= (uint64_t)sh[0] << shift;
    pmask |= 255ull << shift;
    rem -= sh[1];
    const bool whole = lh[sh[0]] == rem;  // every key with this prefix is selected
    __syncthreads();
    if (whole) break;
  }
  if (tid == 0) sh[2] = 0u;
  __syncthreads();
  for (int64_t i = tid; i < cnt; i += 1024) {
    const uint64_t key = in_lds ? sk[i] : kb[i];
    if (key >= prefix) {
      const uint32_t pos = atomicAdd(&sh[2], 1u);
      if (pos < (uint32_t)kk) out[pos] = key;
    }
  }
}

// Stage 3b: rank of each selected key among the row's kk selected keys (the
// number of larger keys) -> output slot.  A workgroup takes 64 slots; its four
// waves count against four quarters of the keys.
__global__ void __launch_bounds__(256) dsa_rank_kernel(const uint64_t* __restrict__ sel,
                                                       const uint32_t* __restrict__ counts,
                                                       const int32_t* __restrict__ lengths, int64_t L, int topk,
                                                       int offset, int32_t* __restrict__ idx_out) {
  __shared__ uint64_t sk[kSortCap];
  __shared__ uint32_t part[4][64];
  const int b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t n = row_length(lengths, b, L);
  const int kk = (int)min((int64_t)topk, min((int64_t)counts[b], n));
  const int e0 = blockIdx.x * 64;
  int32_t* dst = idx_out + (int64_t)b * topk;
  if (tid < 64 && e0 + tid < topk && e0 + tid >= kk) dst[e0 + tid] = -1;
  if (e0 >= kk) return;
  const uint64_t* sb = sel + (int64_t)b * kSortCap;
  for (int i = tid; i < kk; i += 256) sk[i] = sb[i];
  __syncthreads();
  const int e = e0 + lane;
  const uint64_t mine = e < kk ? sk[e] : ~0ull;
  const int f0 = (int)((int64_t)kk * wv / 4), f1 = (int)((int64_t)kk * (wv + 1) / 4);
  uint32_t r = 0;
  int f = f0;
  for (; f + 8 <= f1; f += 8) {  // eight keys per step, four independent LDS reads
    uint64_t v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = sk[f + i];
#pragma unroll
    for (int i = 0; i < 8; ++i) r += v[i] > mine ? 1u : 0u;
  }
  for (; f < f1; ++f) r += sk[f] > mine ? 1u : 0u;
  part[wv][lane] = r;
  __syncthreads();
  if (wv == 0 && e < kk) {
    const uint32_t rank = part[0][lane] + part[1][lane] + part[2][lane] + part[3][lane];
    dst[rank] = (int32_t)(0xFFFFFFFFu - (uint32_t)mine) + offset;
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
  __shared__ int tok_id[kMlaBT];
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
    if (tid < kMlaBT) {
      const int ti = t0 + tid;
      const int id = ti < t_end ? idx[(int64_t)b * topk + ti] : -1;
      tok_id[tid] = (id >= 0 && (int64_t)id < n) ? id : -1;
    }
    __syncthreads();
    // gather: (token, 64-wide latent segment) items -> bf16 rows of Kt and columns of Vt
    for (int item = tid; item < kMlaBT * 8; item += NW * 64) {
      const int tk = item >> 3, seg = item & 7;
      const int id = tok_id[tk];
      const bool ok = id >= 0;
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
        const int id = tok_id[tk];
        const bool ok = id >= 0;
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
    for (int j = 0; j < 4; ++j) st[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < DQK / 32; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        st[j] = mfma_bf16(*reinterpret_cast<const bf16x8_t*>(Kt + (16 * j + c) * KS + 8 * qd + 32 * s), qb[s], st[j]);
    float sc[4][4];
    float bm = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sc[j][r] = tok_id[16 * j + 4 * qd + r] >= 0 ? st[j][r] * scale : -INFINITY;
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

// Merge the splits of one (row, head) with the sink term and normalize: one
// wave turns the split maxima/sums into weights, then each thread blends
// four consecutive output columns over the splits.
__global__ void __launch_bounds__(128) mla_combine_kernel(const float* __restrict__ part_o,
                                                          const float* __restrict__ part_ml,
                                                          const float* __restrict__ sink, uint16_t* __restrict__ out,
                                                          int H, int S) {
  __shared__ float wgt[64];
  const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  if (tid < 64) {
    const bool ok = tid < S;
    const float m = ok ? part_ml[(((int64_t)b * S + tid) * H + h) * 2] : -INFINITY;
    const float l = ok ? part_ml[(((int64_t)b * S + tid) * H + h) * 2 + 1] : 0.f;
    float M = m;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
    const float e = (m == -INFINITY) ? 0.f : __expf(m - M);
    const float lsum = wave_sum_f32(l * e) + ((sink && M != -INFINITY) ? __expf(sink[h] - M) : 0.f);
    wgt[tid] = (M == -INFINITY) ? 0.f : e / lsum;
  }
  __syncthreads();
  const int d = 4 * tid;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  const float* po = part_o + ((int64_t)b * S * H + h) * kMlaDl + d;
#pragma unroll 8
  for (int s = 0; s < S; ++s) {
    const f32x4_t v = *reinterpret_cast<const f32x4_t*>(po + (int64_t)s * H * kMlaDl);
    acc += wgt[s] * v;
  }
  uint16_t* dst = out + ((int64_t)b * H + h) * kMlaDl + d;
  const uint32_t w0 = (uint32_t)f32_bf16(acc[0]) | ((uint32_t)f32_bf16(acc[1]) << 16);
  const uint32_t w1 = (uint32_t)f32_bf16(acc[2]) | ((uint32_t)f32_bf16(acc[3]) << 16);
  *reinterpret_cast<uint2*>(dst) = uint2{w0, w1};
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct IndexerWs {
  float *lo, *hi;
  uint64_t *keys, *sel;
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
  uint64_t* sel = (uint64_t*)take((size_t)b * kSortCap * 8);
  const size_t zbytes = (size_t)b * kHistBins * 4 * 2 + (size_t)b * 4;
  uint32_t* z = (uint32_t*)take(zbytes);
  if (w) {
    w->lo = lo;
    w->hi = hi;
    w->keys = keys;
    w->sel = sel;
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

// tokens per rescoring workgroup: about 512 workgroups over the batch, a
// multiple of 64, at most the LDS candidate list
static int rescore_range(int64_t b, int64_t l) {
  const int64_t target = std::max<int64_t>(1, 512 / std::max<int64_t>(b, 1));
  int64_t r = (l + target - 1) / target;
  r = (r + 63) / 64 * 64;
  return (int)std::min<int64_t>(std::max<int64_t>(r, 64), kRsMaxRange);
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
    const int range = rescore_range(b, l);
    hipLaunchKernelGGL(dsa_rescore_kernel, dim3((unsigned)((l + range - 1) / range), (unsigned)b), dim3(256), 0, st, q,
                       q_s, k, k_s, w, lengths, ws.hi, ws.hist1, ws.hist2, ws.keys, ws.counts, (float*)nullptr, l,
                       (int)h, (int)topk, range);
  }
  hipLaunchKernelGGL(dsa_select_kernel, dim3((unsigned)b), dim3(1024), 0, st, ws.keys, ws.counts, lengths, l, (int)topk,
                     ws.sel);
  hipLaunchKernelGGL(dsa_rank_kernel, dim3((unsigned)((topk + 63) / 64), (unsigned)b), dim3(256), 0, st, ws.sel,
                     ws.counts, lengths, l, (int)topk, (int)offset, idx_out);
  MOSAIC_RETURN_LAUNCH("dsa_indexer_topk");
}

extern "C" int mosaic_dsa_indexer_scores(const uint8_t* q, const float* q_s, const uint8_t* k, const float* k_s,
                                         const float* w, float* scores, int64_t b, int64_t h, int64_t d, int64_t l,
                                         void* stream) {
  int rc = check_indexer(q, q_s, k, k_s, w, b, h, d, l);
  if (rc) return rc;
  MOSAIC_CHECK_ARG(scores, "dsa_indexer_scores: null output");
  if (b == 0 || l == 0) return kOk;
  const int range = rescore_range(b, l);
  hipLaunchKernelGGL(dsa_rescore_kernel, dim3((unsigned)((l + range - 1) / range), (unsigned)b), dim3(256), 0,
                     (hipStream_t)stream, q, q_s, k, k_s, w, (const int32_t*)nullptr, (const float*)nullptr,
                     (const uint32_t*)nullptr, (const uint32_t*)nullptr, (uint64_t*)nullptr, (uint32_t*)nullptr,
                     scores, l, (int)h, 0, range);
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
