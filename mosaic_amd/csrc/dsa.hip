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
//   1. dsa_index_bound_kernel streams k once, converts the codes to bf16
//      (exact) and takes the dots on the bf16 MFMA, whose sums behave like fp32
//      additions; it writes per token an interval [lo, hi] that contains the
//      canonical score.  The half-width is
//        2^-14 * 448 * |k_scale[t]| * sum_h |w_h| |q_scale[h]| ||q_h||_1 * (1 + 2^-9),
//      where 448 ||q_h||_1 bounds sum_d |q_hd k_td| (|k| <= 448): at least 8x the
//      error of any fp32 summation order of the 128 products (< 2^-17 of their
//      absolute sum) and 4x that error plus the rounding of the remaining steps.
//      (The fp8 MFMA does not allow such a bound: it adds each run of 8 products
//      aligned to the largest one and keeps only about 14 bits below it, so a
//      small product next to a large one is dropped.)
//   2. tau = the lower edge of the histogram digit (top kHistBits bits of the
//      order key) that holds the k-th largest lo.  Any token with hi < tau is
//      beaten by k tokens whose lo >= tau, so the true top-k lies inside
//      {t : hi >= tau}.  Those candidates (typically k + a few tens of percent)
//      get the exact score, then the k best are ranked (dsa_finish_kernel).
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
//   e4m3 * scale -> bf16, rope bf16], v_t = latent.  Online softmax over 32-token
//   blocks in each of several token splits, then a combine over splits.
#include <algorithm>

#include "common.h"
#include "../../include/mosaic_amd.h"

namespace mosaic {

// ===================================================================== indexer
constexpr int kIdxD = 128;
constexpr int kHistBits = 13;       // lower-bound key digits: sign, exponent, 4 mantissa bits
constexpr int kHistBins = 1 << kHistBits;
constexpr int kHistShift = 32 - kHistBits;
constexpr int kSortCap = 4096;      // candidates ranked in LDS
constexpr int kMaxTopk = 4096;
constexpr float kBoundFactor = 448.0f / 16384.0f * (1.0f + 1.0f / 512.0f);

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

// Sum over the 64 lanes (all lanes active) on DPP moves (the wave_max_u32
// steps), broadcast from lane 63
__device__ __forceinline__ float wave_sum_f32(float v) {
  v += __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(v), 0xB1, 0xF));
  v += __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(v), 0x4E, 0xF));
  v += __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(v), 0x141, 0xF));
  v += __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(v), 0x140, 0xF));
  v += __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(v), 0x142, 0xA));
  v += __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(v), 0x143, 0xC));
  return __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(v), 63));
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

// Sum over the four lanes c, c + 16, c + 32, c + 48 of a 16-column MFMA result
// (v_permlane16/32_swap: no LDS round trip), the same value in all four.
__device__ __forceinline__ float sum_lane_quad(float x) {
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float y = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}

// The 32 e4m3 codes of one fp8 MFMA operand lane -> 4 x 8 bf16 (exact), chunk
// kc = code bytes [8 kc, 8 kc + 8); `neg` flips every sign.
__device__ __forceinline__ void fp8x32_to_bf16(const i32x8_t v, bf16x8_t (&out)[4], bool neg) {
  const uint32_t flip = neg ? 0x80008000u : 0u;
#pragma unroll
  for (int kc = 0; kc < 4; ++kc) {
    uint32_t p[4];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const bf16x2_t lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[2 * kc + h], 1.0f, false);
      const bf16x2_t hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[2 * kc + h], 1.0f, true);
      p[2 * h] = __builtin_bit_cast(uint32_t, lo) ^ flip;
      p[2 * h + 1] = __builtin_bit_cast(uint32_t, hi) ^ flip;
    }
    const u32x4_t pv = {p[0], p[1], p[2], p[3]};
    out[kc] = __builtin_bit_cast(bf16x8_t, pv);
  }
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

// Buffer resource over `records` bytes from `base` (raw addressing): loads past
// the range read zero and stores past it are dropped.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, int records) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, records, 0x00020000);
}

// Stage 1: fp8 MFMA scores with a rigorous interval; optional histogram of the
// top kHistBits bits of the lower-bound keys (per row, merged with global atomics per
// workgroup).  grid (gx, B): wave wid of row b takes the groups g = wid, wid +
// nw, ... of U 16-token tiles and streams them through a register ring of D
// groups.  Each group's loads and stores go through buffer resources that end
// at the row's length, so tokens past it read as zero and are not written: the
// ring issues every load unconditionally and its waits stay exact.  `lo` may
// be null (the top-k path reads only the upper bounds and the histogram).
template <int HT, int U, int D>
__global__ void __launch_bounds__(256) dsa_index_bound_kernel(
    const uint8_t* __restrict__ q, const float* __restrict__ qs, const uint8_t* __restrict__ k,
    const float* __restrict__ ks, const float* __restrict__ w, const int32_t* __restrict__ lengths,
    float* __restrict__ lo, float* __restrict__ hi, uint32_t* __restrict__ hist1, int64_t L, int kdiv,
    int64_t kstride) {
  constexpr int H = HT * 16;
  constexpr int GT = 16 * U;  // tokens per group
  constexpr int kQv = H * kIdxD / 16;  // 16-byte pieces of the q row
  __shared__ uint32_t lh[kHistBins];
  __shared__ u32x4_t qsh[kQv];
  __shared__ float qssh[H], wsh[H];
  const int b = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int c = lane & 15, qq = lane >> 4;
  const int64_t n = row_length(lengths, b, L);
  // the q row, its scales and weights are loaded once per workgroup (first,
  // so that staging them waits for nothing else) and read from LDS below
  u32x4_t qv[(kQv + 255) / 256];
  {
    const u32x4_t* q4 = reinterpret_cast<const u32x4_t*>(q + (int64_t)b * H * kIdxD);
#pragma unroll
    for (int i = 0; i < (kQv + 255) / 256; ++i)
      if (kQv % 256 == 0 || threadIdx.x + 256 * i < kQv) qv[i] = q4[threadIdx.x + 256 * i];
  }
  const float qsl = threadIdx.x < H ? qs[(int64_t)b * H + threadIdx.x] : 0.f;
  const float wl = threadIdx.x < H ? w[(int64_t)b * H + threadIdx.x] : 0.f;
  const int64_t n_groups = (n + GT - 1) / GT;
  const int64_t nw = (int64_t)gridDim.x * 4, wid = (int64_t)blockIdx.x * 4 + wv;
  const int64_t iters = wid < n_groups ? (n_groups - 1 - wid) / nw + 1 : 0;
  // kdiv query rows share one key cache; caches start kstride tokens apart
  const uint8_t* kb = k + (int64_t)(b / kdiv) * kstride * kIdxD;
  const float* ksb = ks + (int64_t)(b / kdiv) * kstride;
  float* hib = hi + (int64_t)b * L;
  float* lob = lo ? lo + (int64_t)b * L : hib;  // without lo: a zero-length range, the stores drop
  i32x8_t kr[D][U];
  float sr[D][U];
  // tokens of group g inside the row (wave-uniform)
  auto group_tokens = [&](int64_t g) { return (int)min((int64_t)GT, n - g * GT); };
  auto load = [&](int s, int64_t i) {
    const int64_t g = wid + (i < iters ? i : iters - 1) * nw;  // past the end: reload the last group
    const int nt = group_tokens(g);
    const __amdgpu_buffer_rsrc_t rk = buf_rsrc(kb + g * GT * kIdxD, nt * kIdxD);
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(ksb + g * GT, nt * 4);
    // the scales first: the wait for a group's codes then covers them too
#pragma unroll
    for (int u = 0; u < U; ++u) sr[s][u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, (16 * u + c) * 4, 0, 0));
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int off = (16 * u + c) * kIdxD + 16 * qq;
      const u32x4_t a0 = __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0);
      const u32x4_t a1 = __builtin_amdgcn_raw_buffer_load_b128(rk, off + 64, 0, 0);
      kr[s][u] = i32x8_t{(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
    }
  };
  // the ring's first groups go out before the q setup below, so their latency
  // overlaps it (the k stream does not depend on q)
  if (iters > 0) {
#pragma unroll
    for (int s = 0; s < D; ++s) load(s, s);
  }
  if (hist1)
    for (int i = threadIdx.x; i < kHistBins; i += 256) lh[i] = 0u;
#pragma unroll
  for (int i = 0; i < (kQv + 255) / 256; ++i)
    if (kQv % 256 == 0 || threadIdx.x + 256 * i < kQv) qsh[threadIdx.x + 256 * i] = qv[i];
  if (threadIdx.x < H) {
    qssh[threadIdx.x] = qsl;
    wsh[threadIdx.x] = wl;
  }
  __syncthreads();
  // A operands: head rows 16 j + c as bf16, in 4 chunks of 8 of this lane's 32
  // code bytes (the same byte order as the k operand, so every K pairs once),
  // negated where q_scale < 0; per-lane weights c = w |q_scale| of the D rows
  // (heads 16 j + 4 qq + r)
  bf16x8_t qa[HT][4];
  float cw[HT][4];
  i32x8_t raw[HT];
  float qsr[HT], wr[HT], cq[HT][4], cwr[HT][4];
#pragma unroll
  for (int j = 0; j < HT; ++j) {
    const u32x4_t a0 = qsh[(16 * j + c) * (kIdxD / 16) + qq], a1 = qsh[(16 * j + c) * (kIdxD / 16) + 4 + qq];
    raw[j] = i32x8_t{(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
    qsr[j] = qssh[16 * j + c];
    wr[j] = wsh[16 * j + c];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      cq[j][r] = qssh[16 * j + 4 * qq + r];
      cwr[j][r] = wsh[16 * j + 4 * qq + r];
    }
  }
  float bound = 0.f;
#pragma unroll
  for (int j = 0; j < HT; ++j) {
    const float l1 = sum_lane_quad(abs_sum_fp8(raw[j]));  // |q| sum of head row 16 j + c over the 4 lanes
    bound += qq == 0 ? fabsf(wr[j]) * fabsf(qsr[j]) * l1 : 0.f;
    fp8x32_to_bf16(raw[j], qa[j], qsr[j] < 0.f);
#pragma unroll
    for (int r = 0; r < 4; ++r) cw[j][r] = cwr[j][r] * fabsf(cq[j][r]);
  }
  const float qbound = wave_sum_f32(bound) * kBoundFactor;  // any fp32 summation order is within the slack
  auto compute = [&](int s, int64_t i) {
    const int64_t g = wid + i * nw;
    const int nt = group_tokens(g);
    const __amdgpu_buffer_rsrc_t rl = buf_rsrc(lob + g * GT, lo ? nt * 4 : 0);
    const __amdgpu_buffer_rsrc_t rh = buf_rsrc(hib + g * GT, nt * 4);
    f32x4_t d[U][HT];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      bf16x8_t kv[4];
      fp8x32_to_bf16(kr[s][u], kv, false);
#pragma unroll
      for (int j = 0; j < HT; ++j) {
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kc = 0; kc < 4; ++kc) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[j][kc], kv[kc], acc, 0, 0, 0);
        d[u][j] = acc;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      // with d' = d sign(q_scale): max(d q_scale k_scale, 0) w
      //   = |q_scale k_scale| w (|d'| + sign(k_scale) d') / 2
      // partial sums per head row r (independent chains), then across r and lanes
      float pa[4], pb[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pa[r] = cw[0][r] * fabsf(d[u][0][r]);
        pb[r] = cw[0][r] * d[u][0][r];
      }
#pragma unroll
      for (int j = 1; j < HT; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          pa[r] = fmaf(cw[j][r], fabsf(d[u][j][r]), pa[r]);
          pb[r] = fmaf(cw[j][r], d[u][j][r], pb[r]);
        }
      const float sa = sum_lane_quad((pa[0] + pa[1]) + (pa[2] + pa[3]));
      const float sb = sum_lane_quad((pb[0] + pb[1]) + (pb[2] + pb[3]));
      const float ksu = sr[s][u];
      const float part = 0.5f * fabsf(ksu) * (ksu < 0.f ? sa - sb : sa + sb);
      const float e = fabsf(sr[s][u]) * qbound;
      const float l = part - e, h = part + e;
      // lanes qq > 0 hold the same token: their stores fall outside the range
      const int off = qq == 0 ? (16 * u + c) * 4 : 0x40000000;
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(l), rl, off, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(h), rh, off, 0, 0);
      if (hist1 && qq == 0 && 16 * u + c < nt) atomicAdd(&lh[key_low_nan(l) >> kHistShift], 1u);
    }
  };
  if (iters > 0) {
    int64_t i0 = 0;
    for (; i0 + D < iters; i0 += D) {
#pragma unroll
      for (int s = 0; s < D; ++s) {
        compute(s, i0 + s);
        load(s, i0 + s + D);
      }
    }
#pragma unroll
    for (int s = 0; s < D; ++s)
      if (i0 + s < iters) compute(s, i0 + s);
  }
  if (hist1) {
    __syncthreads();
    // adjacent digits share one 64-bit add (each count < 2^32: no carry between them)
    unsigned long long* h2 = reinterpret_cast<unsigned long long*>(hist1 + (int64_t)b * kHistBins);
    for (int i = threadIdx.x; i < kHistBins / 2; i += 256) {
      const unsigned long long v = (unsigned long long)lh[2 * i] | ((unsigned long long)lh[2 * i + 1] << 32);
      if (v) atomicAdd(&h2[i], v);
    }
  }
}

typedef __attribute__((ext_vector_type(4))) int i32x4_v;

// 4 e4m3 codes -> three int8 limb words: 512 v = L2 2^14 + L1 2^7 + L0
__device__ __forceinline__ void e4m3_limbs_word(uint32_t x, int (&o)[3]) {
  const f32x2_t a = __builtin_amdgcn_cvt_pk_f32_fp8((int)x, false);
  const f32x2_t c = __builtin_amdgcn_cvt_pk_f32_fp8((int)x, true);
  const int v0 = (int)(a[0] * 512.f), v1 = (int)(a[1] * 512.f);
  const int v2 = (int)(c[0] * 512.f), v3 = (int)(c[1] * 512.f);
  o[0] = (v0 & 127) | ((v1 & 127) << 8) | ((v2 & 127) << 16) | ((v3 & 127) << 24);
  o[1] = ((v0 >> 7) & 127) | (((v1 >> 7) & 127) << 8) | (((v2 >> 7) & 127) << 16) | (((v3 >> 7) & 127) << 24);
  o[2] = ((v0 >> 14) & 255) | (((v1 >> 14) & 255) << 8) | (((v2 >> 14) & 255) << 16) | ((v3 >> 14) << 24);
}
// 16 e4m3 codes -> three int8 limb vectors
__device__ __forceinline__ void e4m3_limbs(const u32x4_t x, i32x4_v (&o)[3]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int t[3];
    e4m3_limbs_word(x[i], t);
    o[0][i] = t[0];
    o[1][i] = t[1];
    o[2][i] = t[2];
  }
}

// First kernel of a top-k call: clears the row histograms and writes q's int8
// limbs in the rescoring kernel's operand order, so that its workgroups load
// them (one coalesced 6 KB block per 16 heads) instead of converting q each:
// row r, heads 16 j + c, dims 64 ch + 16 qd + 4 i .. +3, limb la is word
// ((((r * HT + j) * 2 + ch) * 3 + la) * 64 + c + 16 qd) * 4 + i, HT = heads / 16.
__global__ void dsa_prep_kernel(uint32_t* __restrict__ hist, int64_t n_hist, const uint32_t* __restrict__ q,
                                uint32_t* __restrict__ qlimbs, int64_t n_qwords, int heads) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n_hist) hist[i] = 0u;
  if (i < n_qwords) {
    constexpr int W = kIdxD / 4;  // code words per head row
    const int64_t hrow = i / W;    // row * heads + head
    const int wd = (int)(i - hrow * W), head = (int)(hrow % heads);
    const int64_t r = hrow / heads;
    const int j = head >> 4, c = head & 15, ch = wd >> 4, qd = (wd >> 2) & 3, e = wd & 3;
    const int64_t base = (r * (heads >> 4) + j) * 2 + ch;
    int t[3];
    e4m3_limbs_word(q[i], t);
#pragma unroll
    for (int la = 0; la < 3; ++la) qlimbs[((base * 3 + la) * 64 + c + 16 * qd) * 4 + e] = (uint32_t)t[la];
  }
}

__device__ __forceinline__ i32x4_v mfma_i8(const i32x4_v a, const i32x4_v b, const i32x4_v c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// Stage 2: exact scores.  A workgroup owns `range` consecutive tokens of one
// row.  With `hi` set it keeps the tokens whose upper bound reaches tau, the
// lower edge of the histogram digit that holds the topk-th largest lower bound
// (at least topk tokens have lo >= tau, so a token with hi < tau is beaten by
// topk others), scores them 16 at a time on the MFMA (lanes = 16 candidates x
// 4 head groups) and appends 64-bit keys (score key << 32 | ~index) to the
// row's key list; without `hi` it scores every token into `scores`.  The
// histogram, the range's upper bounds and q are loaded together up front, and
// a range of at most kRsPfRange tokens loads its k rows and scales with them
// into LDS (PF), so the candidates' rows are there once tau is known.  The
// histogram is scanned from registers.
constexpr int kRsMaxRange = 4096;
constexpr int kRsPer = kRsMaxRange / 256;
constexpr int kRsMaxWgs = 4096;  // rescoring workgroups per row (rows up to 2^24 tokens)
constexpr int kRsPfRange = 256;  // ranges up to this many tokens stage their k rows in LDS up front
static_assert(kHistBins == 8 * 4 * 256, "the threshold scan gives each of 256 threads 8 vectors of 4 digits");
template <int HT, bool PF, bool QL>
__global__ void __launch_bounds__(256) dsa_rescore_kernel(
    const uint8_t* __restrict__ q, const float* __restrict__ qs, const uint8_t* __restrict__ k,
    const float* __restrict__ ks, const float* __restrict__ w, const int32_t* __restrict__ lengths,
    const float* __restrict__ hi, const uint32_t* __restrict__ hist1, const uint32_t* __restrict__ qlimbs,
    uint64_t* __restrict__ keys, uint32_t* __restrict__ wg_counts, float* __restrict__ scores, int64_t L, int topk,
    int range, int kdiv, int64_t kstride) {
  constexpr int H = HT * 16;
  constexpr int kCand = PF ? kRsPfRange : kRsMaxRange;
  constexpr int kPfVec = PF ? kRsPfRange * kIdxD / 16 : 1;  // 16-byte pieces of the staged k rows
  constexpr int kPfPer = PF ? kPfVec / 256 : 1;
  __shared__ uint32_t sh[1];
  __shared__ uint32_t hsum[8][4];
  __shared__ uint32_t wsum[4];
  __shared__ int cand[kCand];
  __shared__ float terms[4][16][H + 1];
  __shared__ u32x4_t kpf[kPfVec];
  __shared__ float kspf[PF ? kRsPfRange : 1];
  constexpr int kQlVec = HT * 2 * 3 * 64;  // 16-byte vectors of this row's q limbs
  constexpr int kQlPer = (kQlVec + 255) / 256;
  __shared__ i32x4_v qls[QL ? kQlVec : 1];
  const int b = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane((int)(tid >> 6));
  const int c = lane & 15, qd = lane >> 4;
  const int64_t n = row_length(lengths, b, L);
  const int64_t t_begin = (int64_t)blockIdx.x * range;
  if (t_begin >= n) return;
  const int nr = (int)min((int64_t)range, n - t_begin);  // tokens of this workgroup
  const bool select = hi != nullptr && n > topk;
  const uint8_t* kb = k + (int64_t)(b / kdiv) * kstride * kIdxD;
  const float* ksb = ks + (int64_t)(b / kdiv) * kstride;
  // in flight together: the row's histogram (thread tid holds digit vectors
  // v = tid + 256 i, digits 4 v .. 4 v + 3, coalesced), this range's upper
  // bounds, q, and the range's k rows and scales when they are staged
  u32x4_t hbuf[8];
  if (select) {
    const u32x4_t* src = reinterpret_cast<const u32x4_t*>(hist1 + (int64_t)b * kHistBins);
#pragma unroll
    for (int i = 0; i < 8; ++i) hbuf[i] = src[tid + 256 * i];
  }
  constexpr int kPer = PF ? kRsPfRange / 256 : kRsPer;  // tokens per thread
  float hv[kPer];
  if (hi) {
    const __amdgpu_buffer_rsrc_t rh = buf_rsrc(hi + (int64_t)b * L + t_begin, nr * 4);
#pragma unroll
    for (int i = 0; i < kPer; ++i)
      hv[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rh, (tid + 256 * i) * 4, 0, 0));
  }
  // A operands (rows = heads 16 j + c) as int8 limbs of dims 64 ch + 16 qd ..+16:
  // with QL the row's limbs (written by the prep kernel) are staged in LDS once
  // per workgroup and read after the compaction, otherwise converted here;
  // per-lane constants of the D layout (heads 16 j + 4 qd + r)
  i32x4_v ql[HT][2][3];
  i32x4_v qlb[kQlPer];
  if constexpr (QL) {
    const i32x4_v* src = reinterpret_cast<const i32x4_v*>(qlimbs) + (int64_t)b * kQlVec;
#pragma unroll
    for (int i = 0; i < kQlPer; ++i)
      if (kQlVec % 256 == 0 || tid + 256 * i < kQlVec) qlb[i] = src[tid + 256 * i];
  }
  float qsv[HT][4], wvv[HT][4];
#pragma unroll
  for (int j = 0; j < HT; ++j) {
    if constexpr (!QL) {
      const uint8_t* qrow = q + ((int64_t)b * H + 16 * j + c) * kIdxD + 16 * qd;
#pragma unroll
      for (int ch = 0; ch < 2; ++ch) e4m3_limbs(*reinterpret_cast<const u32x4_t*>(qrow + 64 * ch), ql[j][ch]);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      qsv[j][r] = qs[(int64_t)b * H + 16 * j + 4 * qd + r];
      wvv[j][r] = w[(int64_t)b * H + 16 * j + 4 * qd + r];
    }
  }
  // the staged k rows go out last: tau and the compaction wait only for the
  // loads issued before them
  u32x4_t kbuf[kPfPer];
  float ksv = 0.f;
  if constexpr (PF) {
    const __amdgpu_buffer_rsrc_t rk = buf_rsrc(kb + t_begin * kIdxD, nr * kIdxD);
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(ksb + t_begin, nr * 4);
#pragma unroll
    for (int i = 0; i < kPfPer; ++i) kbuf[i] = __builtin_amdgcn_raw_buffer_load_b128(rk, (tid + 256 * i) * 16, 0, 0);
    ksv = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, tid * 4, 0, 0));
  }
  // tau: the digit holding the topk-th largest lower bound.  Chunk i (digits
  // 1024 i .. 1024 i + 1023) is one vector per thread: a block scan per chunk
  // gives each vector the count of digits above it (the chunks above, plus the
  // higher vectors of its chunk), and the thread whose digits cross topk names it.
  uint32_t tau = 0u;
  if (select) {
    uint32_t vs[8], incl[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      vs[i] = (hbuf[i][0] + hbuf[i][1]) + (hbuf[i][2] + hbuf[i][3]);
      incl[i] = wave_incl_scan_u32(vs[i]);
    }
    if (lane == 63)
#pragma unroll
      for (int i = 0; i < 8; ++i) hsum[i][wv] = incl[i];
    __syncthreads();
    const uint32_t rem = (uint32_t)topk;
    uint32_t above = 0;  // digits in the chunks above chunk i
#pragma unroll
    for (int i = 7; i >= 0; --i) {
      uint32_t tot = 0, before = 0;
#pragma unroll
      for (int w2 = 0; w2 < 4; ++w2) {
        tot += hsum[i][w2];
        before += w2 < wv ? hsum[i][w2] : 0u;
      }
      uint32_t acc = above + (tot - (before + incl[i]));  // digits above this thread's top digit
#pragma unroll
      for (int r = 3; r >= 0; --r) {
        const uint32_t cnt = hbuf[i][r];
        if (acc < rem && rem <= acc + cnt) sh[0] = (uint32_t)(4 * (tid + 256 * i) + r);
        acc += cnt;
      }
      above += tot;
    }
    __syncthreads();
    tau = sh[0] << kHistShift;
  }
  if constexpr (QL) {  // visible after the compaction's barriers
#pragma unroll
    for (int i = 0; i < kQlPer; ++i)
      if (kQlVec % 256 == 0 || tid + 256 * i < kQlVec) qls[tid + 256 * i] = qlb[i];
  }
  if constexpr (PF) {
#pragma unroll
    for (int i = 0; i < kPfPer; ++i) kpf[tid + 256 * i] = kbuf[i];
    kspf[tid] = ksv;
  }
  // compaction: thread tid's tokens are tid + 256 i; a block scan of the
  // per-thread counts places them
  uint32_t keep = 0u, nk = 0u;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const bool ok = tid + 256 * i < nr && (!hi || key_high_nan(hv[i]) >= tau);
    keep |= ok ? 1u << i : 0u;
    nk += ok ? 1u : 0u;
  }
  const uint32_t incl = wave_incl_scan_u32(nk);
  if (lane == 63) wsum[wv] = incl;
  __syncthreads();
  uint32_t pos = incl - nk;
#pragma unroll
  for (int i = 0; i < 4; ++i) pos += i < wv ? wsum[i] : 0u;
  const int C = (int)(wsum[0] + wsum[1] + wsum[2] + wsum[3]);
#pragma unroll
  for (int i = 0; i < kPer; ++i)
    if (keep & (1u << i)) cand[pos++] = (int)(t_begin + tid + 256 * i);
  __syncthreads();
  // the keys go to this workgroup's own token range, keys[b][t_begin + i] for
  // candidate i, and the count to wg_counts[b][blockIdx.x] (no atomics)
  if (hi && tid == 0) wg_counts[(int64_t)b * kRsMaxWgs + blockIdx.x] = (uint32_t)C;
  const int nb = __builtin_amdgcn_readfirstlane((C + 15) / 16);  // batches of 16 candidates (block-uniform)
  if (nb == 0) return;
  if constexpr (QL) {
#pragma unroll
    for (int j = 0; j < HT; ++j)
#pragma unroll
      for (int ch = 0; ch < 2; ++ch)
#pragma unroll
        for (int la = 0; la < 3; ++la) ql[j][ch][la] = qls[((j * 2 + ch) * 3 + la) * 64 + lane];
  }
  struct Batch {
    u32x4_t x[2];
    float ks;
    int t;
  };
  auto load_batch = [&](int bt, Batch& o) {
    const int i = bt * 16 + c;
    const bool ok = i < C;
    o.t = ok ? cand[i] : -1;
    const int64_t tt = ok ? o.t : cand[0];
    if constexpr (PF) {
      const int r = (int)(tt - t_begin);
      o.ks = kspf[r];
#pragma unroll
      for (int ch = 0; ch < 2; ++ch) o.x[ch] = kpf[r * (kIdxD / 16) + 4 * ch + qd];
    } else {
      o.ks = ksb[tt];
#pragma unroll
      for (int ch = 0; ch < 2; ++ch)
        o.x[ch] = *reinterpret_cast<const u32x4_t*>(kb + tt * kIdxD + 64 * ch + 16 * qd);
    }
  };
  // head tile j of a batch (18 MFMAs): the terms of heads 16 j .. 16 j + 15 into tm[candidate][head]
  auto head_tile = [&](int j, const i32x4_v (&kl)[2][3], float kscale, float (*tm)[H + 1]) {
    i32x4_v g[5];
#pragma unroll
    for (int mm = 0; mm < 5; ++mm) g[mm] = i32x4_v{0, 0, 0, 0};
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
      const float a = (d * qsv[j][r]) * kscale;
      const float rr = a > 0.f ? a : 0.f;
      tm[c][16 * j + 4 * qd + r] = rr * wvv[j][r];
    }
  };
  // candidate i (token t): its terms summed in head order, then its key (or score)
  auto emit = [&](int i, int t, const float* row) {
    float tv[H];
#pragma unroll
    for (int h = 0; h < H; ++h) tv[h] = row[h];
    float sc = 0.f;
#pragma unroll
    for (int h = 0; h < H; ++h) sc = sc + tv[h];
    if (hi)
      keys[(int64_t)b * L + t_begin + i] = ((uint64_t)key_low_nan(sc) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)t);
    else
      scores[(int64_t)b * L + t] = sc;
  };
  if (HT == 4 && nb <= 4) {
    // At most 64 candidates: the four waves share the batches' head tiles,
    // each wave one batch (4 / nbw waves per batch, nbw tiles each), and the
    // terms meet in LDS.
    const int nbw = nb == 3 ? 4 : nb;
    const int bt = wv * nbw / 4, j0 = (wv % (4 / nbw)) * nbw;
    Batch in;
    load_batch(bt, in);  // a batch past the candidates reads candidate 0's row and writes unused terms
    i32x4_v kl[2][3];
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) e4m3_limbs(in.x[ch], kl[ch]);
#pragma unroll
    for (int j = 0; j < HT; ++j)
      if (j >= j0 && j < j0 + nbw) head_tile(j, kl, in.ks, terms[bt]);
    __syncthreads();
    if (tid < C) emit(tid, cand[tid], terms[tid >> 4][tid & 15]);
    return;
  }
  // More candidates: wave wv scores batches bt = wv, wv + 4, ... whole.
  const int my_batches = nb > wv ? (nb - 1 - wv) / 4 + 1 : 0;
  if (my_batches == 0) return;
  auto score_batch = [&](int m, const Batch& in) {
    i32x4_v kl[2][3];
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) e4m3_limbs(in.x[ch], kl[ch]);
#pragma unroll
    for (int j = 0; j < HT; ++j) head_tile(j, kl, in.ks, terms[wv]);
    wave_lds_fence();  // the terms are in LDS
    if (qd == 0 && in.t >= 0) emit(16 * (wv + 4 * m) + c, in.t, terms[wv][c]);
    __builtin_amdgcn_wave_barrier();
  };
  // ping-pong over this wave's batches (bt = wv + 4 m).  The loads are
  // unconditional (a batch past the candidates reads candidate 0's row and
  // scores nothing): a branch around them would make the compiler wait for
  // them at its join, before the current batch is scored.
  Batch ba, bb;
  load_batch(wv, ba);
  for (int m = 0; m < my_batches; m += 2) {
    const bool more = m + 1 < my_batches;
    load_batch(wv + 4 * (m + 1), bb);
    score_batch(m, ba);
    if (!more) break;
    load_batch(wv + 4 * (m + 2), ba);
    score_batch(m + 1, bb);
  }
}

// 64-bit min / max over the 64 lanes (all lanes active) on DPP moves of both
// halves (the wave_max_u32 steps; lanes without a source get the identity),
// broadcast from lane 63
#define MOSAIC_DPP64(ident, v, ctrl, rmask)                                                       \
  (((uint64_t)MOSAIC_DPP((uint32_t)((ident) >> 32), (uint32_t)((v) >> 32), ctrl, rmask) << 32) | \
   (uint64_t)MOSAIC_DPP((uint32_t)(ident), (uint32_t)(v), ctrl, rmask))
__device__ __forceinline__ uint64_t wave_bcast63_u64(uint64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 63);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 63);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
  constexpr uint64_t I = ~0ull;
  uint64_t o;
  o = MOSAIC_DPP64(I, v, 0xB1, 0xF);
  v = o < v ? o : v;
  o = MOSAIC_DPP64(I, v, 0x4E, 0xF);
  v = o < v ? o : v;
  o = MOSAIC_DPP64(I, v, 0x141, 0xF);
  v = o < v ? o : v;
  o = MOSAIC_DPP64(I, v, 0x140, 0xF);
  v = o < v ? o : v;
  o = MOSAIC_DPP64(I, v, 0x142, 0xA);
  v = o < v ? o : v;
  o = MOSAIC_DPP64(I, v, 0x143, 0xC);
  v = o < v ? o : v;
  return wave_bcast63_u64(v);
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  constexpr uint64_t I = 0ull;
  uint64_t o;
  o = MOSAIC_DPP64(I, v, 0xB1, 0xF);
  v = o > v ? o : v;
  o = MOSAIC_DPP64(I, v, 0x4E, 0xF);
  v = o > v ? o : v;
  o = MOSAIC_DPP64(I, v, 0x141, 0xF);
  v = o > v ? o : v;
  o = MOSAIC_DPP64(I, v, 0x140, 0xF);
  v = o > v ? o : v;
  o = MOSAIC_DPP64(I, v, 0x142, 0xA);
  v = o > v ? o : v;
  o = MOSAIC_DPP64(I, v, 0x143, 0xC);
  v = o > v ? o : v;
  return wave_bcast63_u64(v);
}

// Stage 3: the kk best of the row's candidate keys (unique: exact score key <<
// 32 | ~index), in descending order, to idx_out.  One workgroup of 1024
// threads per row.  Rescoring workgroup w left wg_counts[b][w] keys at
// keys[b][w * range ..].
//  - At most kSortCap candidates: every key goes to registers (4 per thread),
//    placed through the prefix of the per-workgroup counts (the first key
//    slots of every workgroup are read together with the counts).  Otherwise a radix
//    select over the keys in global memory finds the kk-th largest key and
//    only the kk keys at or above it are kept.
//  - Keys are bucketed by (key - smallest key) >> shift into kBuckets buckets,
//    the buckets are laid out largest first by a scan of their counts, and a
//    key's rank is its bucket's start plus the number of larger keys in it.
constexpr int kBuckets = 4096;
static_assert(kBuckets == kRsMaxWgs, "the bucket edges hold the workgroup prefix first");
__global__ void __launch_bounds__(1024) dsa_finish_kernel(const uint64_t* __restrict__ keys,
                                                          const uint32_t* __restrict__ wg_counts,
                                                          const int32_t* __restrict__ lengths, int64_t L, int range,
                                                          int topk, int offset, int32_t* __restrict__ idx_out) {
  __shared__ uint64_t bk[kSortCap];
  __shared__ uint32_t edge[kBuckets + 1];  // workgroup prefix
  __shared__ uint32_t bcnt[kBuckets];      // bucket counts, then bucket edges
  __shared__ uint32_t lh[256];
  __shared__ uint32_t sh[4];
  __shared__ uint64_t red[2][16];
  __shared__ uint32_t wtot[16];
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  for (int i = tid; i < kBuckets; i += 1024) bcnt[i] = 0u;  // visible after the prefix's barriers
  const int64_t n = row_length(lengths, b, L);
  const int nwg = (int)((n + range - 1) / range);
  const uint64_t* kb = keys + (int64_t)b * L;
  // In flight with the counts: the first 4 S key slots of every rescoring
  // workgroup (S = 1024 / nwg threads each), read before their counts are
  // known and kept where the count covers them.
  const int S = nwg <= 1024 ? 1024 / nwg : 0;
  const bool spec = S > 0 && tid < S * nwg;
  const int sw = spec ? tid / S : 0, ss = spec ? tid - sw * S : 0;
  uint32_t sc = 0u;
  uint64_t sk[4];
  if (spec) {
    sc = wg_counts[(int64_t)b * kRsMaxWgs + sw];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t slot = (int64_t)sw * range + ss + S * r;
      sk[r] = slot < L ? kb[slot] : 0ull;
    }
  }
  // edge[w] = first slot of rescoring workgroup w (exclusive prefix)
  {
    uint32_t cw[4], local = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int w = 4 * tid + r;
      cw[r] = w < nwg ? wg_counts[(int64_t)b * kRsMaxWgs + w] : 0u;
      local += cw[r];
    }
    const uint32_t incl = wave_incl_scan_u32(local);
    if (lane == 63) wtot[wv] = incl;
    __syncthreads();
    uint32_t acc = incl - local;
    for (int i = 0; i < wv; ++i) acc += wtot[i];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      edge[4 * tid + r] = acc;
      acc += cw[r];
    }
    __syncthreads();
  }
  uint32_t total = 0;
  for (int i = 0; i < 16; ++i) total += wtot[i];
  const int64_t cnt = min((int64_t)total, n);
  const int kk = (int)min((int64_t)topk, cnt);
  int32_t* dst = idx_out + (int64_t)b * topk;
  for (int i = kk + tid; i < topk; i += 1024) dst[i] = -1;
  if (kk == 0) return;
  // slot i -> its key: the last workgroup w with edge[w] <= i owns it
  auto key_at = [&](int i) -> uint64_t {
    int lo = 0, hi = nwg - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (edge[mid] <= (uint32_t)i) lo = mid; else hi = mid - 1;
    }
    return kb[(int64_t)lo * range + (i - (int)edge[lo])];
  };
  int m;
  uint64_t x[4];
  if (cnt <= kSortCap && S > 0) {
    // the keys into LDS at their workgroup's edge (the slots past 4 S one at a time), then 4 per thread
    m = (int)cnt;
    if (spec) {
      const uint32_t e0 = edge[sw];
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if ((uint32_t)(ss + S * r) < sc) bk[e0 + ss + S * r] = sk[r];
      for (uint32_t j = (uint32_t)(ss + 4 * S); j < sc; j += (uint32_t)S) bk[e0 + j] = kb[(int64_t)sw * range + j];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 4; ++r) x[r] = tid + 1024 * r < m ? bk[tid + 1024 * r] : 0ull;
  } else if (cnt <= kSortCap) {
    m = (int)cnt;
#pragma unroll
    for (int r = 0; r < 4; ++r) x[r] = tid + 1024 * r < m ? key_at(tid + 1024 * r) : 0ull;
  } else {
    // radix select of the kk-th largest key, 8 bits at a time
    uint64_t prefix = 0, pmask = 0;
    uint32_t rem = (uint32_t)kk;
    for (int shift = 56; shift >= 0; shift -= 8) {
      if (tid < 256) lh[tid] = 0u;
      __syncthreads();
      for (int i = tid; i < (int)cnt; i += 1024) {
        const uint64_t key = key_at(i);
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
    for (int i = tid; i < (int)cnt; i += 1024) {
      const uint64_t key = key_at(i);
      if (key >= prefix) bk[atomicAdd(&sh[2], 1u)] = key;
    }
    __syncthreads();
    m = kk;
#pragma unroll
    for (int r = 0; r < 4; ++r) x[r] = tid + 1024 * r < m ? bk[tid + 1024 * r] : 0ull;
  }
  // smallest and largest key
  uint64_t mn = ~0ull, mx = 0ull;
#pragma unroll
  for (int r = 0; r < 4; ++r)
    if (tid + 1024 * r < m) {
      mn = x[r] < mn ? x[r] : mn;
      mx = x[r] > mx ? x[r] : mx;
    }
  mn = wave_min_u64(mn);
  mx = wave_max_u64(mx);
  if (lane == 0) {
    red[0][wv] = mn;
    red[1][wv] = mx;
  }
  __syncthreads();
  mn = red[0][0];
  mx = red[1][0];
#pragma unroll
  for (int i = 1; i < 16; ++i) {
    mn = red[0][i] < mn ? red[0][i] : mn;
    mx = red[1][i] > mx ? red[1][i] : mx;
  }
  const uint64_t span = mx - mn;
  const int bits = span == 0 ? 0 : 64 - __clzll((long long)span);
  const int shift = bits > 12 ? bits - 12 : 0;
  uint32_t bx[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    bx[r] = (uint32_t)((x[r] - mn) >> shift);
    if (tid + 1024 * r < m) atomicAdd(&bcnt[bx[r]], 1u);
  }
  __syncthreads();
  // descending exclusive scan: bcnt[d] = number of keys in buckets above d
  // (thread tid owns buckets kBuckets-1-4 tid .. kBuckets-4-4 tid)
  uint32_t cb[4], local = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    cb[i] = bcnt[kBuckets - 1 - (4 * tid + i)];
    local += cb[i];
  }
  const uint32_t incl = wave_incl_scan_u32(local);
  if (lane == 63) wtot[wv] = incl;
  __syncthreads();
  uint32_t acc = incl - local;
  for (int i = 0; i < wv; ++i) acc += wtot[i];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bcnt[kBuckets - 1 - (4 * tid + i)] = acc;
    acc += cb[i];
  }
  __syncthreads();
  // scatter into bucket order; afterwards bcnt[d] = the end of bucket d
#pragma unroll
  for (int r = 0; r < 4; ++r)
    if (tid + 1024 * r < m) bk[atomicAdd(&bcnt[bx[r]], 1u)] = x[r];
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    if (tid + 1024 * r >= m) continue;
    const uint32_t s = bx[r] + 1 < kBuckets ? bcnt[bx[r] + 1] : 0u, e = bcnt[bx[r]];
    uint32_t rank = s;
    for (uint32_t j = s; j < e; ++j) rank += bk[j] > x[r] ? 1u : 0u;
    if (rank < (uint32_t)kk) dst[rank] = (int32_t)(0xFFFFFFFFu - (uint32_t)x[r]) + offset;
  }
}

// ===================================================================== MLA
constexpr int kMlaBT = 32;        // tokens per online-softmax block
constexpr int kMlaDl = 512;       // latent (value) width
constexpr int kMlaDt = kMlaDl / 16;  // 16-wide latent column tiles
constexpr int kPsStride = 40;     // bf16 per row of the P exchange (32 tokens + 8)
constexpr int kMlaMaxSplits = 64;
// A head's running maximum moves only when a block's maximum exceeds it by
// more than this (natural log units): probabilities stay below e^8, which
// bf16 P and the fp32 sums hold with their usual relative precision, and the
// O rescale is skipped for almost every block after the first.
constexpr float kMlaLazyMax = 8.f;

constexpr int kMlaMaxChunk = 1024;  // token ids of one split (staged in LDS)
// FP8 gather stages: raw latent rows, scale rows (up to 32 floats), rope rows
constexpr int kMlaStages = 3;
constexpr int kMlaStgLat = kMlaBT * kMlaDl;
constexpr int kMlaStgSc = kMlaBT * 32 * 4;
constexpr int kMlaStgRope = kMlaBT * 64 * 2;
constexpr int kMlaStage = kMlaStgLat + kMlaStgSc + kMlaStgRope;
constexpr int kMlaCopies = 9;  // copies per wave per block: 4 latent, 4 scale, 1 rope

typedef short mla_v4s __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t mla_lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// one 16-byte (resp. 4-byte) global -> LDS copy per lane; the LDS address of
// lane i is base + 16 i (resp. 4 i).  Issued from inline asm so the compiler
// neither waits for them before LDS reads nor stages them in registers; the
// kernel waits with explicit vmcnt counts.
__device__ __forceinline__ void mla_copy16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(__builtin_amdgcn_readfirstlane(lds)),
               "v"(g) : "memory", "m0");
}
__device__ __forceinline__ void mla_copy4(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off" ::"s"(__builtin_amdgcn_readfirstlane(lds)),
               "v"(g) : "memory", "m0");
}

__device__ __forceinline__ f32x4_t mfma_bf16(const bf16x8_t a, const bf16x8_t b, const f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Token order inside a block: MFMA K index / P slot p = 8 g + 4 r + i holds
// block token 8 g + 2 i + r.  With it the four 4-token LDS transpose reads of
// two 16-lane groups touch 8 rows whose bank offsets (36 dwords apart) are
// 8 dwords apart, and a QK A-operand read still takes 16 rows distinct mod 16.
__device__ __forceinline__ int mla_slot_token(int p) { return (p & ~7) | ((p & 3) << 1) | ((p >> 2) & 1); }

// 4 bf16 of V column c' (of a 16-column tile) for 4 tokens, from row-major
// K rows in LDS: with lane 4 i + j of a 16-lane group pointing at row token_i,
// columns 4 j .. 4 j + 3, lane c' receives row token_i, column c' as element i.
__device__ __forceinline__ mla_v4s lds_read_tr16(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) mla_v4s*)(p));
}

// max / sum over the 16 lanes of each row (pair, quad, half-row and row
// mirrors); every lane of the row gets the result
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(v), 0xB1, 0xF)));
  v = fmaxf(v, __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(v), 0x4E, 0xF)));
  v = fmaxf(v, __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(v), 0x141, 0xF)));
  return fmaxf(v, __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(v), 0x140, 0xF)));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(v), 0xB1, 0xF));
  v += __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(v), 0x4E, 0xF));
  v += __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(v), 0x141, 0xF));
  return v + __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(v), 0x140, 0xF));
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
// one group of 16*HT heads (HT head tiles): partial (m, l, O) per head.  The
// split's token ids are staged in LDS first (masked or out-of-range ids as -1).
// Blocks of kMlaBT tokens then go through two LDS buffers of bf16 K rows
// (latent then rope).  FP8 caches: raw rows, their scales and rope rows are
// copied global -> LDS directly (global_load_lds) into a ring of kMlaStages
// stages, issued three blocks ahead of their conversion to bf16, so the gather
// latency hides behind three blocks of math; every wave issues kMlaCopies
// copies per block, so `s_waitcnt vmcnt` + a barrier hands a stage over.  BF16
// caches: each thread gathers its item of block i + 1 into registers while
// block i is multiplied out, and stores it after.
//
// Four waves.  Wave w < HT scores and soft-maxes head tile w (S = Q K^T:
// its heads' q kept in registers as the A operand, K rows from LDS as B), then
// the workgroup swaps roles for O += P V: P (bf16) and the per-head rescale
// factors go through LDS, and each wave multiplies every head of the group
// into its own quarter of the 512 latent columns, reading V straight out of
// the K rows with LDS transpose reads.  So V is read once per workgroup rather
// than once per 16 heads, and no transposed copy of it is written.  A
// workgroup runs one wave per SIMD, which leaves room for the O tiles (16 HT
// heads x 128 columns per wave) in accumulation registers.
template <int HT, bool FP8, int DR>
__global__ void __launch_bounds__(256) mla_decode_split_kernel(
    const uint16_t* __restrict__ q, const MlaKv kv, const int32_t* __restrict__ idx, uint16_t* __restrict__ part_o,
    float* __restrict__ part_ml, int topk, float scale, int chunk) {
  constexpr int DQK = kMlaDl + DR;
  constexpr int KS = DQK + 8;  // bf16 per K row in LDS: 16-byte reads of 16 rows hit distinct banks
  constexpr int NW = 4, NT = NW * 64;
  constexpr int RAWV = FP8 ? 4 : 8;               // 16-byte vectors per (token, 64-wide segment) item
  constexpr int DTW = kMlaDt / NW;                // latent column tiles per wave in O += P V
  static_assert(kMlaBT * 8 == NT && (DR == 0 || kMlaBT * (DR / 8) == NT), "one item and one rope chunk a thread");
  static_assert(!FP8 || DR == 64, "FP8 caches carry a 64-wide bf16 rope");
  __shared__ __attribute__((aligned(16))) uint16_t Kt[2][kMlaBT * KS];
  __shared__ __attribute__((aligned(16))) uint8_t Stg[FP8 ? kMlaStages * kMlaStage : 16];
  __shared__ __attribute__((aligned(16))) uint16_t Ps[16 * HT * kPsStride];
  __shared__ __attribute__((aligned(16))) float As[16 * HT];
  __shared__ int Fl[HT];
  __shared__ int Ids[kMlaMaxChunk];
  const int H = HT * 16 * gridDim.z;
  const int split = blockIdx.x, b = blockIdx.y, S = gridDim.x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool scorer = wv < HT;             // this wave scores head tile wv
  const int hw = (int)blockIdx.z * HT + (scorer ? wv : 0);  // its 16-head group in the row
  const int c = lane & 15, qd = lane >> 4;
  const int head = 16 * hw + c;
  const int dt0 = wv * DTW;  // this wave's first latent column tile
  const int64_t n = kv.n;
  const int64_t kvb = b / kv.rows_per_kv;
  const int t_begin = split * chunk;
  const int t_end = min(topk, t_begin + chunk);
  // (an empty cache masks every token: nothing is read)
  const int nblk = t_end > t_begin && n > 0 ? (t_end - t_begin + kMlaBT - 1) / kMlaBT : 0;
  const int nsc = kMlaDl >> kv.sb_shift;  // scales per FP8 row
  // the split's ids (loaded first, so that they fly together with q)
  constexpr int IDS_PT = kMlaMaxChunk / NT;
  int idv[IDS_PT];
#pragma unroll
  for (int k = 0; k < IDS_PT; ++k) {
    const int s = tid + NT * k, ti = t_begin + s;
    idv[k] = s < nblk * kMlaBT && ti < t_end ? idx[(int64_t)b * topk + ti] : -1;
  }
  // q as the A operand of S = Q K^T: lane (c, qd) holds q[head][32 s + 8 qd .. +8]
  // (kept in registers: the empty asm stops the compiler from re-loading q in
  // every block, where those loads would queue behind the gather)
  bf16x8_t qb[DQK / 32];
  {
    const uint16_t* qrow = q + ((int64_t)b * H + head) * DQK;
#pragma unroll
    for (int s = 0; s < DQK / 32; ++s) qb[s] = *reinterpret_cast<const bf16x8_t*>(qrow + 32 * s + 8 * qd);
#pragma unroll
    for (int s = 0; s < DQK / 32; ++s) asm volatile("" : "+v"(qb[s]));
  }
#pragma unroll
  for (int k = 0; k < IDS_PT; ++k) {
    const int s = tid + NT * k;
    if (s < nblk * kMlaBT) Ids[s] = idv[k] >= 0 && (int64_t)idv[k] < n ? idv[k] : -1;
  }
  __syncthreads();
  // row of the cache that token t of block j reads (masked tokens read row 0
  // of their batch and are zeroed when converted)
  auto row_of = [&](int j, int t) -> int64_t {
    const int id = Ids[j * kMlaBT + t];
    return kvb * n + (id >= 0 ? id : 0);
  };
  // ---- FP8: global -> LDS copies of block j into stage j % kMlaStages.  Latent
  // rows keep their 16-byte chunks XOR-swizzled by (token & 15) and scale rows
  // their floats by (token & 31), so the conversion's reads of 16 tokens hit
  // distinct banks.
  auto issue_fp8 = [&](int j) {
    uint8_t* st = &Stg[(j % kMlaStages) * kMlaStage];
#pragma unroll
    for (int k = 0; k < 4; ++k) {  // latent: tokens 8 wv + 2 k (lanes 0-31) and + 1 (lanes 32-63)
      const int t = 8 * wv + 2 * k + (lane >> 5), p = lane & 31;
      const uint8_t* src = reinterpret_cast<const uint8_t*>(kv.lat) + row_of(j, t) * kMlaDl + 16 * (p ^ (t & 15));
      mla_copy16(src, mla_lds_addr(st + (8 * wv + 2 * k) * kMlaDl));
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {  // scales: floats 64 (wv + 4 k) + lane = (token f / 32, slot f % 32)
      const int f = 64 * (wv + 4 * k) + lane, t = f >> 5, p = f & 31;
      const int e = min(p ^ (t & 31), nsc - 1);
      mla_copy4(kv.lat_s + row_of(j, t) * nsc + e, mla_lds_addr(st + kMlaStgLat + 256 * (wv + 4 * k)));
    }
    {  // rope: tokens 8 wv .. 8 wv + 7
      const int t = 8 * wv + (lane >> 3), pc = lane & 7;
      mla_copy16(kv.rope + row_of(j, t) * DR + 8 * pc, mla_lds_addr(st + kMlaStgLat + kMlaStgSc + 1024 * wv));
    }
  };
  // wait until at most `after` blocks' copies of this wave are in flight, then barrier
  auto wait_stage = [&](int after) {
    if (after >= 2)
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(2 * kMlaCopies) : "memory");
    else if (after == 1)
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(kMlaCopies) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  };
  // item of thread tid: token tid % 32, latent segment tid / 32 (64 values);
  // rope chunk: token tid / 8, 8 values at 8 (tid % 8)
  const int tk = tid % kMlaBT, seg = tid / kMlaBT;
  const int rtk = tid / 8, rpc = tid % 8;
  // stage of block j -> bf16 K rows of buffer j & 1
  auto convert_fp8 = [&](int j) {
    const uint8_t* st = &Stg[(j % kMlaStages) * kMlaStage];
    const bool ok = Ids[j * kMlaBT + tk] >= 0;
    const float* srow = reinterpret_cast<const float*>(st + kMlaStgLat) + tk * 32;
    uint32_t outw[32];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const u32x4_t w = *reinterpret_cast<const u32x4_t*>(st + tk * kMlaDl + 16 * ((4 * seg + v) ^ (tk & 15)));
      const float sc = srow[((seg * 64 + 16 * v) >> kv.sb_shift) ^ (tk & 31)];
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        // exact e4m3 -> fp32, fp32 product with the scale, one RNE rounding to bf16
        f32x2_t a2 = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[e2], false);
        f32x2_t b2 = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[e2], true);
        a2[0] *= sc;
        a2[1] *= sc;
        b2[0] *= sc;
        b2[1] *= sc;
        outw[8 * v + 2 * e2] = __builtin_bit_cast(uint32_t, __builtin_convertvector(a2, bf16x2_t));
        outw[8 * v + 2 * e2 + 1] = __builtin_bit_cast(uint32_t, __builtin_convertvector(b2, bf16x2_t));
      }
    }
    u32x4_t* kdst = reinterpret_cast<u32x4_t*>(&Kt[j & 1][tk * KS + seg * 64]);
#pragma unroll
    for (int v = 0; v < 8; ++v)
      kdst[v] = ok ? u32x4_t{outw[4 * v], outw[4 * v + 1], outw[4 * v + 2], outw[4 * v + 3]} : u32x4_t{0u, 0u, 0u, 0u};
    const u32x4_t r = *reinterpret_cast<const u32x4_t*>(st + kMlaStgLat + kMlaStgSc + rtk * 128 + 16 * rpc);
    *reinterpret_cast<u32x4_t*>(&Kt[j & 1][rtk * KS + kMlaDl + 8 * rpc]) =
        Ids[j * kMlaBT + rtk] >= 0 ? r : u32x4_t{0u, 0u, 0u, 0u};
  };
  // ---- BF16: register-staged gather of block j, stored by fill_bf16
  u32x4_t raw[RAWV];
  u32x4_t rrope;
  auto issue_bf16 = [&](int j) {
    const uint16_t* src = reinterpret_cast<const uint16_t*>(kv.lat) + row_of(j, tk) * DQK + seg * 64;
#pragma unroll
    for (int v = 0; v < RAWV; ++v) raw[v] = *reinterpret_cast<const u32x4_t*>(src + 8 * v);
    if constexpr (DR > 0)
      rrope = *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const uint16_t*>(kv.lat) + row_of(j, rtk) * DQK +
                                                 kMlaDl + 8 * rpc);
  };
  auto fill_bf16 = [&](int j) {
    const bool ok = Ids[j * kMlaBT + tk] >= 0;
    u32x4_t* kdst = reinterpret_cast<u32x4_t*>(&Kt[j & 1][tk * KS + seg * 64]);
#pragma unroll
    for (int v = 0; v < 8; ++v) kdst[v] = ok ? raw[v] : u32x4_t{0u, 0u, 0u, 0u};
    if constexpr (DR > 0)
      *reinterpret_cast<u32x4_t*>(&Kt[j & 1][rtk * KS + kMlaDl + 8 * rpc]) =
          Ids[j * kMlaBT + rtk] >= 0 ? rrope : u32x4_t{0u, 0u, 0u, 0u};
  };
  // O tiles: rows = heads 16 ht + 4 qd + r of the group, columns 16 (dt0 + dl) + c
  f32x4_t o[HT][DTW];
#pragma unroll
  for (int ht = 0; ht < HT; ++ht)
#pragma unroll
    for (int dl = 0; dl < DTW; ++dl) o[ht][dl] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // running maximum and sum of heads 16 hw + 4 qd + r (all 16 lanes of a row agree)
  float m_run[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY}, l_run[4] = {0.f, 0.f, 0.f, 0.f};
  if (nblk > 0) {
    if constexpr (FP8) {
      issue_fp8(0);
      if (nblk > 1) issue_fp8(1);
      wait_stage(nblk > 1 ? 1 : 0);
      convert_fp8(0);
      if (nblk > 2) issue_fp8(2);
    } else {
      issue_bf16(0);
      fill_bf16(0);
    }
  }
  // V transpose reads: lane 4 vi + vj of group qd points at block token
  // 8 qd + 2 vi (+ 1 for the second read), columns 4 vj .. 4 vj + 3 of a tile
  const int vi = c >> 2, vj = c & 3;
  for (int blk = 0; blk < nblk; ++blk) {
    const int bf = blk & 1;
    const int* bid = &Ids[blk * kMlaBT];
    __syncthreads();  // buffer bf is filled; buffer bf ^ 1, its stage, P and the rescale flags are no longer read
    const bool more = blk + 1 < nblk;
    if constexpr (FP8) {
      if (blk + 3 < nblk) issue_fp8(blk + 3);  // into the stage block blk came from
    } else {
      if (more) issue_bf16(blk + 1);  // block blk + 1 flies while block blk is multiplied out
    }
    if (scorer) {  // QK and the online softmax of head tile wv
      // S tiles (rows = heads 4 qd + r of the tile, column = slot 16 j + c): A = q
      // (registers), B = K rows; two accumulators per tile (even and odd K steps)
      // halve the dependent MFMA chain.  The ids of this lane's two tokens are
      // read first so that their LDS latency hides behind the products.
      bool live[kMlaBT / 16];
#pragma unroll
      for (int j = 0; j < kMlaBT / 16; ++j) live[j] = bid[mla_slot_token(16 * j + c)] >= 0;
      f32x4_t st[kMlaBT / 16], st2[kMlaBT / 16];
#pragma unroll
      for (int j = 0; j < kMlaBT / 16; ++j) st[j] = st2[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      // K fragments in batches of KB steps, double-buffered: batch i + 1's LDS
      // reads are issued before batch i's products (the scheduling barriers keep
      // the compiler from interleaving them into a read-wait-multiply chain)
      constexpr int KB = 3, NSQ = DQK / 32, NKB = (NSQ + KB - 1) / KB;
      bf16x8_t kop[2][KB][kMlaBT / 16];
      int krow[kMlaBT / 16];
#pragma unroll
      for (int j = 0; j < kMlaBT / 16; ++j) krow[j] = mla_slot_token(16 * j + c) * KS + 8 * qd;
      auto read_k = [&](int kb2, bf16x8_t (&dst)[KB][kMlaBT / 16]) {
#pragma unroll
        for (int ss = 0; ss < KB; ++ss)
#pragma unroll
          for (int j = 0; j < kMlaBT / 16; ++j)
            if (kb2 * KB + ss < NSQ)
              dst[ss][j] = *reinterpret_cast<const bf16x8_t*>(&Kt[bf][krow[j] + 32 * (kb2 * KB + ss)]);
      };
      read_k(0, kop[0]);
#pragma unroll
      for (int kb2 = 0; kb2 < NKB; ++kb2) {
        if (kb2 + 1 < NKB) read_k(kb2 + 1, kop[(kb2 + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ss = 0; ss < KB; ++ss)
#pragma unroll
          for (int j = 0; j < kMlaBT / 16; ++j) {
            const int s = kb2 * KB + ss;
            if (s >= NSQ) continue;
            if (s & 1)
              st2[j] = mfma_bf16(qb[s], kop[kb2 & 1][ss][j], st2[j]);
            else
              st[j] = mfma_bf16(qb[s], kop[kb2 & 1][ss][j], st[j]);
          }
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int j = 0; j < kMlaBT / 16; ++j) st[j] += st2[j];
      // online softmax of heads 4 qd + r: reductions over the 16 lanes of a row
      float sc[kMlaBT / 16][4], p[kMlaBT / 16][4], alpha[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float bm = -INFINITY;
#pragma unroll
        for (int j = 0; j < kMlaBT / 16; ++j) {
          sc[j][r] = live[j] ? st[j][r] * scale : -INFINITY;
          bm = fmaxf(bm, sc[j][r]);
        }
        bm = row16_max(bm);
        // the running maximum moves only past the lazy margin (or from -inf)
        const bool move = bm > m_run[r] + kMlaLazyMax;
        const float m_new = move ? bm : m_run[r];
        alpha[r] = (move && m_run[r] != -INFINITY) ? __expf(m_run[r] - m_new) : 1.f;
        float psum = 0.f;
#pragma unroll
        for (int j = 0; j < kMlaBT / 16; ++j) {
          p[j][r] = m_new == -INFINITY ? 0.f : __expf(sc[j][r] - m_new);
          psum += p[j][r];
        }
        l_run[r] = l_run[r] * alpha[r] + row16_sum(psum);
        m_run[r] = m_new;
      }
      // P (bf16, rows = the tile's heads, columns = slots) and the heads' O
      // rescale factors into LDS; a flag per wave says whether any is not 1
#pragma unroll
      for (int j = 0; j < kMlaBT / 16; ++j)
#pragma unroll
        for (int r = 0; r < 4; r += 2) {
          const uint32_t pw =
              __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{p[j][r], p[j][r + 1]}, bf16x2_t));
          Ps[(16 * wv + 4 * qd + r) * kPsStride + 16 * j + c] = (uint16_t)(pw & 0xFFFFu);
          Ps[(16 * wv + 4 * qd + r + 1) * kPsStride + 16 * j + c] = (uint16_t)(pw >> 16);
        }
      if (c == 0) *reinterpret_cast<f32x4_t*>(&As[16 * wv + 4 * qd]) = f32x4_t{alpha[0], alpha[1], alpha[2], alpha[3]};
      const bool rescale = __ballot(alpha[0] != 1.f || alpha[1] != 1.f || alpha[2] != 1.f || alpha[3] != 1.f) != 0;
      if (lane == 0) Fl[wv] = rescale ? 1 : 0;
    }
    __syncthreads();  // P, the factors and the flags of every wave are in
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) {
      if (__builtin_amdgcn_readfirstlane(Fl[ht])) {  // the same word for every lane
        const f32x4_t al = *reinterpret_cast<const f32x4_t*>(&As[16 * ht + 4 * qd]);
#pragma unroll
        for (int dl = 0; dl < DTW; ++dl) o[ht][dl] *= al;
      }
    }
    // O += P V over this wave's column tiles: A = P rows of every head tile
    // (k = slots 8 qd .. 8 qd + 7), B = V by two transpose reads per tile
    bf16x8_t pa[HT];
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) pa[ht] = *reinterpret_cast<const bf16x8_t*>(&Ps[(16 * ht + c) * kPsStride + 8 * qd]);
    const uint16_t* vbase = &Kt[bf][(8 * qd + 2 * vi) * KS + 4 * vj];
    constexpr int VB = 4, NVB = DTW / VB;
    bf16x8_t vv[2][VB];
    auto read_v = [&](int vb2, bf16x8_t (&dst)[VB]) {
#pragma unroll
      for (int dd = 0; dd < VB; ++dd) {
        const uint16_t* vp = vbase + 16 * (dt0 + vb2 * VB + dd);
        const mla_v4s a = lds_read_tr16(vp), e = lds_read_tr16(vp + KS);
        dst[dd] = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(a, e, 0, 1, 2, 3, 4, 5, 6, 7));
      }
    };
    read_v(0, vv[0]);
#pragma unroll
    for (int vb2 = 0; vb2 < NVB; ++vb2) {
      if (vb2 + 1 < NVB) read_v(vb2 + 1, vv[(vb2 + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int dd = 0; dd < VB; ++dd)
#pragma unroll
        for (int ht = 0; ht < HT; ++ht)
          o[ht][vb2 * VB + dd] = mfma_bf16(pa[ht], vv[vb2 & 1][dd], o[ht][vb2 * VB + dd]);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (more) {
      if constexpr (FP8) {
        wait_stage(min(2, nblk - blk - 2));  // block blk + 1's copies (of every wave) have landed
        convert_fp8(blk + 1);
      } else {
        fill_bf16(blk + 1);
      }
    }
  }
  // partial O (bf16, un-normalized) in MFMA tile order:
  // part_o[b][split][head tile][column tile][lane][4] (rows = heads 16 tile + 4 qd + r,
  // column 16 tile + c); bf16 halves the partials' store and the combine's read
  uint16_t* po = part_o + ((int64_t)b * S + split) * (H / 16) * (kMlaDt * 256);
#pragma unroll
  for (int ht = 0; ht < HT; ++ht)
#pragma unroll
    for (int dl = 0; dl < DTW; ++dl) {
      const f32x4_t v = o[ht][dl];
      *reinterpret_cast<uint2*>(po + (((int64_t)(blockIdx.z * HT + ht) * kMlaDt + dt0 + dl) * 64 + lane) * 4) =
          uint2{(uint32_t)f32_bf16(v[0]) | ((uint32_t)f32_bf16(v[1]) << 16),
                (uint32_t)f32_bf16(v[2]) | ((uint32_t)f32_bf16(v[3]) << 16)};
    }
  if (scorer && c == 0) {
    float* pml = part_ml + (((int64_t)b * S + split) * H + 16 * hw + 4 * qd) * 2;
    *reinterpret_cast<f32x4_t*>(pml) = f32x4_t{m_run[0], l_run[0], m_run[1], l_run[1]};
    *reinterpret_cast<f32x4_t*>(pml + 4) = f32x4_t{m_run[2], l_run[2], m_run[3], l_run[3]};
  }
}

// Merge the splits of one (row, 16-head tile, 16-column tile) with the sink
// term and normalize.  Each wave turns the split maxima/sums of four heads
// into weights (lane = split); then wave w blends splits w, w + 4, ... of the
// tile's 64 x 4 partial values, and wave 0 sums the four and writes bf16.
__global__ void __launch_bounds__(256) mla_combine_kernel(const uint16_t* __restrict__ part_o,
                                                          const float* __restrict__ part_ml,
                                                          const float* __restrict__ sink, uint16_t* __restrict__ out,
                                                          int H, int S) {
  __shared__ float wgt[kMlaMaxSplits][16];
  __shared__ f32x4_t red[4][64];
  const int dt = blockIdx.x, ht = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int hh = 4 * wv + k, h = 16 * ht + hh;
    const bool ok = lane < S;
    const float m = ok ? part_ml[(((int64_t)b * S + lane) * H + h) * 2] : -INFINITY;
    const float l = ok ? part_ml[(((int64_t)b * S + lane) * H + h) * 2 + 1] : 0.f;
    // DPP max (exact in any order); a NaN lane is left out, as fmaxf would
    const float M = wave_max_f32(m == m ? m : -INFINITY);
    const float e = (m == -INFINITY) ? 0.f : __expf(m - M);
    const float lsum = wave_sum_f32(l * e) + ((sink && M != -INFINITY) ? __expf(sink[h] - M) : 0.f);
    if (ok) wgt[lane][hh] = (M == -INFINITY) ? 0.f : e / lsum;
  }
  __syncthreads();
  const int hq = lane >> 4;  // rows 4 hq + r of the tile
  const int64_t sstride = (int64_t)(H / 16) * kMlaDt * 256;
  const uint16_t* po = part_o + (int64_t)b * S * sstride + ((int64_t)ht * kMlaDt + dt) * 256 + lane * 4;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int s = wv; s < S; s += 4) {
    const uint2 raw = *reinterpret_cast<const uint2*>(po + s * sstride);
    const float v[4] = {__uint_as_float(raw.x << 16), __uint_as_float(raw.x & 0xFFFF0000u),
                        __uint_as_float(raw.y << 16), __uint_as_float(raw.y & 0xFFFF0000u)};
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] += wgt[s][4 * hq + r] * v[r];
  }
  red[wv][lane] = acc;
  __syncthreads();
  if (wv == 0) {
    const f32x4_t v = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
#pragma unroll
    for (int r = 0; r < 4; ++r)
      out[((int64_t)b * H + 16 * ht + 4 * hq + r) * kMlaDl + 16 * dt + (lane & 15)] = f32_bf16(v[r]);
  }
}

// The same merge for grids of many rows: a workgroup takes four 16-column
// tiles, and wave w blends every split of column tile 4 x + w (x = blockIdx.x)
// in split order and writes bf16 (no cross-wave sum).  A wave's first 32
// splits are loaded before the weights are formed.  Four times fewer
// workgroups, each reading its splits' tiles once: used from 4 rows of 128
// heads up (B = 8: 35.7 -> 33.7 us a call; at B = 1 the 64 workgroups were
// slower, 19.5 against 17.5 us).
constexpr int kMlaCombineTiles = 4;  // 16-column tiles a workgroup

__global__ void __launch_bounds__(256) mla_combine_tiles_kernel(const uint16_t* __restrict__ part_o,
                                                          const float* __restrict__ part_ml,
                                                          const float* __restrict__ sink, uint16_t* __restrict__ out,
                                                          int H, int S) {
  __shared__ float wgt[kMlaMaxSplits][16];
  const int ht = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int dt = blockIdx.x * kMlaCombineTiles + wv;
  const int hq = lane >> 4;  // rows 4 hq + r of the tile
  const int64_t sstride = (int64_t)(H / 16) * kMlaDt * 256;
  const uint16_t* po = part_o + (int64_t)b * S * sstride + ((int64_t)ht * kMlaDt + dt) * 256 + lane * 4;
  constexpr int CH = 32;
  uint2 raw[CH];
  auto load_chunk = [&](int s0) {
#pragma unroll
    for (int i = 0; i < CH; ++i)
      raw[i] = s0 + i < S ? *reinterpret_cast<const uint2*>(po + (s0 + i) * sstride) : make_uint2(0u, 0u);
  };
  load_chunk(0);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int hh = 4 * wv + k, h = 16 * ht + hh;
    const bool ok = lane < S;
    const float m = ok ? part_ml[(((int64_t)b * S + lane) * H + h) * 2] : -INFINITY;
    const float l = ok ? part_ml[(((int64_t)b * S + lane) * H + h) * 2 + 1] : 0.f;
    // DPP max (exact in any order); a NaN lane is left out, as fmaxf would
    const float M = wave_max_f32(m == m ? m : -INFINITY);
    const float e = (m == -INFINITY) ? 0.f : __expf(m - M);
    const float lsum = wave_sum_f32(l * e) + ((sink && M != -INFINITY) ? __expf(sink[h] - M) : 0.f);
    if (ok) wgt[lane][hh] = (M == -INFINITY) ? 0.f : e / lsum;
  }
  __syncthreads();
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < S; s0 += CH) {
    if (s0) load_chunk(s0);
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      if (s0 + i < S) {
        const float v[4] = {__uint_as_float(raw[i].x << 16), __uint_as_float(raw[i].x & 0xFFFF0000u),
                            __uint_as_float(raw[i].y << 16), __uint_as_float(raw[i].y & 0xFFFF0000u)};
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] += wgt[s0 + i][4 * hq + r] * v[r];
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r)
    out[((int64_t)b * H + 16 * ht + 4 * hq + r) * kMlaDl + 16 * dt + (lane & 15)] = f32_bf16(acc[r]);
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct IndexerWs {
  float* hi;
  uint64_t* keys;
  uint32_t *wg_counts, *hist1;
  size_t zero_words;  // hist1
  uint32_t* qlimbs;   // q's int8 limbs, written by the prep kernel
};

static size_t indexer_ws(int64_t b, int64_t l, char* base, IndexerWs* w) {
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? base + off : nullptr;
    off += align256(bytes);
    return p;
  };
  float* hi = (float*)take((size_t)b * l * 4);
  uint64_t* keys = (uint64_t*)take((size_t)b * l * 8);
  uint32_t* wgc = (uint32_t*)take((size_t)b * kRsMaxWgs * 4);
  const size_t zbytes = (size_t)b * kHistBins * 4;
  uint32_t* z = (uint32_t*)take(zbytes);
  uint32_t* qlimbs = (uint32_t*)take((size_t)b * 64 * 3 * kIdxD);  // q's int8 limbs, up to 64 heads
  if (w) {
    w->hi = hi;
    w->keys = keys;
    w->wg_counts = wgc;
    w->hist1 = z;
    w->zero_words = zbytes / 4;
    w->qlimbs = qlimbs;
  }
  return off;
}

// Bound kernel shape: one 16-token tile per group, a ring of up to 4 groups
// (its registers then leave three waves per SIMD: about 3072 resident waves on
// 256 CUs) spread over the rows, and at least one full ring per wave where the
// rows are short (each workgroup merges its whole histogram once).
constexpr int kBoundU = 1;
static void bound_shape(int64_t b, int64_t l, int& gx, int& depth) {
  const int64_t groups = (l + 16 * kBoundU - 1) / (16 * kBoundU);
  int64_t g = (768 + b - 1) / b;
  g = std::min<int64_t>(g, (groups + 15) / 16);
  gx = (int)std::max<int64_t>(g, 1);
  const int64_t iters = (groups + 4 * gx - 1) / (4 * gx);
  depth = iters >= 4 ? 4 : (iters >= 2 ? 2 : 1);
}

template <int HT, int D>
static void launch_bound_d(const uint8_t* q, const float* qs, const uint8_t* k, const float* ks, const float* w,
                           const int32_t* lengths, float* lo, float* hi, uint32_t* hist1, int64_t b, int64_t l,
                           int gx, int kdiv, int64_t kstride, hipStream_t st) {
  MOSAIC_LAUNCH((dsa_index_bound_kernel<HT, kBoundU, D>), dim3((unsigned)gx, (unsigned)b), dim3(256), 0, st, q,
                     qs, k, ks, w, lengths, lo, hi, hist1, l, kdiv, kstride);
}

template <int HT>
static void launch_bound(const uint8_t* q, const float* qs, const uint8_t* k, const float* ks, const float* w,
                         const int32_t* lengths, float* lo, float* hi, uint32_t* hist1, int64_t b, int64_t l,
                         int kdiv, int64_t kstride, hipStream_t st) {
  int gx, depth;
  bound_shape(b, l, gx, depth);
  if (depth == 4)
    launch_bound_d<HT, 4>(q, qs, k, ks, w, lengths, lo, hi, hist1, b, l, gx, kdiv, kstride, st);
  else if (depth == 2)
    launch_bound_d<HT, 2>(q, qs, k, ks, w, lengths, lo, hi, hist1, b, l, gx, kdiv, kstride, st);
  else
    launch_bound_d<HT, 1>(q, qs, k, ks, w, lengths, lo, hi, hist1, b, l, gx, kdiv, kstride, st);
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
                           int64_t l, int kdiv, int64_t kstride, hipStream_t st) {
  switch (h / 16) {
    case 1: launch_bound<1>(q, qs, k, ks, w, lengths, lo, hi, hist1, b, l, kdiv, kstride, st); break;
    case 2: launch_bound<2>(q, qs, k, ks, w, lengths, lo, hi, hist1, b, l, kdiv, kstride, st); break;
    case 3: launch_bound<3>(q, qs, k, ks, w, lengths, lo, hi, hist1, b, l, kdiv, kstride, st); break;
    default: launch_bound<4>(q, qs, k, ks, w, lengths, lo, hi, hist1, b, l, kdiv, kstride, st); break;
  }
}

// tokens per rescoring workgroup: about one workgroup per CU over the batch
// (its registers leave one wave per SIMD), a multiple of 64, at most the LDS
// candidate list, and few enough workgroups per row for the finish kernel
static int rescore_range(int64_t b, int64_t l) {
  const int64_t target = std::max<int64_t>(1, 256 / std::max<int64_t>(b, 1));
  int64_t r = (l + target - 1) / target;
  r = std::max<int64_t>(r, (l + kRsMaxWgs - 1) / kRsMaxWgs);
  r = (r + 63) / 64 * 64;
  return (int)std::min<int64_t>(std::max<int64_t>(r, 64), kRsMaxRange);
}

static void launch_rescore(const uint8_t* q, const float* qs, const uint8_t* k, const float* ks, const float* w,
                           const int32_t* lengths, const float* hi, const uint32_t* hist1, const uint32_t* qlimbs,
                           uint64_t* keys, uint32_t* wg_counts, float* scores, int64_t b, int64_t h, int64_t l,
                           int topk, int kdiv, int64_t kstride, hipStream_t st) {
  const int range = rescore_range(b, l);
  const dim3 grid((unsigned)((l + range - 1) / range), (unsigned)b);
#define MOSAIC_RESCORE(HT)                                                                                          \
  if (!qlimbs)                                                                                                      \
    MOSAIC_LAUNCH((dsa_rescore_kernel<HT, false, false>), grid, dim3(256), 0, st, q, qs, k, ks, w, lengths,   \
                       hi, hist1, qlimbs, keys, wg_counts, scores, l, topk, range, kdiv, kstride);                           \
  else if (range <= kRsPfRange)                                                                                     \
    MOSAIC_LAUNCH((dsa_rescore_kernel<HT, true, true>), grid, dim3(256), 0, st, q, qs, k, ks, w, lengths, hi, \
                       hist1, qlimbs, keys, wg_counts, scores, l, topk, range, kdiv, kstride);                             \
  else                                                                                                              \
    MOSAIC_LAUNCH((dsa_rescore_kernel<HT, false, true>), grid, dim3(256), 0, st, q, qs, k, ks, w, lengths,    \
                       hi, hist1, qlimbs, keys, wg_counts, scores, l, topk, range, kdiv, kstride);
  switch (h / 16) {
    case 1: MOSAIC_RESCORE(1) break;
    case 2: MOSAIC_RESCORE(2) break;
    case 3: MOSAIC_RESCORE(3) break;
    default: MOSAIC_RESCORE(4) break;
  }
#undef MOSAIC_RESCORE
}

struct MlaWs {
  uint16_t* part_o;
  float* part_ml;
};

// splits per row: about 256 workgroups over the batch (two head groups per
// row), at most one per block and at most 32
static int mla_splits(int64_t b, int64_t topk) {
  const int64_t blocks = (topk + kMlaBT - 1) / kMlaBT;
  int64_t s = (128 + b - 1) / b;
  s = std::min<int64_t>(s, blocks);
  s = std::min<int64_t>(s, 32);
  // a split's ids must fit the LDS id buffer
  s = std::max<int64_t>(s, (blocks + kMlaMaxChunk / kMlaBT - 1) / (kMlaMaxChunk / kMlaBT));
  static_assert(32 <= kMlaMaxSplits, "the combine kernel weighs at most kMlaMaxSplits splits");
  return (int)std::max<int64_t>(s, 1);
}
// head tiles per workgroup: as many as divide the heads (at most 4), fewer
// while the grid has fewer workgroups than CUs (B = 1, 128 heads: 32 splits x
// 8 groups of 16 heads, 18.3 against 19.6 us for 4 groups of 32 heads)
static int mla_head_tiles(int64_t b, int64_t h, int S) {
  int ht = 4;
  while (ht > 1 && (h / 16) % ht != 0) --ht;
  while (ht > 1 && (h / 16) % (ht / 2) == 0 && (int64_t)S * b * (h / (16 * ht)) < 256) ht /= 2;
  return ht;
}
static size_t mla_ws(int64_t b, int64_t h, int64_t topk, char* base, MlaWs* w) {
  const int64_t S = mla_splits(b, topk);
  const size_t ob = align256((size_t)b * S * h * kMlaDl * 2);
  const size_t mb = align256((size_t)b * S * h * 2 * 4);
  if (w) {
    w->part_o = (uint16_t*)base;
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

namespace mosaic {
static int indexer_topk_impl(const uint8_t* q, const float* q_s, const uint8_t* k, const float* k_s, const float* w,
                             const int32_t* lengths, int32_t* idx_out, int64_t b, int64_t h, int64_t d, int64_t l,
                             int64_t topk, int32_t offset, int64_t kdiv, int64_t kstride, void* workspace,
                             size_t workspace_bytes, void* stream) {
  int rc = check_indexer(q, q_s, k, k_s, w, b, h, d, l);
  if (rc) return rc;
  MOSAIC_CHECK_ARG(idx_out, "dsa_indexer_topk: null output");
  MOSAIC_CHECK_ARG(topk >= 1 && topk <= kMaxTopk, "dsa_indexer_topk: topk %lld (1..%d)", (long long)topk, kMaxTopk);
  MOSAIC_CHECK_ARG(l <= (int64_t)kRsMaxWgs * kRsMaxRange, "dsa_indexer_topk: l %lld (at most %lld)", (long long)l,
                   (long long)kRsMaxWgs * kRsMaxRange);
  MOSAIC_CHECK_ARG(kdiv >= 1 && b % kdiv == 0, "dsa_indexer_topk: %lld query rows do not split into groups of %lld",
                   (long long)b, (long long)kdiv);
  MOSAIC_CHECK_ARG(kstride >= l && kstride < (1ll << 40), "dsa_indexer_topk: cache length %lld < l %lld",
                   (long long)kstride, (long long)l);
  const size_t need = indexer_ws(b, l, nullptr, nullptr);
  MOSAIC_CHECK_ARG(workspace && workspace_bytes >= need, "dsa_indexer_topk: workspace %zu bytes < %zu",
                   workspace_bytes, need);
  if (b == 0) return kOk;
  hipStream_t st = (hipStream_t)stream;
  IndexerWs ws;
  indexer_ws(b, l, (char*)workspace, &ws);
  const int64_t qwords = b * h * (kIdxD / 4);
  const int64_t prep_n = std::max<int64_t>((int64_t)ws.zero_words, qwords);
  MOSAIC_LAUNCH(dsa_prep_kernel, dim3((unsigned)((prep_n + 255) / 256)), dim3(256), 0, st, ws.hist1,
                     (int64_t)ws.zero_words, reinterpret_cast<const uint32_t*>(q), ws.qlimbs, qwords, (int)h);
  if (l > 0) {
    dispatch_bound(q, q_s, k, k_s, w, lengths, nullptr, ws.hi, ws.hist1, b, h, l, (int)kdiv, kstride, st);
    launch_rescore(q, q_s, k, k_s, w, lengths, ws.hi, ws.hist1, ws.qlimbs, ws.keys, ws.wg_counts, nullptr, b, h, l,
                   (int)topk, (int)kdiv, kstride, st);
  }
  MOSAIC_LAUNCH(dsa_finish_kernel, dim3((unsigned)b), dim3(1024), 0, st, ws.keys, ws.wg_counts, lengths, l,
                     rescore_range(b, l), (int)topk, (int)offset, idx_out);
  MOSAIC_RETURN_LAUNCH("dsa_indexer_topk");
}
}  // namespace mosaic

extern "C" int mosaic_dsa_indexer_topk(const uint8_t* q, const float* q_s, const uint8_t* k, const float* k_s,
                                       const float* w, const int32_t* lengths, int32_t* idx_out, int64_t b, int64_t h,
                                       int64_t d, int64_t l, int64_t topk, int32_t offset, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  return indexer_topk_impl(q, q_s, k, k_s, w, lengths, idx_out, b, h, d, l, topk, offset, 1, l, workspace,
                           workspace_bytes, stream);
}

extern "C" int mosaic_dsa_indexer_topk_shared(const uint8_t* q, const float* q_s, const uint8_t* k, const float* k_s,
                                              const float* w, const int32_t* lengths, int32_t* idx_out, int64_t rows,
                                              int64_t h, int64_t d, int64_t l, int64_t cache_len, int64_t rows_per_k,
                                              int64_t topk, int32_t offset, void* workspace, size_t workspace_bytes,
                                              void* stream) {
  return indexer_topk_impl(q, q_s, k, k_s, w, lengths, idx_out, rows, h, d, l, topk, offset, rows_per_k, cache_len,
                           workspace, workspace_bytes, stream);
}

extern "C" int mosaic_dsa_indexer_scores(const uint8_t* q, const float* q_s, const uint8_t* k, const float* k_s,
                                         const float* w, float* scores, int64_t b, int64_t h, int64_t d, int64_t l,
                                         void* stream) {
  int rc = check_indexer(q, q_s, k, k_s, w, b, h, d, l);
  if (rc) return rc;
  MOSAIC_CHECK_ARG(scores, "dsa_indexer_scores: null output");
  if (b == 0 || l == 0) return kOk;
  launch_rescore(q, q_s, k, k_s, w, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, scores, b, h, l, 0, 1, l,
                 (hipStream_t)stream);
  MOSAIC_RETURN_LAUNCH("dsa_indexer_scores");
}

extern "C" int mosaic_dsa_indexer_bounds(const uint8_t* q, const float* q_s, const uint8_t* k, const float* k_s,
                                         const float* w, float* lo, float* hi, int64_t b, int64_t h, int64_t d,
                                         int64_t l, void* stream) {
  int rc = check_indexer(q, q_s, k, k_s, w, b, h, d, l);
  if (rc) return rc;
  MOSAIC_CHECK_ARG(lo && hi, "dsa_indexer_bounds: null output");
  if (b == 0 || l == 0) return kOk;
  dispatch_bound(q, q_s, k, k_s, w, nullptr, lo, hi, nullptr, b, h, l, 1, l, (hipStream_t)stream);
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
  const int ht = mla_head_tiles(rows, h, S);
  dim3 grid((unsigned)S, (unsigned)rows, (unsigned)(h / (16 * ht)));
  switch (ht) {
#define MLA_CASE(HTV)                                                                                                  \
  case HTV:                                                                                                            \
    MOSAIC_LAUNCH((mla_decode_split_kernel<HTV, FP8, DR>), grid, dim3(256), 0, st, q, kv, idx, ws.part_o,       \
                       ws.part_ml, (int)topk, softmax_scale, chunk);                                                   \
    break;
    MLA_CASE(1) MLA_CASE(2) MLA_CASE(3) MLA_CASE(4)
#undef MLA_CASE
  }
  MOSAIC_LAUNCH_CHECK("mla_decode_split");
  if (rows * (h / 16) * (kMlaDt / kMlaCombineTiles) >= 256)
    MOSAIC_LAUNCH(mla_combine_tiles_kernel,
                  dim3((unsigned)(kMlaDt / kMlaCombineTiles), (unsigned)(h / 16), (unsigned)rows), dim3(256), 0, st,
                  ws.part_o, ws.part_ml, sink, out, (int)h, S);
  else
    MOSAIC_LAUNCH(mla_combine_kernel, dim3((unsigned)kMlaDt, (unsigned)(h / 16), (unsigned)rows), dim3(256), 0, st,
                  ws.part_o, ws.part_ml, sink, out, (int)h, S);
  MOSAIC_RETURN_LAUNCH("mla_sparse_decode");
}

static int check_mla_common(int64_t rows, int64_t h, int64_t n, int64_t topk, int64_t rows_per_kv, void* workspace,
                            size_t workspace_bytes) {
  MOSAIC_CHECK_ARG(h >= 16 && h <= 256 && h % 16 == 0 && (h <= 64 || h % 64 == 0),
                   "mla_sparse_decode: heads %lld (16, 32, 48, 64 or a multiple of 64 up to 256)", (long long)h);
  MOSAIC_CHECK_ARG(rows >= 0 && rows <= 65535 && n >= 0 && n < (1ll << 31) && topk >= 0 &&
                       topk <= (int64_t)kMlaMaxSplits * kMlaMaxChunk,
                   "mla_sparse_decode: shape out of range (topk at most %d)", kMlaMaxSplits * kMlaMaxChunk);
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
