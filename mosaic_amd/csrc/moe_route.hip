// Router top-k (A10), stable expert sort (A11) and uncapped tile list (A12).
//
// One 1024-thread workgroup does all three for up to kRouteMaxAssign
// assignments: routing writes ids/weights, then every assignment gets its
// stable position inside its expert segment (ascending flat index), then the
// tile list (expert, m_start, rows) is emitted in ascending expert order.
// Everything stays on the device; nothing is read back by the host.
#include "common.h"
#include "moe_internal.h"
#include "../../include/mosaic_amd.h"

namespace mosaic {

constexpr int kRouteThreads = 1024;
constexpr int kRouteWaves = kRouteThreads / 64;
constexpr int kRouteMaxAssign = 8192;   // A_ext limit of the single-workgroup path
constexpr int kRouteMaxExperts = 512;   // routed experts (+1 virtual shared expert)
constexpr int kRouteMaxTopK = 16;

// fp32 -> unsigned key with the same order (NaN -> smallest)
__device__ __forceinline__ uint32_t order_key(float f) {
  if (f != f) return 0u;
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float score_of(float logit, int func) {
  if (func == MOSAIC_SCORE_SIGMOID) return 1.0f / (1.0f + expf(-logit));
  if (func == MOSAIC_SCORE_SQRTSOFTPLUS) {
    float sp = logit > 20.f ? logit : log1pf(expf(logit));
    return sqrtf(sp);
  }
  return logit;  // softmax handled by the caller
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  uint32_t lo = __shfl_xor((uint32_t)v, m, 64);
  uint32_t hi = __shfl_xor((uint32_t)(v >> 32), m, 64);
  return ((uint64_t)hi << 32) | lo;
}

// One wave routes one token.  Selection key: the logit when there is no bias
// (every score function is monotone), else score + bias.  Ties -> lower index.
__device__ void route_one_token(const float* __restrict__ lg, int E, int K, int func, int renorm, float scale,
                                const float* __restrict__ bias, int32_t* ids_out, float* w_out) {
  const int lane = threadIdx.x & 63;
  constexpr int kPer = kRouteMaxExperts / 64;
  float lv[kPer];
  uint64_t key[kPer];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    int e = lane + 64 * j;
    lv[j] = (e < E) ? lg[e] : -INFINITY;
    if (e < E) mx = fmaxf(mx, lv[j]);
  }
  float denom = 1.f;
  if (func == MOSAIC_SCORE_SOFTMAX) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      int e = lane + 64 * j;
      if (e < E) s += expf(lv[j] - mx);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    denom = s;
  }
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    int e = lane + 64 * j;
    if (e < E) {
      float k = lv[j];
      if (bias) {
        float sc = (func == MOSAIC_SCORE_SOFTMAX) ? expf(lv[j] - mx) / denom : score_of(lv[j], func);
        k = sc + bias[e];
      }
      key[j] = ((uint64_t)order_key(k) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)e);
    } else {
      key[j] = 0;  // never selected while a real expert remains
    }
  }
  float wsel[kRouteMaxTopK];
  int isel[kRouteMaxTopK];
  for (int r = 0; r < K; ++r) {
    uint64_t best = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) best = key[j] > best ? key[j] : best;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      uint64_t o = shfl_xor_u64(best, off);
      best = o > best ? o : best;
    }
    int e = (int)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFull));
#pragma unroll
    for (int j = 0; j < kPer; ++j)
      if (lane + 64 * j == e) key[j] = 0;
    float l = lg[e];
    float sc = (func == MOSAIC_SCORE_SOFTMAX) ? expf(l - mx) / denom : score_of(l, func);
    isel[r] = e;
    wsel[r] = sc;
  }
  if (lane == 0) {
    float sum = 0.f;
    for (int r = 0; r < K; ++r) sum += wsel[r];
    for (int r = 0; r < K; ++r) {
      float w = wsel[r];
      if (renorm && func != MOSAIC_SCORE_SOFTMAX) w = w / sum;
      w_out[r] = w * scale;
      ids_out[r] = isel[r];
    }
  }
}


// Flat assignment a < M*K is (token a/K, slot a%K); a >= M*K is the shared
// expert's row for token a - M*K (virtual expert id E, weight 1).
__global__ void __launch_bounds__(kRouteThreads) route_layout_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias, int32_t* ids, float* weights, int M, int E,
    int K, int func, int renorm, float route_scale, int has_shared, int block_m, int tile_cap, LayoutOut out) {
  __shared__ int16_t s_ids[kRouteMaxAssign];
  __shared__ int32_t s_cnt[kRouteMaxExperts + 2];
  __shared__ int32_t s_off[kRouteMaxExperts + 2];
  __shared__ int32_t s_run[kRouteMaxExperts + 2];
  __shared__ int32_t s_tab[kRouteWaves][kRouteMaxExperts + 2];
  __shared__ int32_t s_toff[kRouteMaxExperts + 2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int A = M * K;
  const int A_ext = A + (has_shared ? M : 0);
  const int E_ext = E + (has_shared ? 1 : 0);

  // 1. routing (one wave per token) or read the given ids
  if (logits) {
    for (int t = wave; t < M; t += kRouteWaves)
      route_one_token(logits + (int64_t)t * E, E, K, func, renorm, route_scale, bias, ids + (int64_t)t * K,
                      weights + (int64_t)t * K);
    __threadfence();
  }
  __syncthreads();
  for (int a = tid; a < A_ext; a += kRouteThreads) {
    int e;
    if (a < A) {
      e = ids[a];  // written above by another wave of this workgroup
      e = (e < 0 || e >= E) ? -1 : e;
    } else {
      e = E;
    }
    s_ids[a] = (int16_t)e;
  }
  for (int e = tid; e < E_ext; e += kRouteThreads) { s_cnt[e] = 0; s_run[e] = 0; }
  __syncthreads();
  // 2. counts (integer atomics: order-independent)
  for (int a = tid; a < A_ext; a += kRouteThreads) {
    int e = s_ids[a];
    if (e >= 0) atomicAdd(&s_cnt[e], 1);
  }
  __syncthreads();
  // 3. exclusive scans of counts and of tile counts (wave 0, 64 lanes in chunks)
  if (wave == 0) {
    int carry = 0, tcarry = 0;
    for (int base = 0; base < E_ext; base += 64) {
      int e = base + lane;
      int c = (e < E_ext) ? s_cnt[e] : 0;
      int tc = (c + block_m - 1) / block_m;
      int inc = c, tinc = tc;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        int o = __shfl_up(inc, off, 64), to = __shfl_up(tinc, off, 64);
        if (lane >= off) { inc += o; tinc += to; }
      }
      if (e < E_ext) { s_off[e] = carry + inc - c; s_toff[e] = tcarry + tinc - tc; }
      carry += __shfl(inc, 63, 64);
      tcarry += __shfl(tinc, 63, 64);
    }
    if (lane == 0) { s_off[E_ext] = carry; s_toff[E_ext] = tcarry; }
  }
  __syncthreads();
  // 4. stable positions: chunks of 1024 assignments in order; inside a wave the
  //    rank comes from an exact-match ballot mask, across waves from s_tab.
  int nbits = 1;
  while ((1 << nbits) <= E_ext) ++nbits;
  for (int base = 0; base < A_ext; base += kRouteThreads) {
    for (int i = tid; i < kRouteWaves * E_ext; i += kRouteThreads) s_tab[i / E_ext][i % E_ext] = 0;
    __syncthreads();
    const int a = base + tid;
    const bool live = a < A_ext && s_ids[a] >= 0;
    if (a < A_ext && !live) out.inv_pos[a] = -1;
    const int e = live ? s_ids[a] : 0;
    uint64_t mask = __ballot(live);
    for (int b = 0; b < nbits; ++b) {
      uint64_t bb = __ballot(live && ((e >> b) & 1));
      mask &= ((e >> b) & 1) ? bb : ~bb;
    }
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const int rank_w = __popcll(mask & lt);
    if (live && rank_w == 0) s_tab[wave][e] = __popcll(mask);
    __syncthreads();
    if (live) {
      int before = s_run[e];
      for (int w = 0; w < wave; ++w) before += s_tab[w][e];
      const int p = s_off[e] + before + rank_w;
      out.perm[p] = a;
      out.sorted_ids[p] = e;
      out.inv_pos[a] = p;
      if (a < A) {
        out.perm_token[p] = a / K;
        out.perm_weight[p] = weights[a];
      } else {
        out.perm_token[p] = a - A;
        out.perm_weight[p] = 1.0f;
      }
    }
    __syncthreads();
    for (int x = tid; x < E_ext; x += kRouteThreads) {
      int s = 0;
      for (int w = 0; w < kRouteWaves; ++w) s += s_tab[w][x];
      s_run[x] += s;
    }
    __syncthreads();
  }
  // 5. counts / offsets / tile list
  for (int e = tid; e < E_ext; e += kRouteThreads) {
    out.counts[e] = s_cnt[e];
    out.offsets[e] = s_off[e];
    const int nt = (s_cnt[e] + block_m - 1) / block_m;
    for (int t = 0; t < nt; ++t) {
      const int slot = s_toff[e] + t;
      if (slot < tile_cap) {
        out.tile_expert[slot] = e;
        out.tile_start[slot] = t * block_m;
        out.tile_rows[slot] = min(block_m, s_cnt[e] - t * block_m);
      }
    }
  }
  if (tid == 0) {
    out.offsets[E_ext] = s_off[E_ext];
    out.n_tiles[0] = min(s_toff[E_ext], tile_cap);
  }
}

// Routing only: one wave per token.
__global__ void __launch_bounds__(256) route_topk_kernel(const float* __restrict__ logits,
                                                         const float* __restrict__ bias, int32_t* ids, float* w,
                                                         int M, int E, int K, int func, int renorm,
                                                         float route_scale) {
  const int t = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  if (t >= M) return;
  route_one_token(logits + (int64_t)t * E, E, K, func, renorm, route_scale, bias, ids + (int64_t)t * K,
                  w + (int64_t)t * K);
}


// Tile list from expert counts (emit_tiles contract, no per-expert cap).
__global__ void __launch_bounds__(1024) emit_tiles_kernel(const int32_t* __restrict__ counts, int E, int block_m,
                                                          int32_t* tile_expert, int32_t* tile_start,
                                                          int32_t* tile_rows, int32_t* n_tiles, int tile_cap) {
  __shared__ int32_t s_toff[4097];
  const int tid = threadIdx.x, lane = tid & 63;
  if (tid < 64) {
    int carry = 0;
    for (int base = 0; base < E; base += 64) {
      int e = base + lane;
      int c = (e < E) ? counts[e] : 0;
      int tc = c > 0 ? (c + block_m - 1) / block_m : 0;
      int inc = tc;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        int o = __shfl_up(inc, off, 64);
        if (lane >= off) inc += o;
      }
      if (e < E) s_toff[e] = carry + inc - tc;
      carry += __shfl(inc, 63, 64);
    }
    if (lane == 0) s_toff[E] = carry;
  }
  __syncthreads();
  for (int e = tid; e < E; e += blockDim.x) {
    const int c = counts[e];
    const int nt = c > 0 ? (c + block_m - 1) / block_m : 0;
    for (int t = 0; t < nt; ++t) {
      const int slot = s_toff[e] + t;
      if (slot < tile_cap) {
        tile_expert[slot] = e;
        tile_start[slot] = t * block_m;
        tile_rows[slot] = min(block_m, c - t * block_m);
      }
    }
  }
  if (tid == 0) n_tiles[0] = min(s_toff[E], tile_cap);
}

int launch_route_layout(const float* logits, const float* bias, int32_t* ids, float* weights, int64_t M, int64_t E,
                        int64_t K, int func, int renorm, float route_scale, int has_shared, int block_m,
                        int64_t tile_cap, const LayoutOut& out, hipStream_t st) {
  const int64_t A_ext = M * K + (has_shared ? M : 0);
  MOSAIC_CHECK_ARG(M >= 1 && E >= 1 && K >= 1, "moe layout: M=%lld E=%lld K=%lld", (long long)M, (long long)E,
                   (long long)K);
  MOSAIC_CHECK_ARG(E <= kRouteMaxExperts, "moe layout: E=%lld exceeds %d", (long long)E, kRouteMaxExperts);
  MOSAIC_CHECK_ARG(K <= kRouteMaxTopK && K <= E, "moe layout: top_k=%lld (max %d, <= E)", (long long)K,
                   kRouteMaxTopK);
  MOSAIC_CHECK_ARG(A_ext <= kRouteMaxAssign, "moe layout: %lld assignments exceed %d", (long long)A_ext,
                   kRouteMaxAssign);
  MOSAIC_CHECK_ARG(block_m >= 1, "moe layout: block_m=%d", block_m);
  MOSAIC_CHECK_ARG(func >= 0 && func <= 2, "moe layout: score func %d", func);
  hipLaunchKernelGGL(route_layout_kernel, dim3(1), dim3(kRouteThreads), 0, st, logits, bias, ids, weights, (int)M,
                     (int)E, (int)K, func, renorm, route_scale, has_shared, block_m, (int)tile_cap, out);
  MOSAIC_RETURN_LAUNCH("moe_route_layout");
}

}  // namespace mosaic

using namespace mosaic;

extern "C" int mosaic_moe_route_topk(const float* logits, int64_t m, int64_t e, int64_t top_k, int score_func,
                                     int renorm, float route_scale, const float* bias, int32_t* ids, float* weights,
                                     void* stream) {
  MOSAIC_CHECK_ARG(logits && ids && weights, "moe_route_topk: null pointer");
  MOSAIC_CHECK_ARG(e >= 1 && e <= kRouteMaxExperts, "moe_route_topk: E=%lld (1..%d)", (long long)e,
                   kRouteMaxExperts);
  MOSAIC_CHECK_ARG(top_k >= 1 && top_k <= kRouteMaxTopK && top_k <= e, "moe_route_topk: top_k=%lld",
                   (long long)top_k);
  MOSAIC_CHECK_ARG(score_func >= 0 && score_func <= 2, "moe_route_topk: score func %d", score_func);
  if (m <= 0) return kOk;
  unsigned grid = (unsigned)((m * 64 + 255) / 256);
  hipLaunchKernelGGL(route_topk_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, logits, bias, ids, weights,
                     (int)m, (int)e, (int)top_k, score_func, renorm, route_scale);
  MOSAIC_RETURN_LAUNCH("moe_route_topk");
}

extern "C" int mosaic_moe_layout(const int32_t* ids, const float* weights, int64_t m, int64_t top_k, int64_t e,
                                 int has_shared, int block_m, int32_t* counts, int32_t* offsets, int32_t* perm,
                                 int32_t* perm_token, float* perm_weight, int32_t* sorted_ids, int32_t* inv_pos,
                                 int32_t* tile_expert, int32_t* tile_start, int32_t* tile_rows, int32_t* n_tiles,
                                 int64_t tile_cap, void* stream) {
  MOSAIC_CHECK_ARG(ids && weights && counts && offsets && perm && perm_token && perm_weight && sorted_ids &&
                       inv_pos && tile_expert && tile_start && tile_rows && n_tiles,
                   "moe_layout: null pointer");
  LayoutOut out{counts, offsets, perm, perm_token, perm_weight, sorted_ids, inv_pos,
                tile_expert, tile_start, tile_rows, n_tiles};
  return launch_route_layout(nullptr, nullptr, const_cast<int32_t*>(ids), const_cast<float*>(weights), m, e, top_k,
                             0, 0, 1.0f, has_shared, block_m, tile_cap, out, (hipStream_t)stream);
}

extern "C" int mosaic_emit_tiles(const int32_t* counts, int64_t e, int block_m, int32_t* tile_expert,
                                 int32_t* tile_start, int32_t* tile_rows, int32_t* n_tiles, int64_t tile_cap,
                                 void* stream) {
  MOSAIC_CHECK_ARG(counts && tile_expert && tile_start && tile_rows && n_tiles, "emit_tiles: null pointer");
  MOSAIC_CHECK_ARG(e >= 1 && e <= 4096, "emit_tiles: E=%lld (1..4096)", (long long)e);
  MOSAIC_CHECK_ARG(block_m >= 1, "emit_tiles: block_m=%d", block_m);
  MOSAIC_CHECK_ARG(tile_cap >= 0 && tile_cap < (1ll << 31), "emit_tiles: tile_cap=%lld", (long long)tile_cap);
  hipLaunchKernelGGL(emit_tiles_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, counts, (int)e, block_m,
                     tile_expert, tile_start, tile_rows, n_tiles, (int)tile_cap);
  MOSAIC_RETURN_LAUNCH("emit_tiles");
}
