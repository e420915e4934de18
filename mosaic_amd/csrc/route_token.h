// Per-token router shared by the layout kernels and the fused decode kernels:
// scores, top-k with ties to the lower expert index, renormalization.
#pragma once
#include "common.h"
#include "../../include/mosaic_amd.h"

namespace mosaic {

constexpr int kRouteMaxExperts = 512;   // routed experts (+1 virtual shared expert)
constexpr int kRouteMaxTopK = 16;

// fp32 -> unsigned key with the same order (NaN -> smallest)
__device__ __forceinline__ uint32_t order_key(float f) {
  if (f != f) return 0u;
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Router score, defined as the fp32 rounding of the exact function value: it
// is evaluated in fp64 and rounded once, so the device and a CPU restatement
// (also fp64, rounded once) agree bit for bit, ties included.  sqrtsoftplus
// keeps torch's softplus threshold (x > 20 -> x).
__device__ __forceinline__ float score_of(float logit, int func) {
  const double x = (double)logit;
  if (func == MOSAIC_SCORE_SIGMOID) return (float)(1.0 / (1.0 + exp(-x)));
  if (func == MOSAIC_SCORE_SQRTSOFTPLUS) return (float)sqrt(logit > 20.f ? x : log1p(exp(x)));
  return logit;  // softmax handled by the caller
}

// inverse of order_key (0 -> NaN)
__device__ __forceinline__ float key_value(uint32_t k) {
  if (k == 0u) return __uint_as_float(0x7FC00000u);
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// K selection rounds over one wave's candidates (PER per lane, keys khi, ties
// by klo = ~index, a carried float cv).  Each lane's list is sorted once; a
// round then reduces only the lane heads (two 32-bit DPP max-reductions, the
// second only when several lanes hold the winning key) and the winning lane
// shifts its list.  Lane r < K receives pick r's index and carried value.
// Returns the largest key left after the K rounds (0 when none is left).
template <int PER>
__device__ __forceinline__ uint32_t select_rounds(uint32_t (&khi)[PER], uint32_t (&klo)[PER], float (&cv)[PER], int K,
                                                  int& my_pick, float& my_val) {
  const int lane = threadIdx.x & 63;
  auto cex = [&](int i, int j) {  // order candidates i < j descending
    const bool sw = khi[j] > khi[i] || (khi[j] == khi[i] && klo[j] > klo[i]);
    const uint32_t hi_i = sw ? khi[j] : khi[i], hi_j = sw ? khi[i] : khi[j];
    const uint32_t lo_i = sw ? klo[j] : klo[i], lo_j = sw ? klo[i] : klo[j];
    const float c_i = sw ? cv[j] : cv[i], c_j = sw ? cv[i] : cv[j];
    khi[i] = hi_i; khi[j] = hi_j; klo[i] = lo_i; klo[j] = lo_j; cv[i] = c_i; cv[j] = c_j;
  };
  if constexpr (PER == 2) {
    cex(0, 1);
  } else if constexpr (PER == 4) {
    cex(0, 1); cex(2, 3); cex(0, 2); cex(1, 3); cex(1, 2);
  } else if constexpr (PER == 8) {  // Batcher odd-even merge sort
    cex(0, 1); cex(2, 3); cex(4, 5); cex(6, 7);
    cex(0, 2); cex(1, 3); cex(4, 6); cex(5, 7); cex(1, 2); cex(5, 6);
    cex(0, 4); cex(1, 5); cex(2, 6); cex(3, 7); cex(2, 4); cex(3, 5); cex(1, 2); cex(3, 4); cex(5, 6);
  }
  my_pick = -1;
  my_val = 0.f;
  for (int r = 0; r < K; ++r) {
    const uint32_t hi = wave_max_u32(khi[0]);
    const uint64_t at_max = __ballot(khi[0] == hi);
    const uint32_t lo = (__builtin_popcountll(at_max) == 1)
                            ? wave_bcast_u32(klo[0], __builtin_ctzll(at_max))
                            : wave_max_u32(khi[0] == hi ? klo[0] : 0u);
    const int e = (int)(0xFFFFFFFFu - lo);
    const int src = e & 63;  // expert e lives in lane e % 64
    const float c = __uint_as_float(wave_bcast_u32(__float_as_uint(cv[0]), src));
    const bool win = lane == src;
#pragma unroll
    for (int j = 0; j < PER - 1; ++j) {
      khi[j] = win ? khi[j + 1] : khi[j];
      klo[j] = win ? klo[j + 1] : klo[j];
      cv[j] = win ? cv[j + 1] : cv[j];
    }
    khi[PER - 1] = win ? 0u : khi[PER - 1];
    klo[PER - 1] = win ? 0u : klo[PER - 1];
    if (lane == r) {
      my_pick = e;
      my_val = c;
    }
  }
  return wave_max_u32(khi[0]);
}

// One wave routes one token; logits stay in registers (PER per lane, E <=
// 64*PER).  Selection key: the fp32 score (score_of; softmax = exp(x - max) /
// sum in fp64, rounded once), plus bias when given (one fp32 add); ties ->
// lower index.  Without a bias, sigmoid and sqrtsoftplus first select on the
// logit (the scores are a monotone function of it, so the same experts in the
// same order unless two of the picks, or the last pick and the best logit
// left, share one fp32 score); only the K + 1 scores involved are evaluated,
// and a score tie among them (rare) reruns the selection on the scores
// themselves.  On return lane r < K holds pick r (rank order) and its weight:
// score / max(fp32 sum of the K scores in rank order, 1e-9) when
// renormalizing (not softmax), times `scale`; other lanes hold -1 and 0.
template <int PER>
__device__ __forceinline__ void route_token_regs(const float* __restrict__ lg, int E, int K, int func, int renorm,
                                                 float scale, const float* __restrict__ bias, int& pick,
                                                 float& weight) {
  const int lane = threadIdx.x & 63;
  float lv[PER];
  uint32_t khi[PER], klo[PER];
  float cv[PER];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = lane + 64 * j;
    lv[j] = (e < E) ? lg[e] : -INFINITY;
    mx = fmaxf(mx, lv[j]);
  }
  int my_pick = -1;
  float my_score = 0.f;
  bool by_score = bias != nullptr || func == MOSAIC_SCORE_SOFTMAX;
  if (!by_score) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int e = lane + 64 * j;
      khi[j] = (e < E) ? order_key(lv[j]) : 0u;  // absent experts sort below every real one
      klo[j] = (e < E) ? 0xFFFFFFFFu - (uint32_t)e : 0u;
      cv[j] = lv[j];
    }
    float my_logit;
    const uint32_t rest = select_rounds<PER>(khi, klo, cv, K, my_pick, my_logit);
    // lanes < K: the picks' scores; lane K: the score of the best logit left
    const bool more = rest != 0u;
    const float sq = score_of(lane < K ? my_logit : (lane == K && more ? key_value(rest) : 0.f), func);
    const float s_next = __shfl_down(sq, 1, 64);
    const bool has_next = lane + 1 < K || (lane + 1 == K && more);
    by_score = __ballot(lane < K && has_next && sq == s_next) != 0;  // a score tie: select on the scores
    my_score = sq;
  }
  if (by_score) {
    if (func == MOSAIC_SCORE_SOFTMAX) {
      mx = wave_max_f32(mx);
      double ex[PER];
      double sum = 0.0;
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        ex[j] = (lane + 64 * j < E) ? exp((double)lv[j] - (double)mx) : 0.0;
        sum += ex[j];
      }
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
#pragma unroll
      for (int j = 0; j < PER; ++j) cv[j] = (float)(ex[j] / sum);
    } else {
#pragma unroll
      for (int j = 0; j < PER; ++j) cv[j] = (lane + 64 * j < E) ? score_of(lv[j], func) : 0.f;
    }
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int e = lane + 64 * j;
      const float k = (bias && e < E) ? cv[j] + bias[e] : cv[j];
      khi[j] = (e < E) ? order_key(k) : 0u;
      klo[j] = (e < E) ? 0xFFFFFFFFu - (uint32_t)e : 0u;
    }
    (void)select_rounds<PER>(khi, klo, cv, K, my_pick, my_score);
  }
  const float sc = (lane < K) ? my_score : 0.f;
  float sum = 0.f;
  for (int r = 0; r < K; ++r) sum += __uint_as_float(wave_bcast_u32(__float_as_uint(sc), r));  // rank order
  float w = sc;
  if (renorm && func != MOSAIC_SCORE_SOFTMAX) w = w / (sum < 1e-9f ? 1e-9f : sum);  // clamp_min, NaN kept
  w = w * scale;
  pick = lane < K ? my_pick : -1;
  weight = lane < K ? w : 0.f;
}

// route_token_regs, then picks/weights to s_ids/s_w (workgroup scratch; the
// caller synchronizes before reading them) and to ids_out/w_out when given.
template <int PER>
__device__ __forceinline__ void route_one_token_t(const float* __restrict__ lg, int E, int K, int func, int renorm,
                                                  float scale, const float* __restrict__ bias, int16_t* s_ids,
                                                  float* s_w, int32_t* ids_out, float* w_out) {
  const int lane = threadIdx.x & 63;
  int pick;
  float w;
  route_token_regs<PER>(lg, E, K, func, renorm, scale, bias, pick, w);
  if (lane < K) {
    s_ids[lane] = (int16_t)pick;
    s_w[lane] = w;
    if (w_out) {
      w_out[lane] = w;
      ids_out[lane] = pick;
    }
  }
}

// picks in registers (see route_token_regs), E <= 512
__device__ __forceinline__ void route_token_any(const float* __restrict__ lg, int E, int K, int func, int renorm,
                                                float scale, const float* __restrict__ bias, int& pick,
                                                float& weight) {
  if (E <= 64)
    route_token_regs<1>(lg, E, K, func, renorm, scale, bias, pick, weight);
  else if (E <= 128)
    route_token_regs<2>(lg, E, K, func, renorm, scale, bias, pick, weight);
  else if (E <= 256)
    route_token_regs<4>(lg, E, K, func, renorm, scale, bias, pick, weight);
  else
    route_token_regs<8>(lg, E, K, func, renorm, scale, bias, pick, weight);
}

__device__ __forceinline__ void route_one_token(const float* __restrict__ lg, int E, int K, int func, int renorm,
                                                float scale, const float* __restrict__ bias, int16_t* s_ids,
                                                float* s_w, int32_t* ids_out, float* w_out) {
  if (E <= 64)
    route_one_token_t<1>(lg, E, K, func, renorm, scale, bias, s_ids, s_w, ids_out, w_out);
  else if (E <= 128)
    route_one_token_t<2>(lg, E, K, func, renorm, scale, bias, s_ids, s_w, ids_out, w_out);
  else if (E <= 256)
    route_one_token_t<4>(lg, E, K, func, renorm, scale, bias, s_ids, s_w, ids_out, w_out);
  else
    route_one_token_t<8>(lg, E, K, func, renorm, scale, bias, s_ids, s_w, ids_out, w_out);
}

}  // namespace mosaic
