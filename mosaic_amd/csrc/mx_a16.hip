// A16 MXFP4 path on gfx950: bf16 activations against MXFP4 weights decoded in
// registers (v_cvt_scalef32_pk_bf16_fp4, block scale applied in the convert)
// and multiplied on v_mfma_f32_16x16x32_bf16 with fp32 accumulation.
//
// MFMA tile: one wave owns a 16 (tokens) x 16 (weight rows) output tile and
// walks K in super-steps of 128.  In a super-step lane l (c = l%16, q = l/16)
// holds the 16-byte MX block b = 4S+q of weight row c (32 nibbles + one e8m0
// byte) and the 32 bf16 of token row c at the same K, and issues four MFMAs
// over the 8-element sub-slices.  A and B use the same lane->K map, so the K
// order inside the MFMA is irrelevant to the result.
//
// Weight layouts:
//  * raw NK ([N, K/2] + [N, K/32], the checkpoint layout): each wave load
//    touches 16 rows x 64 B;
//  * MXT16 (prepacked, codec.hip): the 64 lanes' blocks of one super-step are
//    one contiguous 1 KB, scales one contiguous 256 B per 4 super-steps, so
//    every weight load is a fully coalesced streaming read.
#include <algorithm>

#include "common.h"
#include "moe_internal.h"
#include "route_token.h"
#include "../../include/mosaic_amd.h"

namespace mosaic {

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

// x operand of one super-step: 32 bf16 of the lane's token row (zeros if invalid)
__device__ __forceinline__ void load_x_step(const uint16_t* __restrict__ xrow, bool xvalid, int q, int S,
                                            u32x4_t (&xv)[4]) {
  if (xvalid) {
    const u32x4_t* xp = reinterpret_cast<const u32x4_t*>(xrow + 32 * (4 * S + q));
#pragma unroll
    for (int j = 0; j < 4; ++j) xv[j] = xp[j];
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) xv[j] = u32x4_t{0u, 0u, 0u, 0u};
  }
}

__device__ __forceinline__ void mfma_block(const u32x4_t w, float sf, const u32x4_t (&xv)[4], f32x4_t& acc) {
  bf16x8_t wb[4];
  mx_block_to_bf16(w, sf, wb);
#pragma unroll
  for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xv[s]), wb[s], acc, 0, 0, 0);
}

// ------------------------------------------------------- raw NK layout -----
template <int T, int U>
__device__ __forceinline__ void raw_batch(const uint8_t* const (&wp)[T], const uint8_t* const (&sp)[T],
                                          const uint16_t* __restrict__ xrow, bool xvalid, int q, int S,
                                          f32x4_t (&acc)[T]) {
  u32x4_t wv[U][T];
  uint32_t sv[U][T];
  u32x4_t xv[U][4];
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int t = 0; t < T; ++t) {
      wv[u][t] = load_nt_u32x4(wp[t] + 16 * (4 * (S + u) + q));
      sv[u][t] = *reinterpret_cast<const uint32_t*>(sp[t] + 4 * (S + u));
    }
#pragma unroll
  for (int u = 0; u < U; ++u) load_x_step(xrow, xvalid, q, S + u, xv[u]);
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int t = 0; t < T; ++t) mfma_block(wv[u][t], e8m0_f32((sv[u][t] >> (8 * q)) & 0xFFu), xv[u], acc[t]);
}

template <int T>
__device__ __forceinline__ void tile_dot_raw(const uint8_t* const (&wp)[T], const uint8_t* const (&sp)[T],
                                             const uint16_t* __restrict__ xrow, bool xvalid, int q, int s0, int s1,
                                             f32x4_t (&acc)[T]) {
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  int S = s0;
  for (; S + 2 <= s1; S += 2) raw_batch<T, 2>(wp, sp, xrow, xvalid, q, S, acc);
  if (S < s1) raw_batch<T, 1>(wp, sp, xrow, xvalid, q, S, acc);
}

// ---------------------------------------------------------- MXT16 layout ---
// wt[t] = packed_t of row group g_t + 16*lane; st[t] = scale_t of g_t + 4*lane.
// A group is the 4 super-steps of one scale dword (S % 4 == 0).
template <int T>
__device__ __forceinline__ void t16_group(const uint8_t* const (&wt)[T], const uint8_t* const (&st)[T],
                                          const uint16_t* __restrict__ xrow, bool xvalid, int q, int S,
                                          f32x4_t (&acc)[T]) {
  u32x4_t wv[4][T];
  uint32_t sv[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
#pragma unroll
    for (int u = 0; u < 4; ++u) wv[u][t] = load_nt_u32x4(wt[t] + (int64_t)(S + u) * 1024);
    sv[t] = *reinterpret_cast<const uint32_t*>(st[t] + (int64_t)(S >> 2) * 256);
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    u32x4_t xv[4];
    load_x_step(xrow, xvalid, q, S + u, xv);
#pragma unroll
    for (int t = 0; t < T; ++t) mfma_block(wv[u][t], e8m0_f32((sv[t] >> (8 * u)) & 0xFFu), xv, acc[t]);
  }
}

template <int T>
__device__ __forceinline__ void t16_step(const uint8_t* const (&wt)[T], const uint8_t* const (&st)[T],
                                         const uint16_t* __restrict__ xrow, bool xvalid, int q, int S,
                                         f32x4_t (&acc)[T]) {
  u32x4_t wv[T];
  uint32_t sv[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    wv[t] = load_nt_u32x4(wt[t] + (int64_t)S * 1024);
    sv[t] = *reinterpret_cast<const uint32_t*>(st[t] + (int64_t)(S >> 2) * 256);
  }
  u32x4_t xv[4];
  load_x_step(xrow, xvalid, q, S, xv);
#pragma unroll
  for (int t = 0; t < T; ++t) mfma_block(wv[t], e8m0_f32((sv[t] >> (8 * (S & 3))) & 0xFFu), xv, acc[t]);
}

// super-steps [s0, s1); s0 is a multiple of 4
template <int T>
__device__ __forceinline__ void tile_dot_t16(const uint8_t* const (&wt)[T], const uint8_t* const (&st)[T],
                                             const uint16_t* __restrict__ xrow, bool xvalid, int q, int s0, int s1,
                                             f32x4_t (&acc)[T]) {
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  int S = s0;
  for (; S + 4 <= s1; S += 4) t16_group<T>(wt, st, xrow, xvalid, q, S, acc);
  for (; S < s1; ++S) t16_step<T>(wt, st, xrow, xvalid, q, S, acc);
}

// K slice of wave ks out of KS: whole 4-step groups, the last wave takes the tail
__device__ __forceinline__ void k_slice(int ns, int ks, int KS, int& s0, int& s1) {
  const int ng = ns / 4;
  s0 = 4 * (ng * ks / KS);
  s1 = (ks == KS - 1) ? ns : 4 * (ng * (ks + 1) / KS);
}

// MXT16 pointers of row group g for this lane
__device__ __forceinline__ void t16_ptrs(const uint8_t* pt, const uint8_t* st, int64_t g, int ns, int lane,
                                         const uint8_t*& w, const uint8_t*& s) {
  const int ns4 = (ns + 3) / 4;
  w = pt + (g * ns * 64 + lane) * 16;
  s = st + (g * ns4 * 64 + lane) * 4;
}

// ---------------------------------------------------- MoE gate/up + SwiGLU --
// One workgroup's share of a tile: Column tiles 0..T/2-1 are gate row groups
// (j0/16 + t), tiles T/2.. the matching up row groups, so after the K
// reduction gate and up of one z element sit in the same lane.  Row c of the
// tile is token toks[c] (c < rows) with route weight rw[c]; z row p0 + c.
template <int T, int KS>
__device__ __forceinline__ void gateup_tile(const uint16_t* __restrict__ x, const uint8_t* bp, const uint8_t* bs,
                                            const int32_t* toks, const float* rw, int rows, int p0,
                                            uint16_t* __restrict__ z, int H, int I, float limit,
                                            f32x4_t (&red)[KS][T][64]) {
  const int lane = threadIdx.x & 63, ks = threadIdx.x >> 6;
  const int c = lane & 15, q = lane >> 4;
  const int j0 = blockIdx.x * 8 * T;
  const int ns = H / 128;
  const uint8_t* wt[T];
  const uint8_t* st[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int g = (t < T / 2) ? (j0 / 16 + t) : ((I + j0) / 16 + t - T / 2);
    t16_ptrs(bp, bs, g, ns, lane, wt[t], st[t]);
  }
  const bool xvalid = c < rows;
  const uint16_t* xrow = x + (int64_t)(xvalid ? toks[c] : 0) * H;
  int s0, s1;
  k_slice(ns, ks, KS, s0, s1);
  f32x4_t acc[T];
  tile_dot_t16<T>(wt, st, xrow, xvalid, q, s0, s1, acc);
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
        const float zv = swiglu_f32(g[r], u[r], limit) * rw[ti];
        z[(int64_t)(p0 + ti) * I + j0 + 16 * t + c] = f32_bf16(zv);
      }
    }
  }
}

// grid (inter/(8T), tile_cap), KS waves: tile blockIdx.y of the layout's list
template <int T, int KS>
__global__ void __launch_bounds__(KS * 64) moe_a16_gateup_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ gu_p, const uint8_t* __restrict__ gu_s,
    const uint8_t* __restrict__ sh_p, const uint8_t* __restrict__ sh_s, const int32_t* __restrict__ tile_expert,
    const int32_t* __restrict__ tile_rows, const int32_t* __restrict__ tile_p0, const int32_t* __restrict__ n_tiles,
    const int32_t* __restrict__ perm_token, const float* __restrict__ perm_weight, uint16_t* __restrict__ z, int H,
    int I, int E, float limit) {
  __shared__ f32x4_t red[KS][T][64];
  const int tile = blockIdx.y;
  if (tile >= n_tiles[0]) return;
  const int e = tile_expert[tile], rows = tile_rows[tile], p0 = tile_p0[tile];
  const int ns4 = (H / 128 + 3) / 4;
  const int64_t ebytes = (int64_t)2 * I * (H / 2), sbytes = (int64_t)(2 * I / 16) * ns4 * 256;
  const uint8_t* bp = (e == E) ? sh_p : gu_p + (int64_t)e * ebytes;
  const uint8_t* bs = (e == E) ? sh_s : gu_s + (int64_t)e * sbytes;
  gateup_tile<T, KS>(x, bp, bs, perm_token + p0, perm_weight + p0, rows, p0, z, H, I, limit, red);
}

// 2..kSmallGuTokens tokens routed on the device, without a layout launch:
// grid (inter/(8T), R), KS >= M waves, R rows of workgroups small enough for
// the whole grid to be resident, so every workgroup routes once.  Wave t
// routes token t (the arithmetic of the layout kernels, so ids and weights are
// identical); wave 0 then sorts the M*K picks by (expert id, flat index) as
// the layout does (positions = ranks; one tile per distinct expert in
// ascending id, at most one row per token; the shared expert's tile last, its
// rows at positions M*K.., every pick being valid) into an LDS tile table, and
// the workgroup takes tiles blockIdx.y, blockIdx.y + R, ...  Workgroup (0, 0)
// also writes the ids / weights and what the down kernel reads: the tile
// list, perm_token and perm_weight.
constexpr int kSmallGuTokens = 4;
constexpr int kSmallGuTiles = kSmallGuTokens * kRouteMaxTopK + 1;
constexpr int kSmallGuResidentWgs = 768;  // 3 four-wave workgroups per CU at <= 168 VGPRs

template <int T, int KS>
__global__ void __launch_bounds__(KS * 64) moe_small_gateup_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ logits, const float* __restrict__ bias,
    int32_t* __restrict__ ids_out, float* __restrict__ w_out, const uint8_t* __restrict__ gu_p,
    const uint8_t* __restrict__ gu_s, const uint8_t* __restrict__ sh_p, const uint8_t* __restrict__ sh_s,
    int32_t* __restrict__ tile_expert, int32_t* __restrict__ tile_rows, int32_t* __restrict__ tile_p0,
    int32_t* __restrict__ n_tiles, int32_t* __restrict__ perm_token, float* __restrict__ perm_weight,
    uint16_t* __restrict__ z, int M, int H, int I, int E, int K, int has_shared, int func, int renorm,
    float route_scale, float limit) {
  static_assert(KS >= kSmallGuTokens, "one routing wave per token");
  __shared__ f32x4_t red[KS][T][64];
  __shared__ int16_t s_ids[kSmallGuTokens * kRouteMaxTopK];
  __shared__ float s_w[kSmallGuTokens * kRouteMaxTopK];
  __shared__ int s_te[kSmallGuTiles], s_rows[kSmallGuTiles], s_p0[kSmallGuTiles];
  __shared__ int32_t s_tok[kSmallGuTiles][kSmallGuTokens];
  __shared__ float s_rw[kSmallGuTiles][kSmallGuTokens];
  __shared__ int s_nt;
  const int lane = threadIdx.x & 63, ks = threadIdx.x >> 6;
  const int A = M * K;
  // 1. routing: wave t routes token t
  if (ks < M)
    route_one_token(logits + (int64_t)ks * E, E, K, func, renorm, route_scale, bias, s_ids + ks * K, s_w + ks * K,
                    nullptr, nullptr);
  __syncthreads();
  // 2. wave 0: lane a < A holds pick a; its stable rank by (expert, a), the
  //    count of its expert, first occurrence, and the rank of its expert among
  //    the distinct experts -> the tile table
  if (ks == 0) {
    const bool va = lane < A;
    const int ea = va ? s_ids[lane] : 0x7FFF;
    const float wa = va ? s_w[lane] : 0.f;
    int rank = 0, cnt = 0, dup = 0;  // dup: earlier picks of the same expert = row in its tile
    for (int b = 0; b < A; ++b) {
      const int eb = __builtin_amdgcn_readlane(ea, b);
      rank += (eb < ea || (eb == ea && b < lane)) ? 1 : 0;
      cnt += eb == ea ? 1 : 0;
      dup += (eb == ea && b < lane) ? 1 : 0;
    }
    const bool first = dup == 0;
    const uint64_t fm = __ballot(va && first);
    int dr = 0;
    for (int b = 0; b < A; ++b) {
      const int eb = __builtin_amdgcn_readlane(ea, b);
      dr += (((fm >> b) & 1ull) && eb < ea) ? 1 : 0;
    }
    const int n_routed = __builtin_popcountll(fm);
    if (va && first) {
      s_te[dr] = ea;
      s_rows[dr] = cnt;
      s_p0[dr] = rank;
    }
    // row dup of tile dr: the pick's token and route weight (the picks of one
    // token are distinct experts, so dup < M)
    if (va) {
      s_tok[dr][dup] = lane / K;
      s_rw[dr][dup] = wa;
    }
    if (has_shared && lane < kSmallGuTokens) {
      s_tok[n_routed][lane] = min(lane, M - 1);
      s_rw[n_routed][lane] = 1.0f;
    }
    if (lane == 0) {
      if (has_shared) {
        s_te[n_routed] = E;
        s_rows[n_routed] = M;
        s_p0[n_routed] = A;
      }
      s_nt = n_routed + has_shared;
    }
    if (blockIdx.x == 0 && blockIdx.y == 0) {
      if (va) {
        ids_out[lane] = ea;
        w_out[lane] = wa;
        perm_token[rank] = lane / K;
        perm_weight[rank] = wa;
        if (first) {
          tile_expert[dr] = ea;
          tile_rows[dr] = cnt;
          tile_p0[dr] = rank;
        }
      }
      if (has_shared && lane < M) {
        perm_token[A + lane] = lane;
        perm_weight[A + lane] = 1.0f;
      }
      if (lane == 0) {
        if (has_shared) {
          tile_expert[n_routed] = E;
          tile_rows[n_routed] = M;
          tile_p0[n_routed] = A;
        }
        n_tiles[0] = n_routed + has_shared;
      }
    }
  }
  __syncthreads();
  const int ns4 = (H / 128 + 3) / 4;
  const int64_t ebytes = (int64_t)2 * I * (H / 2), sbytes = (int64_t)(2 * I / 16) * ns4 * 256;
  const int nt = s_nt;
  for (int u = blockIdx.y; u < nt; u += gridDim.y) {
    const int e = s_te[u];
    const uint8_t* bp = e == E ? sh_p : gu_p + (int64_t)e * ebytes;
    const uint8_t* bs = e == E ? sh_s : gu_s + (int64_t)e * sbytes;
    gateup_tile<T, KS>(x, bp, bs, s_tok[u], s_rw[u], s_rows[u], s_p0[u], z, H, I, limit, red);
    __syncthreads();  // red is rewritten by the next tile
  }
}

// ------------------------------------------------------------- MoE down ----
// grid (H/(16T), tile_cap), KS waves: fp32 partial rows yp[p][h] per sorted
// assignment position p.
template <int T, int KS>
__global__ void __launch_bounds__(KS * 64) moe_a16_down_kernel(
    const uint16_t* __restrict__ z, const uint8_t* __restrict__ d_p, const uint8_t* __restrict__ d_s,
    const uint8_t* __restrict__ sh_p, const uint8_t* __restrict__ sh_s, const int32_t* __restrict__ tile_expert,
    const int32_t* __restrict__ tile_rows, const int32_t* __restrict__ tile_p0, const int32_t* __restrict__ n_tiles,
    float* __restrict__ yp, int H, int I, int E) {
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
  for (int t = 0; t < T; ++t) t16_ptrs(bp, bs, h0 / 16 + t, ns, lane, wt[t], st[t]);
  const bool xvalid = c < rows;
  const uint16_t* zrow = z + (int64_t)(p0 + (xvalid ? c : 0)) * I;
  int s0, s1;
  k_slice(ns, ks, KS, s0, s1);
  f32x4_t acc[T];
  tile_dot_t16<T>(wt, st, zrow, xvalid, q, s0, s1, acc);
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
      if (ti < rows) yp[(int64_t)(p0 + ti) * H + h0 + 16 * t + c] = v[r];
    }
  }
}

// ------------------------------------------------------------ combine ------
// y[t][h] = bf16( sum over j of yp[combine_pos[t][j]][h] ): the token's expert
// partials in ascending expert id, the shared expert last.  W <= kCombineMaxW:
// every partial load is issued before the in-order sum (a loop over W would
// wait for each position and partial in turn).
__global__ void __launch_bounds__(256) moe_combine_kernel(const float* __restrict__ yp,
                                                          const int32_t* __restrict__ combine_pos,
                                                          uint16_t* __restrict__ y, int M, int W, int H) {
  const int t = blockIdx.y;
  const int h = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= M || h >= H) return;
  float v[kCombineMaxW];
  bool ok[kCombineMaxW];
#pragma unroll
  for (int j = 0; j < kCombineMaxW; ++j) {
    const int p = j < W ? combine_pos[(int64_t)t * W + j] : -1;
    ok[j] = p >= 0;
    v[j] = ok[j] ? yp[(int64_t)p * H + h] : 0.f;
  }
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < kCombineMaxW; ++j)
    if (ok[j]) sum += v[j];
  y[(int64_t)t * H + h] = f32_bf16(sum);
}

// ------------------------------------------------------- single linear -----
// y [M, N] = x [M, K] . W^T.  grid (ceil(N/(16T)), ceil(M/16)), KS waves take
// K slices of the same T column tiles; slices meet in LDS in slice order.
template <int T, int KS, bool TILED>
__global__ void __launch_bounds__(KS * 64) mx_linear_a16_kernel(const uint16_t* __restrict__ x,
                                                                 const uint8_t* __restrict__ packed,
                                                                 const uint8_t* __restrict__ scale,
                                                                 uint16_t* __restrict__ y, int M, int N, int K) {
  __shared__ f32x4_t red[KS][T][64];
  const int lane = threadIdx.x & 63, ks = threadIdx.x >> 6;
  const int c = lane & 15, q = lane >> 4;
  const int n0 = blockIdx.x * 16 * T, m0 = blockIdx.y * 16;
  const bool xvalid = (m0 + c) < M;
  const uint16_t* xrow = x + (int64_t)(xvalid ? m0 + c : 0) * K;
  const int ns = K / 128;
  f32x4_t acc[T];
  if constexpr (TILED) {
    const uint8_t* wt[T];
    const uint8_t* st[T];
#pragma unroll
    for (int t = 0; t < T; ++t) t16_ptrs(packed, scale, min(n0 / 16 + t, N / 16 - 1), ns, lane, wt[t], st[t]);
    int s0, s1;
    k_slice(ns, ks, KS, s0, s1);
    tile_dot_t16<T>(wt, st, xrow, xvalid, q, s0, s1, acc);
  } else {
    const uint8_t* wp[T];
    const uint8_t* sp[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int row = min(n0 + 16 * t + c, N - 1);
      wp[t] = packed + (int64_t)row * (K / 2);
      sp[t] = scale + (int64_t)row * (K / 32);
    }
    tile_dot_raw<T>(wp, sp, xrow, xvalid, q, ns * ks / KS, ns * (ks + 1) / KS, acc);
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
      const int mi = m0 + 4 * q + r;
      if (mi < M && n < N) y[(int64_t)mi * N + n] = f32_bf16(v[r]);
    }
  }
}

constexpr int kGuT = 4, kGuKS = 4;   // gate/up: 32 z outputs per workgroup
constexpr int kDnT = 2, kDnKS = 2;   // down: 32 hidden rows per workgroup, K in two halves

template <int T, int KS, bool TILED>
static void launch_linear(const uint16_t* x, const uint8_t* packed, const uint8_t* scale, uint16_t* y, int64_t m,
                          int64_t n, int64_t k, hipStream_t st) {
  dim3 grid((unsigned)((n + 16 * T - 1) / (16 * T)), (unsigned)((m + 15) / 16));
  MOSAIC_LAUNCH((mx_linear_a16_kernel<T, KS, TILED>), grid, dim3(KS * 64), 0, st, x, packed, scale, y, (int)m,
                     (int)n, (int)k);
}

template <bool TILED>
static void dispatch_linear(const uint16_t* x, const uint8_t* packed, const uint8_t* scale, uint16_t* y, int64_t m,
                            int64_t n, int64_t k, hipStream_t st) {
  // enough waves to cover the chip: wide N takes more column tiles per wave
  const int64_t mt = (m + 15) / 16;
  if (((n + 63) / 64) * mt * 8 >= 4096)
    launch_linear<4, 8, TILED>(x, packed, scale, y, m, n, k, st);
  else if (((n + 31) / 32) * mt * 8 >= 4096)
    launch_linear<2, 8, TILED>(x, packed, scale, y, m, n, k, st);
  else
    launch_linear<1, 8, TILED>(x, packed, scale, y, m, n, k, st);
}

}  // namespace mosaic

using namespace mosaic;

extern "C" int mosaic_mx_linear_a16(const uint16_t* x, const uint8_t* packed, const uint8_t* scale, uint16_t* y,
                                    int64_t m, int64_t n, int64_t k, void* stream) {
  MOSAIC_CHECK_ARG(x && packed && scale && y, "mx_linear_a16: null pointer");
  MOSAIC_CHECK_ARG(k > 0 && k % 128 == 0, "mx_linear_a16: K=%lld must be a positive multiple of 128", (long long)k);
  MOSAIC_CHECK_ARG(m >= 0 && n >= 0 && m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 31),
                   "mx_linear_a16: shape out of range");
  if (m == 0 || n == 0) return kOk;
  dispatch_linear<false>(x, packed, scale, y, m, n, k, (hipStream_t)stream);
  MOSAIC_RETURN_LAUNCH("mx_linear_a16");
}

extern "C" int mosaic_mxt16_linear_a16(const uint16_t* x, const uint8_t* packed_t, const uint8_t* scale_t,
                                       uint16_t* y, int64_t m, int64_t n, int64_t k, void* stream) {
  MOSAIC_CHECK_ARG(x && packed_t && scale_t && y, "mxt16_linear_a16: null pointer");
  MOSAIC_CHECK_ARG(k > 0 && k % 128 == 0, "mxt16_linear_a16: K=%lld must be a positive multiple of 128",
                   (long long)k);
  MOSAIC_CHECK_ARG(n > 0 && n % 16 == 0, "mxt16_linear_a16: N=%lld must be a positive multiple of 16", (long long)n);
  MOSAIC_CHECK_ARG(m >= 0 && m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 31),
                   "mxt16_linear_a16: shape out of range");
  if (m == 0) return kOk;
  if (linear_decode1_supported(m, n, k))
    launch_linear_decode1(x, packed_t, scale_t, y, n, k, (hipStream_t)stream);
  else
    dispatch_linear<true>(x, packed_t, scale_t, y, m, n, k, (hipStream_t)stream);
  MOSAIC_RETURN_LAUNCH("mxt16_linear_a16");
}

extern "C" size_t mosaic_moe_a16_workspace_bytes(int64_t m, int64_t hidden, int64_t inter, int64_t n_experts,
                                                 int64_t top_k, int has_shared) {
  return carve_moe_workspace(nullptr, m, hidden, inter, n_experts, top_k, has_shared, kMoeBlockM, false).bytes;
}

extern "C" int mosaic_moe_a16_forward(const uint16_t* x, const float* logits, int32_t* ids, float* weights,
                                      const uint8_t* gu_packed, const uint8_t* gu_scale, const uint8_t* d_packed,
                                      const uint8_t* d_scale, const uint8_t* sh_gu_packed,
                                      const uint8_t* sh_gu_scale, const uint8_t* sh_d_packed,
                                      const uint8_t* sh_d_scale, uint16_t* y, int64_t m, int64_t hidden,
                                      int64_t inter, int64_t n_experts, int64_t top_k, int score_func, int renorm,
                                      float route_scale, const float* route_bias, float swiglu_limit,
                                      void* workspace, size_t workspace_bytes, void* const* stage_events,
                                      void* stream) {
  MOSAIC_CHECK_ARG(x && ids && weights && gu_packed && gu_scale && d_packed && d_scale && y && workspace,
                   "moe_a16_forward: null pointer");
  const int has_shared = sh_gu_packed != nullptr;
  MOSAIC_CHECK_ARG(!has_shared || (sh_gu_scale && sh_d_packed && sh_d_scale),
                   "moe_a16_forward: shared expert needs all four tensors");
  MOSAIC_CHECK_ARG(hidden > 0 && hidden % 128 == 0, "moe_a16_forward: hidden=%lld must be a multiple of 128",
                   (long long)hidden);
  MOSAIC_CHECK_ARG(inter > 0 && inter % 128 == 0, "moe_a16_forward: inter=%lld must be a multiple of 128",
                   (long long)inter);
  MOSAIC_CHECK_ARG(m >= 1, "moe_a16_forward: m=%lld", (long long)m);
  MoeWorkspace w =
      carve_moe_workspace((char*)workspace, m, hidden, inter, n_experts, top_k, has_shared, kMoeBlockM, false);
  MOSAIC_CHECK_ARG(workspace_bytes >= w.bytes, "moe_a16_forward: workspace %zu < %zu bytes", workspace_bytes,
                   w.bytes);
  hipStream_t st = (hipStream_t)stream;
  auto mark = [&](int i) {
    if (stage_events && stage_events[i]) (void)hipEventRecord((hipEvent_t)stage_events[i], st);
  };
  mark(0);
  if (moe_decode1_supported(m, hidden, inter, top_k, has_shared))
    return launch_moe_decode1(x, logits, route_bias, ids, weights, ids, weights, gu_packed, gu_scale, d_packed,
                              d_scale, sh_gu_packed, sh_gu_scale, sh_d_packed, sh_d_scale, y, hidden, inter, n_experts,
                              top_k, has_shared, score_func, renorm, route_scale, swiglu_limit, w.z, w.tile_expert,
                              w.n_tiles, stage_events, st);
  if (logits && m <= kSmallGuTokens && moe_small_down_supported(m, hidden, inter, w.tile_cap)) {
    // 2..4 tokens routed here: routing and the layout run inside the gate/up
    // launch, the combine inside the down launch (two launches in all).  The
    // picks of one token are distinct experts, so a tile has at most one row
    // per token, as the down kernel assumes.
    MOSAIC_CHECK_ARG(n_experts >= 1 && n_experts <= kRouteMaxExperts, "moe_a16_forward: E=%lld (1..%d)",
                     (long long)n_experts, kRouteMaxExperts);
    MOSAIC_CHECK_ARG(top_k >= 1 && top_k <= kRouteMaxTopK && top_k <= n_experts,
                     "moe_a16_forward: top_k=%lld (max %d, <= E)", (long long)top_k, kRouteMaxTopK);
    MOSAIC_CHECK_ARG(score_func >= 0 && score_func <= 2, "moe_a16_forward: score func %d", score_func);
    mark(1);  // no layout stage: routing is part of gate/up
    // rows of workgroups: at most one per tile, and few enough for the grid to be resident
    const int64_t cols = inter / (8 * kGuT);
    const int64_t rows = std::max<int64_t>(1, std::min<int64_t>(m * top_k + has_shared, kSmallGuResidentWgs / cols));
    MOSAIC_LAUNCH((moe_small_gateup_kernel<kGuT, kGuKS>), dim3((unsigned)cols, (unsigned)rows), dim3(kGuKS * 64), 0,
                       st, x, logits, route_bias, ids, weights, gu_packed, gu_scale, sh_gu_packed, sh_gu_scale,
                       w.tile_expert, w.tile_rows, w.tile_p0, w.n_tiles, w.perm_token, w.perm_weight, w.z, (int)m,
                       (int)hidden, (int)inter, (int)n_experts, (int)top_k, has_shared, score_func, renorm,
                       route_scale, swiglu_limit);
    MOSAIC_LAUNCH_CHECK("moe_small_gateup");
    mark(2);
    launch_moe_small_down(w.z, w.tile_expert, w.tile_rows, w.tile_p0, w.n_tiles, w.perm_token, d_packed, d_scale,
                          sh_d_packed, sh_d_scale, y, m, hidden, inter, n_experts, has_shared, st);
    MOSAIC_LAUNCH_CHECK("moe_small_down");
    mark(3);
    mark(4);  // the combine is fused into the down kernel
    return kOk;
  }
  // counts/offsets are not read by the MoE kernels, so small decode batches may
  // take the single-wave layout path
  LayoutOut lo{w.counts, w.offsets, w.perm, w.perm_token, w.perm_weight, w.sorted_ids, w.inv_pos,
               w.combine_pos, w.tile_expert, w.tile_start, w.tile_rows, w.tile_p0, w.n_tiles, nullptr, 0, 1,
               w.chunk_counts, w.chunk_base};
  int rc = launch_route_layout(logits, route_bias, ids, weights, ids, weights, m, n_experts, top_k, score_func,
                               renorm, route_scale, has_shared, kMoeBlockM, w.tile_cap, lo, st);
  if (rc != 0) return rc;
  mark(1);
  const unsigned tcap = (unsigned)w.tile_cap;
  MOSAIC_LAUNCH((moe_a16_gateup_kernel<kGuT, kGuKS>), dim3((unsigned)(inter / (8 * kGuT)), tcap),
                     dim3(kGuKS * 64), 0, st, x, gu_packed, gu_scale, sh_gu_packed, sh_gu_scale, w.tile_expert,
                     w.tile_rows, w.tile_p0, w.n_tiles, w.perm_token, w.perm_weight, w.z, (int)hidden, (int)inter,
                     (int)n_experts, swiglu_limit);
  MOSAIC_LAUNCH_CHECK("moe_a16_gateup");
  mark(2);
  MOSAIC_LAUNCH((moe_a16_down_kernel<kDnT, kDnKS>), dim3((unsigned)(hidden / (16 * kDnT)), tcap),
                     dim3(kDnKS * 64), 0, st, w.z, d_packed, d_scale, sh_d_packed, sh_d_scale, w.tile_expert,
                     w.tile_rows, w.tile_p0, w.n_tiles, w.yp, (int)hidden, (int)inter, (int)n_experts);
  MOSAIC_LAUNCH_CHECK("moe_a16_down");
  mark(3);
  MOSAIC_LAUNCH(moe_combine_kernel, dim3((unsigned)((hidden + 255) / 256), (unsigned)m), dim3(256), 0, st,
                     w.yp, w.combine_pos, y, (int)m, (int)(top_k + has_shared), (int)hidden);
  MOSAIC_LAUNCH_CHECK("moe_combine");
  mark(4);
  return kOk;
}
