// Router top-k (A10), stable expert sort (A11) and uncapped tile list (A12).
//
// One 1024-thread workgroup does all three for up to kRouteMaxAssign
// assignments: routing writes ids/weights, then every assignment gets its
// stable position inside its expert segment (ascending flat index), then the
// tile list (expert, m_start, rows) is emitted in ascending expert order.
// Everything stays on the device; nothing is read back by the host.
#include "common.h"
#include "moe_internal.h"
#include "route_token.h"
#include "../../include/mosaic_amd.h"

namespace mosaic {

static_assert(kCombineMaxW == kRouteMaxTopK + 1, "combine width covers top_k + shared");

constexpr int kRouteThreads = 1024;
constexpr int kRouteWaves = kRouteThreads / 64;
constexpr int kRouteMaxAssign = 4096;   // A_ext limit of the single-workgroup path

// Flat assignment a < M*K is (token a/K, slot a%K); a >= M*K is the shared
// expert's row for token a - M*K (virtual expert id E, weight 1).
__global__ void __launch_bounds__(kRouteThreads) route_layout_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias, const int32_t* ids_in,
    const float* weights_in, int32_t* ids_out, float* weights_out, int M, int E, int K, int func, int renorm,
    float route_scale, int has_shared, int block_m, int tile_cap, LayoutOut out) {
  __shared__ int16_t s_ids[kRouteMaxAssign];
  __shared__ float s_w[kRouteMaxAssign];
  __shared__ int32_t s_cnt[kRouteMaxExperts + 2];
  __shared__ int32_t s_off[kRouteMaxExperts + 2];
  __shared__ int32_t s_run[kRouteMaxExperts + 2];
  __shared__ int16_t s_tab[kRouteWaves][kRouteMaxExperts + 2];
  __shared__ int32_t s_toff[kRouteMaxExperts + 2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int A = M * K;
  const int A_ext = A + (has_shared ? M : 0);
  const int E_ext = E + (has_shared ? 1 : 0);
  const int W = K + (has_shared ? 1 : 0);

  for (int i = tid; i < out.n_counters; i += kRouteThreads) out.counters[i] = 0;
  // 1. routing (one wave per token) into s_ids/s_w, or read the given ids
  if (logits) {
    for (int t = wave; t < M; t += kRouteWaves)
      route_one_token(logits + (int64_t)t * E, E, K, func, renorm, route_scale, bias, s_ids + t * K, s_w + t * K,
                      ids_out + (int64_t)t * K, weights_out + (int64_t)t * K);
  } else {
    for (int a = tid; a < A; a += kRouteThreads) {
      int e = ids_in[a];
      s_ids[a] = (int16_t)((e < 0 || e >= E) ? -1 : e);
      s_w[a] = weights_in[a];
    }
  }
  for (int a = A + tid; a < A_ext; a += kRouteThreads) {
    s_ids[a] = (int16_t)E;
    s_w[a] = 1.0f;
  }
  for (int e = tid; e < E_ext; e += kRouteThreads) { s_cnt[e] = 0; s_run[e] = 0; }
  __syncthreads();
  // 2. counts (integer atomics: order-independent)
  for (int a = tid; a < A_ext; a += kRouteThreads) {
    int e = s_ids[a];
    if (e >= 0) atomicAdd(&s_cnt[e], 1);
  }
  __syncthreads();
  // 3. exclusive scans of counts and of tile counts (wave 0, DPP scans over 64-lane chunks)
  if (wave == 0) {
    uint32_t carry = 0, tcarry = 0;
    for (int base = 0; base < E_ext; base += 64) {
      const int e = base + lane;
      const uint32_t c = (e < E_ext) ? (uint32_t)s_cnt[e] : 0u;
      const uint32_t tc = (c + block_m - 1) / block_m;
      const uint32_t inc = wave_incl_scan_u32(c), tinc = wave_incl_scan_u32(tc);
      if (e < E_ext) { s_off[e] = (int)(carry + inc - c); s_toff[e] = (int)(tcarry + tinc - tc); }
      carry += wave_bcast_u32(inc, 63);
      tcarry += wave_bcast_u32(tinc, 63);
    }
    if (lane == 0) { s_off[E_ext] = (int)carry; s_toff[E_ext] = (int)tcarry; }
  }
  __syncthreads();
  // 4. stable positions: chunks of 1024 assignments in order; inside a wave the
  //    rank comes from an exact-match ballot mask, across waves from s_tab.
  int nbits = 1;
  while ((1 << nbits) <= E_ext) ++nbits;
  for (int base = 0; base < A_ext; base += kRouteThreads) {
    for (int e2 = tid; e2 < E_ext; e2 += kRouteThreads)
#pragma unroll
      for (int w = 0; w < kRouteWaves; ++w) s_tab[w][e2] = 0;
    __syncthreads();
    const int a = base + tid;
    const bool live = a < A_ext && s_ids[a] >= 0;
    const int e = live ? s_ids[a] : 0;
    uint64_t mask = __ballot(live);
    for (int b = 0; b < nbits; ++b) {
      uint64_t bb = __ballot(live && ((e >> b) & 1));
      mask &= ((e >> b) & 1) ? bb : ~bb;
    }
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const int rank_w = __popcll(mask & lt);
    if (live && rank_w == 0) s_tab[wave][e] = (int16_t)__popcll(mask);
    __syncthreads();
    if (a < A_ext) {
      // slot of this assignment in its token's ascending-expert list
      const int t = a < A ? a / K : a - A;
      int rank;
      if (a >= A) {
        rank = K;
      } else {
        const int s = a - t * K;
        const int my = s_ids[a];
        int nvalid = 0, below = 0, inv_before = 0;
        for (int s2 = 0; s2 < K; ++s2) {
          const int o = s_ids[t * K + s2];
          nvalid += (o >= 0);
          below += (o >= 0 && my >= 0 && (o < my || (o == my && s2 < s)));  // repeated ids: slot order
          inv_before += (o < 0 && s2 < s);
        }
        rank = my >= 0 ? below : nvalid + inv_before;
      }
      int p = -1;
      if (live) {
        int before = s_run[e];
        for (int w = 0; w < wave; ++w) before += s_tab[w][e];
        p = s_off[e] + before + rank_w;
        out.perm[p] = a;
        out.sorted_ids[p] = e;
        out.perm_token[p] = t;
        out.perm_weight[p] = s_w[a];
      }
      out.inv_pos[a] = p;
      out.combine_pos[(int64_t)t * W + rank] = p;
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
        out.tile_p0[slot] = s_off[e] + t * block_m;
      }
    }
  }
  if (tid == 0) {
    out.offsets[E_ext] = s_off[E_ext];
    out.n_tiles[0] = min(s_toff[E_ext], tile_cap);
  }
}

// Routing only: one wave per token (4 tokens per 256-thread block).
__global__ void __launch_bounds__(256) route_topk_kernel(const float* __restrict__ logits,
                                                         const float* __restrict__ bias, int32_t* ids, float* w,
                                                         int M, int E, int K, int func, int renorm,
                                                         float route_scale) {
  __shared__ int16_t s_i[4][kRouteMaxTopK];
  __shared__ float s_w[4][kRouteMaxTopK];
  const int wave = threadIdx.x >> 6;
  const int t = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  if (t >= M) return;
  route_one_token(logits + (int64_t)t * E, E, K, func, renorm, route_scale, bias, s_i[wave], s_w[wave],
                  ids + (int64_t)t * K, w + (int64_t)t * K);
}

// Tile list from expert counts (emit_tiles contract, no per-expert cap).
__global__ void __launch_bounds__(1024) emit_tiles_kernel(const int32_t* __restrict__ counts, int E, int block_m,
                                                          int32_t* tile_expert, int32_t* tile_start,
                                                          int32_t* tile_rows, int32_t* n_tiles, int tile_cap) {
  __shared__ int32_t s_toff[4097];
  const int tid = threadIdx.x, lane = tid & 63;
  if (tid < 64) {
    uint32_t carry = 0;
    for (int base = 0; base < E; base += 64) {
      const int e = base + lane;
      const int c = (e < E) ? counts[e] : 0;
      const uint32_t tc = c > 0 ? (uint32_t)((c + block_m - 1) / block_m) : 0u;
      const uint32_t inc = wave_incl_scan_u32(tc);
      if (e < E) s_toff[e] = (int)(carry + inc - tc);
      carry += wave_bcast_u32(inc, 63);
    }
    if (lane == 0) s_toff[E] = (int)carry;
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
  // the true total, as the reference returns tile_offsets[-1:]; entries past tile_cap are not written
  if (tid == 0) n_tiles[0] = s_toff[E];
}

// Small-batch fast path for the MoE forward (A_ext <= 256, M <= 16): one
// wave per token routes (all tokens at once), then four waves lay out every
// assignment (lane a = flat assignment a) by the same rule as
// route_layout_kernel: in-wave exact-match ballot ranks, per-wave counts for
// the ranks across waves, one scan of the expert counts.  Three barriers in
// all.  Writes what the MoE kernels read (perm / perm_token / perm_weight /
// sorted_ids / inv_pos / combine_pos / tile list); counts and offsets are left
// untouched.
constexpr int kSmallAssign = 256;
constexpr int kSmallTokens = 16;
__global__ void __launch_bounds__(1024) route_layout_small_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias, const int32_t* ids_in,
    const float* weights_in, int32_t* ids_out, float* weights_out, int M, int E, int K, int func, int renorm,
    float route_scale, int has_shared, int block_m, LayoutOut out) {
  __shared__ int16_t s_ids[kSmallAssign];
  __shared__ float s_w[kSmallAssign];
  __shared__ int32_t s_cnt[kRouteMaxExperts + 2];
  __shared__ int32_t s_off[kRouteMaxExperts + 2];
  __shared__ int32_t s_toff[kRouteMaxExperts + 2];
  __shared__ int16_t s_wc[4][kRouteMaxExperts + 2];  // per layout wave: its assignments of each expert
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nthr = blockDim.x;
  const int A = M * K;
  const int A_ext = A + (has_shared ? M : 0);
  const int E_ext = E + (has_shared ? 1 : 0);
  const int W = K + (has_shared ? 1 : 0);
  for (int i = tid; i < out.n_counters; i += nthr) out.counters[i] = 0;
  // 1. routing (wave t routes token t) or the given ids
  if (logits) {
    if (wave < M)
      route_one_token(logits + (int64_t)wave * E, E, K, func, renorm, route_scale, bias, s_ids + wave * K,
                      s_w + wave * K, ids_out + (int64_t)wave * K, weights_out + (int64_t)wave * K);
  } else {
    for (int a = tid; a < A; a += nthr) {
      const int e = ids_in[a];
      s_ids[a] = (int16_t)((e < 0 || e >= E) ? -1 : e);
      s_w[a] = weights_in[a];
    }
  }
  for (int a = A + tid; a < A_ext; a += nthr) {
    s_ids[a] = (int16_t)E;
    s_w[a] = 1.0f;
  }
  for (int e = tid; e < E_ext; e += nthr) {
    s_cnt[e] = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) s_wc[w][e] = 0;
  }
  __syncthreads();
  // 2. waves 0..3: in-wave ranks (exact-match ballots on the id bits) and counts
  int nbits = 1;
  while ((1 << nbits) <= E_ext) ++nbits;
  const int a = tid;
  const bool in = wave < 4 && a < A_ext;
  const int e = in ? s_ids[a] : -1;
  const bool live = e >= 0;
  int rank_w = 0;
  if (wave < 4) {
    uint64_t mask = __ballot(live);
    for (int b = 0; b < nbits; ++b) {
      const uint64_t bb = __ballot(live && ((e >> b) & 1));
      mask &= ((e >> b) & 1) ? bb : ~bb;
    }
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    rank_w = __popcll(mask & lt);
    if (live && rank_w == 0) {
      s_wc[wave][e] = (int16_t)__popcll(mask);
      atomicAdd(&s_cnt[e], (int)__popcll(mask));
    }
  }
  __syncthreads();
  // 3. exclusive scans of the counts and of the tile counts (wave 0)
  if (wave == 0) {
    uint32_t carry = 0, tcarry = 0;
    for (int base = 0; base < E_ext; base += 64) {
      const int x = base + lane;
      const uint32_t c = (x < E_ext) ? (uint32_t)s_cnt[x] : 0u;
      const uint32_t tc = (c + block_m - 1) / block_m;
      const uint32_t inc = wave_incl_scan_u32(c), tinc = wave_incl_scan_u32(tc);
      if (x < E_ext) {
        s_off[x] = (int)(carry + inc - c);
        s_toff[x] = (int)(tcarry + tinc - tc);
      }
      carry += wave_bcast_u32(inc, 63);
      tcarry += wave_bcast_u32(tinc, 63);
    }
    if (lane == 0) s_toff[E_ext] = (int)tcarry;
  }
  __syncthreads();
  // 4. place every assignment; the first of each expert emits the expert's tiles
  if (in) {
    const int t = a < A ? a / K : a - A;
    int rank;
    if (a >= A) {
      rank = K;
    } else {
      const int sl = a - t * K;
      int nvalid = 0, below = 0, inv_before = 0;
      for (int s2 = 0; s2 < K; ++s2) {
        const int o = s_ids[t * K + s2];
        nvalid += (o >= 0);
        below += (o >= 0 && live && (o < e || (o == e && s2 < sl)));  // repeated ids: slot order
        inv_before += (o < 0 && s2 < sl);
      }
      rank = live ? below : nvalid + inv_before;
    }
    int p = -1;
    if (live) {
      int before = 0;
      for (int w = 0; w < wave; ++w) before += s_wc[w][e];
      p = s_off[e] + before + rank_w;
      out.perm[p] = a;
      out.sorted_ids[p] = e;
      out.perm_token[p] = t;
      out.perm_weight[p] = s_w[a];
      if (p == s_off[e]) {
        const int cnt = s_cnt[e];
        for (int j = 0; j * block_m < cnt; ++j) {
          const int slot = s_toff[e] + j;
          out.tile_expert[slot] = e;
          out.tile_start[slot] = j * block_m;
          out.tile_rows[slot] = min(block_m, cnt - j * block_m);
          out.tile_p0[slot] = s_off[e] + j * block_m;
        }
      }
    }
    out.inv_pos[a] = p;
    out.combine_pos[(int64_t)t * W + rank] = p;
  }
  if (tid == 0) out.n_tiles[0] = s_toff[E_ext];
}

// ------------------------------------------------ multi-workgroup layout ----
// For more than kRouteMaxAssign assignments: chunks of kLayoutChunk flat
// assignments (tokens' slots in order, then the shared-expert rows) are
// counted per expert (one workgroup per chunk), one workgroup turns the counts
// into expert offsets, per-(chunk, expert) bases and the tile list, and a
// second pass over the chunks places every assignment at base + its rank
// among the same expert's assignments earlier in the chunk: the same stable
// order as the single-workgroup kernel.
__device__ __forceinline__ int assignment_expert(const int32_t* ids, int a, int A, int A_ext, int E) {
  if (a >= A_ext) return -1;
  if (a >= A) return E;
  const int e = ids[a];
  return (e < 0 || e >= E) ? -1 : e;
}

__global__ void __launch_bounds__(kLayoutChunk) layout_count_kernel(const int32_t* __restrict__ ids, int A, int A_ext,
                                                                    int E, int E_ext, int32_t* chunk_counts,
                                                                    int32_t* counters, int n_counters) {
  __shared__ int32_t cnt[kRouteMaxExperts + 2];
  const int tid = threadIdx.x, ch = blockIdx.x;
  for (int e = tid; e < E_ext; e += kLayoutChunk) cnt[e] = 0;
  if (ch == 0)
    for (int i = tid; i < n_counters; i += kLayoutChunk) counters[i] = 0;
  __syncthreads();
  const int e = assignment_expert(ids, ch * kLayoutChunk + tid, A, A_ext, E);
  if (e >= 0) atomicAdd(&cnt[e], 1);
  __syncthreads();
  for (int x = tid; x < E_ext; x += kLayoutChunk) chunk_counts[(int64_t)ch * E_ext + x] = cnt[x];
}

constexpr int kScanTile = 32768;  // chunk counts (ints) the scan stages in LDS at a time: 128 KB

__global__ void __launch_bounds__(1024) layout_scan_kernel(const int32_t* __restrict__ chunk_counts, int n_chunks,
                                                           int E_ext, int block_m, int tile_cap, LayoutOut out) {
  // The [chunk][expert] counts are staged through LDS in tiles of whole chunks with coalesced loads;
  // each expert's walk over the chunks then runs on LDS. A table that fits one tile stays resident
  // between the totals pass and the bases pass.
  __shared__ int32_t s_tile[kScanTile];
  __shared__ int32_t s_cnt[kRouteMaxExperts + 2];
  __shared__ int32_t s_off[kRouteMaxExperts + 2];
  __shared__ int32_t s_toff[kRouteMaxExperts + 2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int cb = kScanTile / E_ext;  // whole chunks per tile (>= 63)
  const bool resident = n_chunks <= cb;
  int tot = 0;
  for (int c0 = 0; c0 < n_chunks; c0 += cb) {
    const int nc = min(cb, n_chunks - c0), n = nc * E_ext;
    const int32_t* src = chunk_counts + (int64_t)c0 * E_ext;
#pragma unroll 8
    for (int i = tid; i < n; i += 1024) s_tile[i] = src[i];
    __syncthreads();
    if (tid < E_ext) {
#pragma unroll 8
      for (int c = 0; c < nc; ++c) tot += s_tile[c * E_ext + tid];
    }
    __syncthreads();
  }
  if (tid < E_ext) s_cnt[tid] = tot;
  __syncthreads();
  if (wave == 0) {
    uint32_t carry = 0, tcarry = 0;
    for (int base = 0; base < E_ext; base += 64) {
      const int e = base + lane;
      const uint32_t c = (e < E_ext) ? (uint32_t)s_cnt[e] : 0u;
      const uint32_t tc = (c + block_m - 1) / block_m;
      const uint32_t inc = wave_incl_scan_u32(c), tinc = wave_incl_scan_u32(tc);
      if (e < E_ext) {
        s_off[e] = (int)(carry + inc - c);
        s_toff[e] = (int)(tcarry + tinc - tc);
      }
      carry += wave_bcast_u32(inc, 63);
      tcarry += wave_bcast_u32(tinc, 63);
    }
    if (lane == 0) {
      s_off[E_ext] = (int)carry;
      s_toff[E_ext] = (int)tcarry;
    }
  }
  __syncthreads();
  // Bases: each expert's running offset replaces its counts in the staged tile, which is then
  // stored whole.
  int run = tid < E_ext ? s_off[tid] : 0;
  for (int c0 = 0; c0 < n_chunks; c0 += cb) {
    const int nc = min(cb, n_chunks - c0), n = nc * E_ext;
    if (!resident) {
      const int32_t* src = chunk_counts + (int64_t)c0 * E_ext;
#pragma unroll 8
      for (int i = tid; i < n; i += 1024) s_tile[i] = src[i];
      __syncthreads();
    }
    if (tid < E_ext) {
#pragma unroll 8
      for (int c = 0; c < nc; ++c) {
        const int v = s_tile[c * E_ext + tid];
        s_tile[c * E_ext + tid] = run;
        run += v;
      }
    }
    __syncthreads();
    int32_t* dst = out.chunk_base + (int64_t)c0 * E_ext;
#pragma unroll 8
    for (int i = tid; i < n; i += 1024) dst[i] = s_tile[i];
    __syncthreads();
  }
  for (int e = tid; e < E_ext; e += 1024) {
    out.counts[e] = s_cnt[e];
    out.offsets[e] = s_off[e];
    const int nt = (s_cnt[e] + block_m - 1) / block_m;
    for (int t = 0; t < nt; ++t) {
      const int slot = s_toff[e] + t;
      if (slot < tile_cap) {
        out.tile_expert[slot] = e;
        out.tile_start[slot] = t * block_m;
        out.tile_rows[slot] = min(block_m, s_cnt[e] - t * block_m);
        out.tile_p0[slot] = s_off[e] + t * block_m;
      }
    }
  }
  if (tid == 0) {
    out.offsets[E_ext] = s_off[E_ext];
    out.n_tiles[0] = min(s_toff[E_ext], tile_cap);
  }
}

__global__ void __launch_bounds__(kLayoutChunk) layout_scatter_kernel(const int32_t* __restrict__ ids,
                                                                      const float* __restrict__ weights, int A,
                                                                      int A_ext, int E, int E_ext, int K, int W,
                                                                      LayoutOut out) {
  constexpr int NW = kLayoutChunk / 64;
  __shared__ int16_t s_tab[NW][kRouteMaxExperts + 2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, ch = blockIdx.x;
  for (int e2 = tid; e2 < E_ext; e2 += kLayoutChunk)
#pragma unroll
    for (int w = 0; w < NW; ++w) s_tab[w][e2] = 0;
  __syncthreads();
  const int a = ch * kLayoutChunk + tid;
  const int my = assignment_expert(ids, a, A, A_ext, E);
  const bool live = my >= 0;
  const int e = live ? my : 0;
  int nbits = 1;
  while ((1 << nbits) <= E_ext) ++nbits;
  uint64_t mask = __ballot(live);
  for (int b = 0; b < nbits; ++b) {
    const uint64_t bb = __ballot(live && ((e >> b) & 1));
    mask &= ((e >> b) & 1) ? bb : ~bb;
  }
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int rank_w = __popcll(mask & lt);
  if (live && rank_w == 0) s_tab[wave][e] = (int16_t)__popcll(mask);
  __syncthreads();
  if (a >= A_ext) return;
  const int t = a < A ? a / K : a - A;
  int rank;
  if (a >= A) {
    rank = K;
  } else {
    const int s = a - t * K;
    int nvalid = 0, below = 0, inv_before = 0;
    for (int s2 = 0; s2 < K; ++s2) {
      const int o = assignment_expert(ids, t * K + s2, A, A_ext, E);
      nvalid += (o >= 0);
      below += (o >= 0 && my >= 0 && (o < my || (o == my && s2 < s)));  // repeated ids: slot order
      inv_before += (o < 0 && s2 < s);
    }
    rank = my >= 0 ? below : nvalid + inv_before;
  }
  int p = -1;
  if (live) {
    int before = 0;
    for (int w = 0; w < wave; ++w) before += s_tab[w][e];
    p = out.chunk_base[(int64_t)ch * E_ext + e] + before + rank_w;
    out.perm[p] = a;
    out.sorted_ids[p] = e;
    out.perm_token[p] = t;
    out.perm_weight[p] = a < A ? weights[a] : 1.0f;
  }
  out.inv_pos[a] = p;
  out.combine_pos[(int64_t)t * W + rank] = p;
}

int launch_route_layout(const float* logits, const float* bias, const int32_t* ids_in, const float* weights_in,
                        int32_t* ids_out, float* weights_out, int64_t M, int64_t E, int64_t K, int func, int renorm,
                        float route_scale, int has_shared, int block_m, int64_t tile_cap, const LayoutOut& out,
                        hipStream_t st) {
  const int64_t A_ext = M * K + (has_shared ? M : 0);
  MOSAIC_CHECK_ARG(M >= 1 && E >= 1 && K >= 1, "moe layout: M=%lld E=%lld K=%lld", (long long)M, (long long)E,
                   (long long)K);
  MOSAIC_CHECK_ARG(E <= kRouteMaxExperts, "moe layout: E=%lld exceeds %d", (long long)E, kRouteMaxExperts);
  MOSAIC_CHECK_ARG(K <= kRouteMaxTopK && K <= E, "moe layout: top_k=%lld (max %d, <= E)", (long long)K,
                   kRouteMaxTopK);
  MOSAIC_CHECK_ARG(A_ext < (1ll << 30), "moe layout: %lld assignments", (long long)A_ext);
  MOSAIC_CHECK_ARG(block_m >= 1, "moe layout: block_m=%d", block_m);
  MOSAIC_CHECK_ARG(func >= 0 && func <= 2, "moe layout: score func %d", func);
  MOSAIC_CHECK_ARG(logits ? (ids_out && weights_out) : (ids_in && weights_in), "moe layout: missing ids/weights");
  if (out.small_ok && A_ext <= kSmallAssign && M <= kSmallTokens) {
    const unsigned threads = logits ? 1024u : 256u;
    MOSAIC_LAUNCH(route_layout_small_kernel, dim3(1), dim3(threads), 0, st, logits, bias, ids_in, weights_in,
                       ids_out, weights_out, (int)M, (int)E, (int)K, func, renorm, route_scale, has_shared, block_m,
                       out);
    MOSAIC_RETURN_LAUNCH("moe_route_layout_small");
  }
  MOSAIC_CHECK_ARG(out.counts && out.offsets, "moe layout: counts/offsets required");
  if (A_ext > kRouteMaxAssign) {
    MOSAIC_CHECK_ARG(out.chunk_counts && out.chunk_base, "moe layout: %lld assignments need the layout scratch",
                     (long long)A_ext);
    const int E_ext = (int)E + (has_shared ? 1 : 0);
    const int A = (int)(M * K);
    const int nch = (int)layout_chunks(A_ext);
    const int32_t* ids = ids_in;
    const float* wts = weights_in;
    if (logits) {
      MOSAIC_LAUNCH(route_topk_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, st, logits, bias, ids_out,
                         weights_out, (int)M, (int)E, (int)K, func, renorm, route_scale);
      ids = ids_out;
      wts = weights_out;
    }
    MOSAIC_LAUNCH(layout_count_kernel, dim3((unsigned)nch), dim3(kLayoutChunk), 0, st, ids, A, (int)A_ext,
                       (int)E, E_ext, out.chunk_counts, out.counters, out.n_counters);
    MOSAIC_LAUNCH(layout_scan_kernel, dim3(1), dim3(1024), 0, st, out.chunk_counts, nch, E_ext, block_m,
                       (int)tile_cap, out);
    MOSAIC_LAUNCH(layout_scatter_kernel, dim3((unsigned)nch), dim3(kLayoutChunk), 0, st, ids, wts, A,
                       (int)A_ext, (int)E, E_ext, (int)K, (int)K + (has_shared ? 1 : 0), out);
    MOSAIC_RETURN_LAUNCH("moe_route_layout_multi");
  }
  MOSAIC_LAUNCH(route_layout_kernel, dim3(1), dim3(kRouteThreads), 0, st, logits, bias, ids_in, weights_in,
                     ids_out, weights_out, (int)M, (int)E, (int)K, func, renorm, route_scale, has_shared, block_m,
                     (int)tile_cap, out);
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
  MOSAIC_LAUNCH(route_topk_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, logits, bias, ids, weights,
                     (int)m, (int)e, (int)top_k, score_func, renorm, route_scale);
  MOSAIC_RETURN_LAUNCH("moe_route_topk");
}

extern "C" size_t mosaic_moe_layout_workspace_bytes(int64_t m, int64_t top_k, int64_t e, int has_shared) {
  if (m < 0 || top_k < 0 || e < 0) return 0;
  return layout_scratch_bytes(m * top_k + (has_shared ? m : 0), e + (has_shared ? 1 : 0));
}

extern "C" int mosaic_moe_layout(const int32_t* ids, const float* weights, int64_t m, int64_t top_k, int64_t e,
                                 int has_shared, int block_m, int32_t* counts, int32_t* offsets, int32_t* perm,
                                 int32_t* perm_token, float* perm_weight, int32_t* sorted_ids, int32_t* inv_pos,
                                 int32_t* combine_pos, int32_t* tile_expert, int32_t* tile_start, int32_t* tile_rows,
                                 int32_t* tile_p0, int32_t* n_tiles, int64_t tile_cap, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  MOSAIC_CHECK_ARG(ids && weights && counts && offsets && perm && perm_token && perm_weight && sorted_ids &&
                       inv_pos && combine_pos && tile_expert && tile_start && tile_rows && tile_p0 && n_tiles,
                   "moe_layout: null pointer");
  const size_t need = mosaic_moe_layout_workspace_bytes(m, top_k, e, has_shared);
  MOSAIC_CHECK_ARG(need == 0 || (workspace && workspace_bytes >= need), "moe_layout: workspace %zu bytes < %zu",
                   workspace_bytes, need);
  int32_t* cc = need ? (int32_t*)workspace : nullptr;
  int32_t* cb = need ? cc + need / 8 : nullptr;
  LayoutOut out{counts, offsets, perm, perm_token, perm_weight, sorted_ids, inv_pos, combine_pos,
                tile_expert, tile_start, tile_rows, tile_p0, n_tiles, nullptr, 0, 0, cc, cb};
  return launch_route_layout(nullptr, nullptr, ids, weights, nullptr, nullptr, m, e, top_k, 0, 0, 1.0f, has_shared,
                             block_m, tile_cap, out, (hipStream_t)stream);
}

extern "C" int mosaic_emit_tiles(const int32_t* counts, int64_t e, int block_m, int32_t* tile_expert,
                                 int32_t* tile_start, int32_t* tile_rows, int32_t* n_tiles, int64_t tile_cap,
                                 void* stream) {
  MOSAIC_CHECK_ARG(counts && tile_expert && tile_start && tile_rows && n_tiles, "emit_tiles: null pointer");
  MOSAIC_CHECK_ARG(e >= 1 && e <= 4096, "emit_tiles: E=%lld (1..4096)", (long long)e);
  MOSAIC_CHECK_ARG(block_m >= 1, "emit_tiles: block_m=%d", block_m);
  MOSAIC_CHECK_ARG(tile_cap >= 0 && tile_cap < (1ll << 31), "emit_tiles: tile_cap=%lld", (long long)tile_cap);
  MOSAIC_LAUNCH(emit_tiles_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, counts, (int)e, block_m,
                     tile_expert, tile_start, tile_rows, n_tiles, (int)tile_cap);
  MOSAIC_RETURN_LAUNCH("emit_tiles");
}
