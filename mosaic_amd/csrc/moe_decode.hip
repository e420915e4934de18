// Batch-1 decode MoE layer (A16 contract) in two launches.
//
// 1. moe_dec1_gateup_kernel: every workgroup of a routed tile routes the token
//    itself (route_token.h, the same arithmetic as the layout kernel, so ids
//    and weights are identical), sorts the picks by expert id and takes the
//    tile-th one; shared-expert workgroups skip routing.  A workgroup owns 16 z
//    columns of one tile (gate row group j and up row group I/16 + j); its KS
//    waves split K into equal parts and each wave streams its part through a
//    register ring of D super-steps (weights + scale dwords loaded D steps
//    ahead, no branches in the steady state), with the x part it needs staged
//    in wave-private LDS.  The parts meet in LDS; SwiGLU and the route weight
//    are applied and z row `tile` is written (the shared expert's row is K).
// 2. moe_dec1_down_kernel: a workgroup owns 16 (or 8) hidden columns and walks
//    every tile (the shared expert first, then the experts in ascending id);
//    its waves again split K (= inter) and stream (tile, super-step) entries
//    through a ring, with z staged in LDS.  Each expert's partial (a fresh
//    MFMA chain) is added to the running fp32 sum of the routed tiles in order,
//    and the shared partial after it, so the combine of the reference
//    (ascending expert id, shared last, fp32) happens in registers and y is
//    written directly: no partial buffer, no combine launch.
//
// Rows: the decode batch has one token, so the x / z operand is row 0 in every
// lane (all 16 MFMA rows carry the same data and only row 0 is stored).
#include <algorithm>

#include <hip/hip_ext.h>

#include "common.h"
#include "moe_internal.h"
#include "route_token.h"
#include "../../include/mosaic_amd.h"

namespace mosaic {

constexpr int kDecXVMax = 8;   // x vectors (16 B) per lane staged by a gate/up wave: part <= 32 super-steps
constexpr int kDecZVMax = 20;  // z vectors per lane staged by a down wave

__device__ __forceinline__ bf16x8_t dec_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

// MXT16 addresses of row group g for this lane: its 16 B code block of super-step 0
// and its scale dword of super-steps 0..3 (add S * 1024 and (S / 4) * 256)
__device__ __forceinline__ void dec_ptrs(const uint8_t* pt, const uint8_t* st, int64_t g, int ns, int lane,
                                         const uint8_t*& w, const uint8_t*& s) {
  const int ns4 = (ns + 3) / 4;
  w = pt + (g * ns * 64 + lane) * 16;
  s = st + (g * ns4 * 64 + lane) * 4;
}

// 16 B of E2M1 (one lane's MX block) x 32 bf16 of x at the same K -> acc
__device__ __forceinline__ void dec_mfma(const u32x4_t w, uint32_t sbyte, const u32x4_t (&xv)[4], f32x4_t& acc) {
  bf16x8_t wb[4];
  mx_block_to_bf16(w, e8m0_f32(sbyte), wb);
#pragma unroll
  for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(dec_bf16x8(xv[s]), wb[s], acc, 0, 0, 0);
}

// x operand of super-step s of a part staged at xs (row-major, 128 bf16 per step)
__device__ __forceinline__ void dec_x(const uint8_t* xs, int s, int q, u32x4_t (&xv)[4]) {
  const u32x4_t* p = reinterpret_cast<const u32x4_t*>(xs + s * 256 + q * 64);
#pragma unroll
  for (int k = 0; k < 4; ++k) xv[k] = p[k];
}

// Route the token in this wave (or read the given ids) and sort the picks by
// (expert id, slot), all in registers: lane i < K ends with pick i (rank order)
// in me/mw and its sorted position in rank; invalid picks (given ids out of
// range) have me = -1 and sort last.  Returns the number of valid picks.
__device__ __forceinline__ int dec1_route(const float* __restrict__ logits, const float* __restrict__ bias,
                                          const int32_t* __restrict__ ids_in, const float* __restrict__ w_in, int E,
                                          int K, int func, int renorm, float scale, int& me, float& mw, int& rank) {
  const int lane = threadIdx.x & 63;
  if (logits) {
    route_token_any(logits, E, K, func, renorm, scale, bias, me, mw);
  } else {
    const int e = lane < K ? ids_in[lane] : -1;
    me = (e < 0 || e >= E) ? -1 : e;
    mw = lane < K ? w_in[lane] : 0.f;
  }
  const int km = me >= 0 ? me : 0x7FFF;
  rank = 0;
  for (int jj = 0; jj < K; ++jj) {
    const int o = __builtin_amdgcn_readlane(me, jj);
    const int ko = o >= 0 ? o : 0x7FFF;
    rank += (ko < km || (ko == km && jj < lane)) ? 1 : 0;
  }
  return __builtin_popcountll(__ballot(lane < K && me >= 0));
}

// grid (I/16, K + has_shared), KS waves; dynamic LDS = H * 2 bytes (the x row, split in parts);
// XV >= the x vectors per lane of a part (nsp / 4)
template <int KS, int D, int XV>
__global__ void __launch_bounds__(KS * 64) moe_dec1_gateup_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ logits, const float* __restrict__ bias,
    const int32_t* __restrict__ ids_in, const float* __restrict__ w_in, int32_t* __restrict__ ids_out,
    float* __restrict__ w_out, const uint8_t* __restrict__ gu_p, const uint8_t* __restrict__ gu_s,
    const uint8_t* __restrict__ sh_p, const uint8_t* __restrict__ sh_s, uint16_t* __restrict__ z,
    int32_t* __restrict__ tile_expert, int32_t* __restrict__ n_tiles, int H, int I, int E, int K, int func,
    int renorm, float route_scale, float limit) {
  extern __shared__ __attribute__((aligned(16))) uint8_t dec_smem[];
  __shared__ float red[KS][2][16];
  __shared__ int s_tile_e;
  __shared__ float s_tile_w;
  const int tile = blockIdx.y;
  const bool is_shared = tile == K;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = lane & 15, q = lane >> 4;
  const int j = blockIdx.x;
  const int ns = H / 128, nsp = ns / KS, sbase = w * nsp, ns4 = (ns + 3) / 4;
  // 1. this wave's x part -> registers (clamped: every lane loads, lanes past the part do not store)
  const int nvec = nsp * 16;
  u32x4_t xst[XV];
#pragma unroll
  for (int v = 0; v < XV; ++v) {
    const int i = min(lane + 64 * v, nvec - 1);
    xst[v] = reinterpret_cast<const u32x4_t*>(x + (int64_t)sbase * 128)[i];
  }
  // 2. routing (routed tiles): wave 0 routes (one wave per workgroup, not
  //    per wave: the DPP rounds would otherwise compete for every SIMD) and
  //    publishes this tile's expert and route weight
  int e = E;
  float rw = 1.0f;
  if (!is_shared) {
    if (w == 0) {
      int me, rank;
      float mw;
      const int nv = dec1_route(logits, bias, ids_in, w_in, E, K, func, renorm, route_scale, me, mw, rank);
      if (blockIdx.x == 0 && tile == 0 && lane < K) {  // outputs + the tile list of the down kernel
        if (logits) {
          ids_out[lane] = me;
          w_out[lane] = mw;
        }
        if (me >= 0) tile_expert[rank] = me;
        if (lane == 0) n_tiles[0] = nv;
      }
      const uint64_t src = __ballot(lane < K && me >= 0 && rank == tile);
      const int sl = src ? __builtin_ctzll(src) : 0;
      const int te = __builtin_amdgcn_readlane(me, sl);
      const float tw = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(mw), sl));
      if (lane == 0) {
        s_tile_e = src ? te : -1;
        s_tile_w = tw;
      }
    }
    __syncthreads();
    e = s_tile_e;
    rw = s_tile_w;
    if (e < 0) return;  // tile >= valid picks (uniform over the workgroup)
  }
  const int64_t ebytes = (int64_t)2 * I * (H / 2), sbytes = (int64_t)(2 * I / 16) * ns4 * 256;
  const uint8_t* bp = is_shared ? sh_p : gu_p + (int64_t)e * ebytes;
  const uint8_t* bs = is_shared ? sh_s : gu_s + (int64_t)e * sbytes;
  const uint8_t* wt[2];
  const uint8_t* st[2];
  dec_ptrs(bp, bs, j, ns, lane, wt[0], st[0]);
  dec_ptrs(bp, bs, I / 16 + j, ns, lane, wt[1], st[1]);
  // 3. ring prologue: steps [0, D) of the part (padded steps past the part load step 0 and get scale 0)
  const int nchunks = (nsp + D - 1) / D;
  u32x4_t rw_w[D][2];
  uint32_t rw_s[D][2];
  auto load_step = [&](int n, u32x4_t (&wv)[2], uint32_t (&sv)[2]) {
    const int S = sbase + (n < nsp ? n : 0);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      wv[t] = load_nt_u32x4(wt[t] + (int64_t)S * 1024);
      sv[t] = *reinterpret_cast<const uint32_t*>(st[t] + (int64_t)(S >> 2) * 256);
    }
  };
#pragma unroll
  for (int s = 0; s < D; ++s) {
    load_step(s, rw_w[s], rw_s[s]);
    asm volatile("" ::: "memory");  // in step order: the compiler's waits count the later loads
  }
  // 4. x part -> wave-private LDS (the wave reads only what it wrote)
  uint8_t* xs = dec_smem + (size_t)w * nsp * 256;
#pragma unroll
  for (int v = 0; v < XV; ++v) {
    const int i = lane + 64 * v;
    if (i < nvec) reinterpret_cast<u32x4_t*>(xs)[i] = xst[v];
  }
  wave_lds_fence();
  f32x4_t acc[2] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
  auto chunk = [&](int ch, auto more) {
#pragma unroll
    for (int s = 0; s < D; ++s) {
      const int n = ch * D + s;
      const int S = sbase + n;
      const bool real = n < nsp;
      u32x4_t xv[4];
      dec_x(xs, real ? n : 0, q, xv);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        // the scale dword is read here, not hoisted to the chunk's start, where
        // its wait would drain every load in flight
        uint32_t sw = rw_s[s][t];
        asm volatile("" : "+v"(sw));
        const uint32_t sb = real ? (sw >> (8 * (S & 3))) & 0xFFu : 0u;  // padded step: scale 0 -> W = 0
        dec_mfma(rw_w[s][t], sb, xv, acc[t]);
      }
      if constexpr (decltype(more)::value) {
        load_step(n + D, rw_w[s], rw_s[s]);
        asm volatile("" ::: "memory");
      }
    }
  };
  for (int ch = 0; ch < nchunks - 1; ++ch) chunk(ch, std::true_type{});
  chunk(nchunks - 1, std::false_type{});
  // 5. parts meet in LDS (row 0 only: lanes 0..15, element 0)
  if (q == 0) {
    red[w][0][c] = acc[0][0];
    red[w][1][c] = acc[1][0];
  }
  __syncthreads();
  if (w == 0 && q == 0) {
    float g = red[0][0][c], u = red[0][1][c];
#pragma unroll
    for (int k2 = 1; k2 < KS; ++k2) {
      g += red[k2][0][c];
      u += red[k2][1][c];
    }
    const float zv = swiglu_f32(g, u, limit) * rw;
    z[(int64_t)tile * I + 16 * j + c] = f32_bf16(zv);
  }
}

// grid H / cpw, KS waves; dynamic LDS = (K + has_shared) * I * 2 bytes (the z
// rows, stored part by part).  A workgroup owns cpw = 16 or 8 consecutive
// hidden columns: 8 when H / 16 would leave CUs idle, which keeps every
// window on whole 128-byte lines (a line is 8 rows of one K quarter); lanes of
// rows past the window load its last row and are not stored.  Its waves take
// one K part each: a part is NSP super-steps (inter / 128 = KS * NSP, NSP <= 4,
// and the part starts at a multiple of NSP so its scale bytes sit in one
// dword); the ring holds DT expert tiles, each NSP code blocks + one scale dword.
template <int KS, int NSP, int DT, int ZV>
__global__ void __launch_bounds__(KS * 64) moe_dec1_down_kernel(
    const uint16_t* __restrict__ z, const int32_t* __restrict__ tile_expert, const int32_t* __restrict__ n_tiles,
    const uint8_t* __restrict__ d_p, const uint8_t* __restrict__ d_s, const uint8_t* __restrict__ sh_p,
    const uint8_t* __restrict__ sh_s, uint16_t* __restrict__ y, int H, int I, int E, int K, int has_shared,
    int cpw) {
  extern __shared__ __attribute__((aligned(16))) uint8_t dec_smem[];
  __shared__ float red[KS][16];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = lane & 15, q = lane >> 4;
  const int col0 = blockIdx.x * cpw;
  const int ns = I / 128, sbase = w * NSP, ns4 = (ns + 3) / 4;
  const int nz = K + has_shared;  // z rows (row K = shared expert)
  // 1. the tile list (scalar loads: they do not wait behind the vector loads
  //    below), then the workgroup's share of z -> registers: 16-byte vector i
  //    is part p, row r, vector o of the LDS layout [part][row][NSP * 16]
  const int nv = n_tiles[0];
  const int nt = nv + has_shared;
  const int pvec = NSP * 16, rvec = nz * pvec, nvec = KS * rvec;
  u32x4_t zst[ZV];
#pragma unroll
  for (int v = 0; v < ZV; ++v) {
    const int i = min((int)threadIdx.x + KS * 64 * v, nvec - 1);
    const int p = i / rvec, rem = i - p * rvec;
    const int r = rem / pvec, o = rem - r * pvec;
    zst[v] = reinterpret_cast<const u32x4_t*>(z + (int64_t)r * I + (int64_t)p * NSP * 128)[o];
  }
  // 2. this lane's weight row and its offsets inside an expert's down matrix
  const bool row_ok = c < cpw;
  const int row = col0 + (row_ok ? c : cpw - 1);
  const int gr = row >> 4, l = q * 16 + (row & 15);
  const uint32_t woff = (uint32_t)gr * ns * 1024u + (uint32_t)sbase * 1024u + (uint32_t)l * 16u;
  const uint32_t soff = (uint32_t)gr * ns4 * 256u + (uint32_t)(sbase >> 2) * 256u + (uint32_t)l * 4u;
  // 3. tiles: the shared expert first (its addresses need no tile list), then
  //    the routed ones in ascending expert id.  The shared partial is kept
  //    apart and added after the routed sum, so the fp32 combine order is
  //    ascending id, shared last.
  const int64_t ebytes = (int64_t)H * (I / 2), sbytes = (int64_t)(H / 16) * ns4 * 256;
  u32x4_t r_w[DT][NSP];
  uint32_t r_s[DT];
  // ring entry t >= has_shared is routed tile t - has_shared; padded entries
  // (t >= nt) read one fixed 1 KB block (cache hits, no HBM bytes) and get
  // scale 0 (selects only: the ring issues its loads without branches)
  auto load_tile = [&](int t, u32x4_t (&wt)[NSP], uint32_t& sv) {
    const uint8_t* wp;
    const uint8_t* sp;
    if (has_shared && t == 0) {
      wp = sh_p;
      sp = sh_s;
    } else {
      const int rt = t < nt ? t - has_shared : 0;
      const int e = nv > 0 ? tile_expert[rt] : 0;
      wp = d_p + (int64_t)e * ebytes;
      sp = d_s + (int64_t)e * sbytes;
    }
    const bool pad = t >= nt;
    const uint32_t wo = pad ? (uint32_t)lane * 16u : woff, so = pad ? (uint32_t)lane * 4u : soff;
    const uint32_t step = pad ? 0u : 1024u;
    if (pad) {
      wp = d_p;
      sp = d_s;
    }
#pragma unroll
    for (int u = 0; u < NSP; ++u) wt[u] = load_nt_u32x4(wp + wo + u * step);
    sv = *reinterpret_cast<const uint32_t*>(sp + so);
  };
  const int nchunks = (nt + DT - 1) / DT;
  if (nt > 0) {
#pragma unroll
    for (int d = 0; d < DT; ++d) load_tile(d, r_w[d], r_s[d]);
  }
  // 4. z -> LDS; this wave's part: row r at zs + r * NSP * 256
#pragma unroll
  for (int v = 0; v < ZV; ++v) {
    const int i = (int)threadIdx.x + KS * 64 * v;
    if (i < nvec) reinterpret_cast<u32x4_t*>(dec_smem)[i] = zst[v];
  }
  __syncthreads();
  const uint8_t* zs = dec_smem + (size_t)w * nz * NSP * 256;
  f32x4_t part = {0.f, 0.f, 0.f, 0.f};
  float ysum = 0.f, ysh = 0.f;
  auto chunk = [&](int ch, auto more) {
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      const int t = ch * DT + d;
      const bool real = t < nt;
      const bool shared_t = has_shared && t == 0;
      const int zrow = shared_t ? K : (real ? t - has_shared : 0);
      const uint8_t* zr = zs + (size_t)zrow * NSP * 256;
#pragma unroll
      for (int u = 0; u < NSP; ++u) {
        u32x4_t xv[4];
        dec_x(zr, u, q, xv);
        const uint32_t sb = real ? (r_s[d] >> (8 * ((sbase + u) & 3))) & 0xFFu : 0u;
        dec_mfma(r_w[d][u], sb, xv, part);
      }
      // this expert's partial is complete: fold it in (selects, no branch)
      ysh = shared_t ? part[0] : ysh;
      ysum += (real && !shared_t) ? part[0] : 0.f;
      part = f32x4_t{0.f, 0.f, 0.f, 0.f};
      if constexpr (decltype(more)::value) load_tile(t + DT, r_w[d], r_s[d]);
    }
  };
  if (nt > 0) {
    for (int ch = 0; ch < nchunks - 1; ++ch) chunk(ch, std::true_type{});
    chunk(nchunks - 1, std::false_type{});
  }
  ysum += ysh;
  if (q == 0) red[w][c] = ysum;
  __syncthreads();
  if (w == 0 && q == 0 && row_ok) {
    float v = red[0][c];
#pragma unroll
    for (int k2 = 1; k2 < KS; ++k2) v += red[k2][c];
    y[row] = f32_bf16(v);
  }
}

// Small-batch down + combine (2 <= M <= kSmallDnRows tokens, after the layout
// and the grouped gate/up kernels).  The same walk as moe_dec1_down_kernel: a
// workgroup owns cpw hidden columns, its KS waves take one K part each, and
// every tile of the list streams through a register ring of DT entries, the
// shared expert first (its weights need no tile list), then the routed tiles
// in list order (ascending expert id).  A tile's rows are up to MR tokens: its
// z rows (this wave's part, 16 bytes a lane a row) ride in the ring with the
// weights and are written to a wave-private LDS buffer just before use, where
// the MFMA operand reads them (lane (c, q) reads row min(c, MR - 1); rows past
// the tile's count repeat its last row and are not used).  Each tile's fresh
// partial rows 0..MR-1 (the q == 0 lanes) are added to their tokens' running
// fp32 sums in tile order and the shared partial after them, so the combine
// order of the reference (ascending expert id, shared last) is kept and y is
// written directly: no partial buffer, no combine launch.
constexpr int kSmallDnRows = 4;    // tokens of the small-batch down kernel
constexpr int kSmallDnTiles = 68;  // tile list entries it stages (M * top_k + M at M = 4, top_k <= 16)

template <int KS, int NSP, int DT, int MR>
__global__ void __launch_bounds__(KS * 64) moe_small_down_kernel(
    const uint16_t* __restrict__ z, const int32_t* __restrict__ tile_expert, const int32_t* __restrict__ tile_rows,
    const int32_t* __restrict__ tile_p0, const int32_t* __restrict__ n_tiles, const int32_t* __restrict__ perm_token,
    const uint8_t* __restrict__ d_p, const uint8_t* __restrict__ d_s, const uint8_t* __restrict__ sh_p,
    const uint8_t* __restrict__ sh_s, uint16_t* __restrict__ y, int M, int H, int I, int E, int has_shared,
    int cpw) {
  constexpr int ZW = NSP * 16;  // 16-byte vectors of one z row in a K part
  __shared__ int s_e[kSmallDnTiles], s_rows[kSmallDnTiles], s_p0[kSmallDnTiles];
  __shared__ int s_tok[kSmallDnTiles * MR];
  __shared__ __attribute__((aligned(16))) u32x4_t zs[KS][MR][ZW + 1];  // +1: rows start on different banks
  __shared__ float red[KS][MR][16];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = lane & 15, q = lane >> 4;
  const int col0 = blockIdx.x * cpw;
  const int ns = I / 128, sbase = w * NSP, ns4 = (ns + 3) / 4;
  const bool row_ok = c < cpw;
  const int row = col0 + (row_ok ? c : cpw - 1);
  const int gr = row >> 4, l = q * 16 + (row & 15);
  const uint32_t woff = (uint32_t)gr * ns * 1024u + (uint32_t)sbase * 1024u + (uint32_t)l * 16u;
  const uint32_t soff = (uint32_t)gr * ns4 * 256u + (uint32_t)(sbase >> 2) * 256u + (uint32_t)l * 4u;
  const int64_t ebytes = (int64_t)H * (I / 2), sbytes = (int64_t)(H / 16) * ns4 * 256;
  const int zl = min(lane, ZW - 1);
  u32x4_t r_w[DT][NSP];
  uint32_t r_s[DT];
  u32x4_t r_z[DT][MR];
  // ring entry t: the shared expert (t == 0 with has_shared, the list's last
  // tile) or routed list tile t - has_shared; padded entries (t >= nt) get
  // scale 0 and are not accumulated
  auto list_index = [&](int t, int nt) { return t >= nt ? 0 : (has_shared ? (t == 0 ? nt - 1 : t - 1) : t); };
  // a padded entry reads one fixed 1 KB block (cache hits, no HBM bytes)
  auto load_w = [&](int li, bool shared_t, bool pad, u32x4_t (&wt)[NSP], uint32_t& sv) {
    const int e = shared_t ? E : s_e[li];
    const uint8_t* wp = pad ? d_p : (e == E ? sh_p : d_p + (int64_t)e * ebytes);
    const uint8_t* sp = pad ? d_s : (e == E ? sh_s : d_s + (int64_t)e * sbytes);
    const uint32_t wo = pad ? (uint32_t)lane * 16u : woff, so = pad ? (uint32_t)lane * 4u : soff;
    const uint32_t step = pad ? 0u : 1024u;
#pragma unroll
    for (int u = 0; u < NSP; ++u) wt[u] = load_nt_u32x4(wp + wo + u * step);
    sv = *reinterpret_cast<const uint32_t*>(sp + so);
  };
  auto load_z = [&](int li, u32x4_t (&zt)[MR]) {
    const int rows = s_rows[li], p0 = s_p0[li];
#pragma unroll
    for (int i = 0; i < MR; ++i) {
      const int pos = p0 + max(min(i, rows - 1), 0);
      zt[i] = reinterpret_cast<const u32x4_t*>(z + (int64_t)pos * I + (int64_t)sbase * 128)[zl];
    }
  };
  // 1. the shared expert's weights need no tile list: issued first
  if (has_shared) load_w(0, true, false, r_w[0], r_s[0]);
  // 2. the tile list (rows, first position and the tokens of its rows) -> LDS
  const int nt = n_tiles[0];
  for (int i = threadIdx.x; i < nt; i += KS * 64) {
    const int rows = tile_rows[i], p0 = tile_p0[i];
    s_e[i] = tile_expert[i];
    s_rows[i] = rows;
    s_p0[i] = p0;
#pragma unroll
    for (int mm = 0; mm < MR; ++mm) s_tok[i * MR + mm] = perm_token[p0 + max(min(mm, rows - 1), 0)];
  }
  __syncthreads();
  // 3. ring prologue
  if (nt > 0) {
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      const int li = list_index(d, nt);
      if (!(has_shared && d == 0)) load_w(li, false, d >= nt, r_w[d], r_s[d]);
      load_z(li, r_z[d]);
    }
  }
  float ysum[MR], ysh[MR];
#pragma unroll
  for (int mm = 0; mm < MR; ++mm) ysum[mm] = ysh[mm] = 0.f;
  const int nchunks = (nt + DT - 1) / DT;
  auto chunk = [&](int ch, auto more) {
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      const int t = ch * DT + d;
      const bool real = t < nt;
      const bool shared_t = has_shared && t == 0;
      const int li = list_index(t, nt);
      // this tile's z rows -> the wave's LDS rows (the previous tile's reads
      // were issued before these writes; the fence orders the reads after them)
      if (lane < ZW) {
#pragma unroll
        for (int i = 0; i < MR; ++i) zs[w][i][lane] = r_z[d][i];
      }
      wave_lds_fence();
      const u32x4_t* zr = zs[w][min(c, MR - 1)];
      f32x4_t part = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < NSP; ++u) {
        u32x4_t xv[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) xv[k] = zr[16 * u + 4 * q + k];
        const uint32_t sb = real ? (r_s[d] >> (8 * ((sbase + u) & 3))) & 0xFFu : 0u;
        dec_mfma(r_w[d][u], sb, xv, part);
      }
      // fold the tile's rows into their tokens' sums (selects; the token and
      // row count are the same in every lane)
      const int rows = real ? s_rows[li] : 0;
#pragma unroll
      for (int i = 0; i < MR; ++i) {
        const int tok = s_tok[li * MR + i];
#pragma unroll
        for (int mm = 0; mm < MR; ++mm) {
          // both arrays updated by selects: a branch between them would make
          // the compiler pick an array by pointer and move both to scratch
          const bool hit = i < rows && tok == mm;
          ysh[mm] = (hit && shared_t) ? part[i] : ysh[mm];
          ysum[mm] = (hit && !shared_t) ? ysum[mm] + part[i] : ysum[mm];
        }
      }
      if constexpr (decltype(more)::value) {
        const int ln = list_index(t + DT, nt);
        load_w(ln, false, t + DT >= nt, r_w[d], r_s[d]);
        load_z(ln, r_z[d]);
      }
    }
  };
  if (nt > 0) {
    for (int ch = 0; ch < nchunks - 1; ++ch) chunk(ch, std::true_type{});
    chunk(nchunks - 1, std::false_type{});
  }
  if (q == 0) {
#pragma unroll
    for (int mm = 0; mm < MR; ++mm) red[w][mm][c] = ysum[mm] + ysh[mm];
  }
  __syncthreads();
  if (w == 0 && q == 0 && row_ok) {
    for (int mm = 0; mm < M; ++mm) {
      float v = red[0][mm][c];
#pragma unroll
      for (int k2 = 1; k2 < KS; ++k2) v += red[k2][mm][c];
      y[(int64_t)mm * H + row] = f32_bf16(v);
    }
  }
}

// Single A16 linear at one token (y [1, N] = x [1, K] . W^T, W MXT16): a
// workgroup owns 16 rows of W (8 when N / 16 < 256); its KS waves split K into equal parts,
// each streaming its part through a register ring of D super-steps with its x
// part staged in wave-private LDS; the parts meet in LDS.
template <int KS, int D, int XV>
__global__ void __launch_bounds__(KS * 64) mx_dec1_linear_kernel(const uint16_t* __restrict__ x,
                                                                 const uint8_t* __restrict__ packed_t,
                                                                 const uint8_t* __restrict__ scale_t,
                                                                 uint16_t* __restrict__ y, int N, int K,
                                                                 int rows) {
  extern __shared__ __attribute__((aligned(16))) uint8_t dec_smem[];
  __shared__ float red[KS][16];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = lane & 15, q = lane >> 4;
  const int ns = K / 128, nsp = ns / KS, sbase = w * nsp;
  // this workgroup's rows (16, or 8 when 16-row groups would leave CUs idle:
  // lanes past them re-read the window's last row, within the same 128-byte line)
  const int row = blockIdx.x * rows + min(c, rows - 1);
  const int g = row >> 4, lr = q * 16 + (row & 15);
  const int nvec = nsp * 16;
  u32x4_t xst[XV];
#pragma unroll
  for (int v = 0; v < XV; ++v) {
    const int i = min(lane + 64 * v, nvec - 1);
    xst[v] = reinterpret_cast<const u32x4_t*>(x + (int64_t)sbase * 128)[i];
  }
  const uint8_t* wt;
  const uint8_t* st;
  dec_ptrs(packed_t, scale_t, g, ns, lr, wt, st);
  const int nchunks = (nsp + D - 1) / D;
  u32x4_t r_w[D];
  uint32_t r_s[D];
  auto load_step = [&](int n, u32x4_t& wv, uint32_t& sv) {
    const int S = sbase + (n < nsp ? n : 0);
    wv = load_nt_u32x4(wt + (int64_t)S * 1024);
    sv = *reinterpret_cast<const uint32_t*>(st + (int64_t)(S >> 2) * 256);
  };
#pragma unroll
  for (int s = 0; s < D; ++s) load_step(s, r_w[s], r_s[s]);
  uint8_t* xs = dec_smem + (size_t)w * nsp * 256;
#pragma unroll
  for (int v = 0; v < XV; ++v) {
    const int i = lane + 64 * v;
    if (i < nvec) reinterpret_cast<u32x4_t*>(xs)[i] = xst[v];
  }
  wave_lds_fence();
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  auto chunk = [&](int ch, auto more) {
#pragma unroll
    for (int s = 0; s < D; ++s) {
      const int n = ch * D + s;
      const int S = sbase + n;
      const bool real = n < nsp;
      u32x4_t xv[4];
      dec_x(xs, real ? n : 0, q, xv);
      const uint32_t sb = real ? (r_s[s] >> (8 * (S & 3))) & 0xFFu : 0u;
      dec_mfma(r_w[s], sb, xv, acc);
      if constexpr (decltype(more)::value) load_step(n + D, r_w[s], r_s[s]);
    }
  };
  for (int ch = 0; ch < nchunks - 1; ++ch) chunk(ch, std::true_type{});
  chunk(nchunks - 1, std::false_type{});
  if (q == 0) red[w][c] = acc[0];
  __syncthreads();
  if (w == 0 && q == 0 && c < rows) {
    float v = red[0][c];
#pragma unroll
    for (int k2 = 1; k2 < KS; ++k2) v += red[k2][c];
    const int n = blockIdx.x * rows + c;
    if (n < N) y[n] = f32_bf16(v);
  }
}

// ring depth of a part of n super-steps: 8, 7 or 4 when it divides n, else the
// largest of 8, 4, 2, 1 not above n (the last chunk is then padded)
static int dec_depth(int n) {
  for (int d : {8, 7, 4})
    if (n % d == 0) return d;
  return n >= 8 ? 8 : (n >= 4 ? 4 : (n >= 2 ? 2 : 1));
}

template <int KS, int XV>
static void launch_dec1_gateup_x(int D, dim3 grid, size_t lds, hipStream_t st, const uint16_t* x, const float* logits,
                                 const float* bias, const int32_t* ids_in, const float* w_in, int32_t* ids_out,
                                 float* w_out, const uint8_t* gu_p, const uint8_t* gu_s, const uint8_t* sh_p,
                                 const uint8_t* sh_s, uint16_t* z, int32_t* te, int32_t* nt, int H, int I, int E,
                                 int K, int func, int renorm, float scale, float limit, hipEvent_t ev_start,
                                 hipEvent_t ev_stop) {
  // the events (stage timing, may be null) are recorded by the dispatch itself:
  // they bracket the kernel's execution, not the launch around it
#define DEC_GU(DV)                                                                                              \
  note_launch();                                                                                                \
  hipExtLaunchKernelGGL((moe_dec1_gateup_kernel<KS, DV, XV>), grid, dim3(KS * 64), lds, st, ev_start, ev_stop, \
                        0u, x, logits, bias, ids_in, w_in, ids_out, w_out, gu_p, gu_s, sh_p, sh_s, z, te, nt, H,  \
                        I, E, K, func, renorm, scale, limit)
  switch (D) {
    case 8: DEC_GU(8); break;
    case 7: DEC_GU(7); break;
    case 4: DEC_GU(4); break;
    case 2: DEC_GU(2); break;
    default: DEC_GU(1); break;
  }
#undef DEC_GU
}

template <int KS, int NSP, int ZV>
static void launch_dec1_down_z(int DT, dim3 grid, size_t lds, hipStream_t st, const uint16_t* z, const int32_t* te,
                               const int32_t* nt, const uint8_t* d_p, const uint8_t* d_s, const uint8_t* sh_p,
                               const uint8_t* sh_s, uint16_t* y, int H, int I, int E, int K, int has_shared, int cpw,
                               hipEvent_t ev_stop) {
#define DEC_DN(DV)                                                                                              \
  note_launch();                                                                                                \
  hipExtLaunchKernelGGL((moe_dec1_down_kernel<KS, NSP, DV, ZV>), grid, dim3(KS * 64), lds, st, nullptr, ev_stop, \
                        0u, z, te, nt, d_p, d_s, sh_p, sh_s, y, H, I, E, K, has_shared, cpw)
  switch (DT) {
    case 4: DEC_DN(4); break;
    case 3: DEC_DN(3); break;
    case 2: DEC_DN(2); break;
    default: DEC_DN(1); break;
  }
#undef DEC_DN
}

template <int KS, int XV>
static void launch_dec1_linear_x(int D, const uint16_t* x, const uint8_t* pt, const uint8_t* st, uint16_t* y,
                                 int64_t n, int64_t k, hipStream_t s) {
  // 8-row workgroups when 16-row groups would leave CUs idle
  const int rows = n / 16 < 256 ? 8 : 16;
  const dim3 grid((unsigned)(n / rows));
  const size_t lds = (size_t)k * 2;
#define DEC_LIN(DV)                                                                                              \
  MOSAIC_LAUNCH((mx_dec1_linear_kernel<KS, DV, XV>), grid, dim3(KS * 64), lds, s, x, pt, st, y, (int)n, (int)k, \
                     rows)
  switch (D) {
    case 8: DEC_LIN(8); break;
    case 7: DEC_LIN(7); break;
    case 4: DEC_LIN(4); break;
    case 2: DEC_LIN(2); break;
    default: DEC_LIN(1); break;
  }
#undef DEC_LIN
}

bool linear_decode1_supported(int64_t m, int64_t n, int64_t k) {
  return m == 1 && n % 16 == 0 && k % 1024 == 0 && (k / 128 / 8) * 16 <= 64 * kDecXVMax;
}

// K split over 8 waves: every wave's part is loaded in one ring fill at K <= 8192
void launch_linear_decode1(const uint16_t* x, const uint8_t* pt, const uint8_t* st, uint16_t* y, int64_t n, int64_t k,
                           hipStream_t s) {
  const int part = (int)(k / 128 / 8);
  const int d = dec_depth(part);
  const int xv = (part * 16 + 63) / 64;
  if (xv <= 2)
    launch_dec1_linear_x<8, 2>(d, x, pt, st, y, n, k, s);
  else if (xv <= 4)
    launch_dec1_linear_x<8, 4>(d, x, pt, st, y, n, k, s);
  else
    launch_dec1_linear_x<8, 8>(d, x, pt, st, y, n, k, s);
}

constexpr int kDecGuKS = 2;   // gate/up: waves (K parts) per workgroup (all workgroups resident: routing latency paid once)
// down: K parts per workgroup and super-steps per part (a part must sit inside
// one 4-step scale dword): 4 waves of 1, 2 or 4 (inter 512, 1024, 2048), 8 of
// 4 (4096); 0 = not handled
static int dec_dn_ks(int64_t nsi) {
  if (nsi == 32) return 8;
  if (nsi == 4 || nsi == 8 || nsi == 16) return 4;
  return 0;
}
// the batch-1 down kernel: 8 parts of 2 steps at inter 2048 as well (3584 waves
// instead of 1792 keep more bytes in flight; measured 13.5-13.7 against
// 13.8-14.2 us at the benchmark decode shape)
static int dec1_dn_ks(int64_t nsi) { return nsi == 16 ? 8 : dec_dn_ks(nsi); }

bool moe_decode1_supported(int64_t m, int64_t hidden, int64_t inter, int64_t top_k, int has_shared) {
  if (m != 1 || top_k < 1 || top_k > kRouteMaxTopK) return false;
  const int64_t nsh = hidden / 128, nsi = inter / 128;
  if (hidden % 128 || inter % 128 || nsh % kDecGuKS || dec1_dn_ks(nsi) == 0) return false;
  const int64_t gu_part = nsh / kDecGuKS, dn_part = nsi / dec1_dn_ks(nsi);
  if (gu_part * 16 > 64 * kDecXVMax) return false;                        // x staging registers
  if ((top_k + has_shared) * dn_part * 16 > 64 * kDecZVMax) return false;  // z staging registers (one wave's share or less)
  if ((size_t)(top_k + has_shared) * inter * 2 > 64 * 1024) return false;
  return true;
}

int launch_moe_decode1(const uint16_t* x, const float* logits, const float* bias, const int32_t* ids_in,
                       const float* w_in, int32_t* ids_out, float* w_out, const uint8_t* gu_p, const uint8_t* gu_s,
                       const uint8_t* d_p, const uint8_t* d_s, const uint8_t* sh_gu_p, const uint8_t* sh_gu_s,
                       const uint8_t* sh_d_p, const uint8_t* sh_d_s, uint16_t* y, int64_t H, int64_t I, int64_t E,
                       int64_t K, int has_shared, int func, int renorm, float route_scale, float limit, uint16_t* z,
                       int32_t* tile_expert, int32_t* n_tiles, void* const* marks, hipStream_t st) {
  MOSAIC_CHECK_ARG(E >= 1 && E <= kRouteMaxExperts && K <= E, "moe decode: E=%lld top_k=%lld", (long long)E,
                   (long long)K);
  MOSAIC_CHECK_ARG(func >= 0 && func <= 2, "moe decode: score func %d", func);
  auto mark = [&](int i) {
    if (marks && marks[i]) (void)hipEventRecord((hipEvent_t)marks[i], st);
  };
  auto ev = [&](int i) { return marks ? (hipEvent_t)marks[i] : (hipEvent_t) nullptr; };
  // routing runs inside the gate/up launch (the layout stage is the dispatch
  // latency); marks 1 and 2 are the gate/up kernel's own start and end
  const int dn_ks = dec1_dn_ks(I / 128);
  const int gu_part = (int)(H / 128 / kDecGuKS), dn_part = (int)(I / 128 / dn_ks);
  const int nz = (int)K + has_shared;
  const int gd = dec_depth(gu_part);
  const int xv = (gu_part * 16 + 63) / 64;
  const dim3 ggrid((unsigned)(I / 16), (unsigned)nz);
#define GU_ARGS gd, ggrid, (size_t)H * 2, st, x, logits, bias, ids_in, w_in, ids_out, w_out, gu_p, gu_s, sh_gu_p, \
                sh_gu_s, z, tile_expert, n_tiles, (int)H, (int)I, (int)E, (int)K, func, renorm, route_scale, limit, \
                ev(1), ev(2)
  if (xv <= 2)
    launch_dec1_gateup_x<kDecGuKS, 2>(GU_ARGS);
  else if (xv <= 4)
    launch_dec1_gateup_x<kDecGuKS, 4>(GU_ARGS);
  else
    launch_dec1_gateup_x<kDecGuKS, 8>(GU_ARGS);
#undef GU_ARGS
  MOSAIC_LAUNCH_CHECK("moe_decode1_gateup");
  // ring of 3 tiles (DT * NSP super-steps in flight), 4 when a part is one step;
  // 8 columns per workgroup when 16 would give fewer workgroups than CUs
  const int dt = dn_part == 1 ? 4 : 3;
  const int cpw = H / 16 >= 256 ? 16 : 8;
  const int zv = (int)(((int64_t)nz * I / 8 + dn_ks * 64 - 1) / (dn_ks * 64));
  const dim3 dgrid((unsigned)(H / cpw));
#define DN_ARGS dt, dgrid, (size_t)nz * I * 2, st, z, tile_expert, n_tiles, d_p, d_s, sh_d_p, sh_d_s, y, (int)H, \
                (int)I, (int)E, (int)K, has_shared, cpw, ev(3)
#define DN_Z(KSV, NSPV)                                  \
  if (zv <= 5)                                           \
    launch_dec1_down_z<KSV, NSPV, 5>(DN_ARGS);           \
  else if (zv <= 10)                                     \
    launch_dec1_down_z<KSV, NSPV, 10>(DN_ARGS);          \
  else                                                   \
    launch_dec1_down_z<KSV, NSPV, kDecZVMax>(DN_ARGS);
  if (dn_ks == 8 && dn_part == 2) {
    DN_Z(8, 2)
  } else if (dn_ks == 8) {
    DN_Z(8, 4)
  } else if (dn_part == 4) {
    DN_Z(4, 4)
  } else if (dn_part == 2) {
    DN_Z(4, 2)
  } else {
    DN_Z(4, 1)
  }
#undef DN_Z
#undef DN_ARGS
  MOSAIC_LAUNCH_CHECK("moe_decode1_down");
  mark(4);  // mark 3 is the down kernel's end; the combine is fused into it
  return kOk;
}

bool moe_small_down_supported(int64_t m, int64_t hidden, int64_t inter, int64_t tile_cap) {
  return m >= 2 && m <= kSmallDnRows && hidden % 128 == 0 && inter % 128 == 0 && dec_dn_ks(inter / 128) != 0 &&
         tile_cap <= kSmallDnTiles;
}

template <int KS, int NSP, int DT>
static void launch_small_down_k(dim3 grid, int mr, hipStream_t st, const uint16_t* z, const int32_t* te,
                                const int32_t* tr, const int32_t* tp, const int32_t* nt, const int32_t* ptok,
                                const uint8_t* d_p, const uint8_t* d_s, const uint8_t* sh_p, const uint8_t* sh_s,
                                uint16_t* y, int M, int H, int I, int E, int has_shared, int cpw) {
  if (mr == 2)
    MOSAIC_LAUNCH((moe_small_down_kernel<KS, NSP, DT, 2>), grid, dim3(KS * 64), 0, st, z, te, tr, tp, nt, ptok,
                       d_p, d_s, sh_p, sh_s, y, M, H, I, E, has_shared, cpw);
  else
    MOSAIC_LAUNCH((moe_small_down_kernel<KS, NSP, DT, 4>), grid, dim3(KS * 64), 0, st, z, te, tr, tp, nt, ptok,
                       d_p, d_s, sh_p, sh_s, y, M, H, I, E, has_shared, cpw);
}

void launch_moe_small_down(const uint16_t* z, const int32_t* tile_expert, const int32_t* tile_rows,
                           const int32_t* tile_p0, const int32_t* n_tiles, const int32_t* perm_token,
                           const uint8_t* d_p, const uint8_t* d_s, const uint8_t* sh_d_p, const uint8_t* sh_d_s,
                           uint16_t* y, int64_t M, int64_t H, int64_t I, int64_t E, int has_shared, hipStream_t st) {
  // K parts as the batch-1 down kernel; 8 columns per workgroup when 16 would
  // give fewer workgroups than CUs
  const int dn_ks = dec_dn_ks(I / 128), dn_part = (int)(I / 128 / dn_ks);
  const int cpw = H / 16 >= 256 ? 16 : 8;
  const dim3 grid((unsigned)(H / cpw));
  const int mr = M <= 2 ? 2 : 4;
#define SD_ARGS grid, mr, st, z, tile_expert, tile_rows, tile_p0, n_tiles, perm_token, d_p, d_s, sh_d_p, sh_d_s, y, \
                (int)M, (int)H, (int)I, (int)E, has_shared, cpw
  if (dn_ks == 8)
    launch_small_down_k<8, 4, 3>(SD_ARGS);
  else if (dn_part == 4)
    launch_small_down_k<4, 4, 3>(SD_ARGS);
  else if (dn_part == 2)
    launch_small_down_k<4, 2, 3>(SD_ARGS);
  else
    launch_small_down_k<4, 1, 4>(SD_ARGS);
#undef SD_ARGS
}

}  // namespace mosaic
