// A16 MXFP4 path on gfx950: bf16 activations against MXFP4 weights decoded in
// registers (v_cvt_scalef32_pk_bf16_fp4, block scale applied in the convert)
// and multiplied on v_mfma_f32_16x16x32_bf16 with fp32 accumulation.
//
// Tile shape: one wave owns a 16 (tokens) x 16 (weight rows) output tile and
// walks K in super-steps of 128.  In a super-step, lane l (c = l%16,
// q = l/16) loads the 16-byte MX block b = 4S+q of weight row c (one 128-bit
// load, 32 nibbles, one e8m0 byte) and the 32 bf16 of its token row c at the
// same K, then issues four MFMAs over the 4 x 8-element sub-slices.  A and B
// use the same lane->K map, so the K order inside the MFMA does not matter.
// Weight bytes are read exactly once per token tile; scales come from one
// aligned dword per super-step (bytes 4S..4S+3 of the scale row).
#include "common.h"
#include "moe_internal.h"
#include "../../include/mosaic_amd.h"

namespace mosaic {

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

template <int U>
__device__ __forceinline__ void a16_steps(const uint8_t* __restrict__ wrow, const uint8_t* __restrict__ srow,
                                          const uint16_t* __restrict__ xrow, bool xvalid, int q, int S,
                                          f32x4_t& acc) {
  u32x4_t wv[U];
  uint32_t sv[U];
  u32x4_t xv[U][4];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    wv[u] = load_nt_u32x4(wrow + 16 * (4 * (S + u) + q));
    sv[u] = *reinterpret_cast<const uint32_t*>(srow + 4 * (S + u));
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (xvalid) {
      const u32x4_t* xp = reinterpret_cast<const u32x4_t*>(xrow + 32 * (4 * (S + u) + q));
#pragma unroll
      for (int j = 0; j < 4; ++j) xv[u][j] = xp[j];
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) xv[u][j] = u32x4_t{0u, 0u, 0u, 0u};
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const float sf = e8m0_f32((sv[u] >> (8 * q)) & 0xFFu);
    bf16x8_t wb[4];
    mx_block_to_bf16(wv[u], sf, wb);
#pragma unroll
    for (int s = 0; s < 4; ++s)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xv[u][s]), wb[s], acc, 0, 0, 0);
  }
}

// D[token 4q+r][col c] += sum over super-steps [s_begin, s_end) of the tile.
__device__ __forceinline__ f32x4_t tile_dot_a16(const uint8_t* __restrict__ wrow, const uint8_t* __restrict__ srow,
                                                const uint16_t* __restrict__ xrow, bool xvalid, int q, int s_begin,
                                                int s_end) {
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  int S = s_begin;
  for (; S + 4 <= s_end; S += 4) a16_steps<4>(wrow, srow, xrow, xvalid, q, S, acc);
  for (; S < s_end; ++S) a16_steps<1>(wrow, srow, xrow, xvalid, q, S, acc);
  return acc;
}

// ---------------------------------------------------- MoE gate/up + SwiGLU --
// grid (inter/32, tile_cap), 256 threads.  Wave w of block x owns inter
// indices j0 = (4x+w)*8 .. j0+7: MFMA columns 0..7 are gate rows j0+c,
// columns 8..15 the matching up rows inter+j0+c-8.  The epilogue pairs
// column c with c+8 (lane l^8), applies SwiGLU and the route weight, and
// stores z[p][j] as bf16 for every sorted assignment position p of the tile.
__global__ void __launch_bounds__(256) moe_a16_gateup_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ gu_p, const uint8_t* __restrict__ gu_s,
    const uint8_t* __restrict__ sh_p, const uint8_t* __restrict__ sh_s, const int32_t* __restrict__ tile_expert,
    const int32_t* __restrict__ tile_start, const int32_t* __restrict__ tile_rows,
    const int32_t* __restrict__ n_tiles, const int32_t* __restrict__ offsets, const int32_t* __restrict__ perm_token,
    const float* __restrict__ perm_weight, uint16_t* __restrict__ z, int H, int I, int E, float limit) {
  const int tile = blockIdx.y;
  if (tile >= n_tiles[0]) return;
  const int e = tile_expert[tile], rows = tile_rows[tile];
  const int p0 = offsets[e] + tile_start[tile];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 15, q = lane >> 4;
  const int j0 = (blockIdx.x * 4 + wave) * 8;
  if (j0 >= I) return;
  const int64_t rb = H / 2, sb = H / 32;
  const uint8_t* bp = (e == E) ? sh_p : gu_p + (int64_t)e * 2 * I * rb;
  const uint8_t* bs = (e == E) ? sh_s : gu_s + (int64_t)e * 2 * I * sb;
  const int wr = (c < 8) ? (j0 + c) : (I + j0 + c - 8);
  const bool xvalid = c < rows;
  const uint16_t* xrow = x + (int64_t)(xvalid ? perm_token[p0 + c] : 0) * H;
  f32x4_t acc = tile_dot_a16(bp + (int64_t)wr * rb, bs + (int64_t)wr * sb, xrow, xvalid, q, 0, H / 128);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float other = __shfl_xor(acc[r], 8, 64);
    const int ti = 4 * q + r;
    if (c < 8 && ti < rows) {
      const float zv = swiglu_f32(acc[r], other, limit) * perm_weight[p0 + ti];
      z[(int64_t)(p0 + ti) * I + j0 + c] = f32_bf16(zv);
    }
  }
}

// ------------------------------------------------------------- MoE down ----
// grid (ceil(H/64), tile_cap), 256 threads; wave tile = 16 hidden rows.
__global__ void __launch_bounds__(256) moe_a16_down_kernel(
    const uint16_t* __restrict__ z, const uint8_t* __restrict__ d_p, const uint8_t* __restrict__ d_s,
    const uint8_t* __restrict__ sh_p, const uint8_t* __restrict__ sh_s, const int32_t* __restrict__ tile_expert,
    const int32_t* __restrict__ tile_start, const int32_t* __restrict__ tile_rows,
    const int32_t* __restrict__ n_tiles, const int32_t* __restrict__ offsets, float* __restrict__ yp, int H, int I,
    int E) {
  const int tile = blockIdx.y;
  if (tile >= n_tiles[0]) return;
  const int e = tile_expert[tile], rows = tile_rows[tile];
  const int p0 = offsets[e] + tile_start[tile];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 15, q = lane >> 4;
  const int h0 = (blockIdx.x * 4 + wave) * 16;
  if (h0 >= H) return;
  const int64_t rb = I / 2, sb = I / 32;
  const uint8_t* bp = (e == E) ? sh_p : d_p + (int64_t)e * H * rb;
  const uint8_t* bs = (e == E) ? sh_s : d_s + (int64_t)e * H * sb;
  const bool xvalid = c < rows;
  const uint16_t* zrow = z + (int64_t)(p0 + (xvalid ? c : 0)) * I;
  f32x4_t acc = tile_dot_a16(bp + (int64_t)(h0 + c) * rb, bs + (int64_t)(h0 + c) * sb, zrow, xvalid, q, 0, I / 128);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int ti = 4 * q + r;
    if (ti < rows) yp[(int64_t)(p0 + ti) * H + h0 + c] = acc[r];
  }
}

// ------------------------------------------------------------ combine ------
// y[t][h] = bf16( sum of t's expert partials in ascending expert id, then the
// shared expert's partial ).  Assignments dropped by the layout (inv_pos < 0)
// contribute nothing.
__global__ void __launch_bounds__(256) moe_combine_kernel(const float* __restrict__ yp,
                                                          const int32_t* __restrict__ ids,
                                                          const int32_t* __restrict__ inv_pos,
                                                          uint16_t* __restrict__ y, int M, int K, int H,
                                                          int has_shared) {
  const int t = blockIdx.y;
  const int h = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= M || h >= H) return;
  int ord[16];
  int key[16];
  for (int s = 0; s < K; ++s) {
    int k = ids[(int64_t)t * K + s];
    int j = s;
    while (j > 0 && key[j - 1] > k) {  // stable insertion sort by expert id
      key[j] = key[j - 1];
      ord[j] = ord[j - 1];
      --j;
    }
    key[j] = k;
    ord[j] = s;
  }
  float acc = 0.f;
  for (int s = 0; s < K; ++s) {
    const int p = inv_pos[(int64_t)t * K + ord[s]];
    if (p >= 0) acc += yp[(int64_t)p * H + h];
  }
  if (has_shared) {
    const int p = inv_pos[(int64_t)M * K + t];
    if (p >= 0) acc += yp[(int64_t)p * H + h];
  }
  y[(int64_t)t * H + h] = f32_bf16(acc);
}

// ------------------------------------------------------- single linear -----
// y [M, N] = x [M, K] . W^T.  grid (ceil(N/16), ceil(M/16)), 8 waves per block:
// wave w takes super-steps [w*S/8, (w+1)*S/8) of the same 16x16 tile, partial
// tiles are summed in wave order through LDS by wave 0.
constexpr int kLinWaves = 8;
__global__ void __launch_bounds__(kLinWaves * 64) mx_linear_a16_kernel(const uint16_t* __restrict__ x,
                                                                        const uint8_t* __restrict__ packed,
                                                                        const uint8_t* __restrict__ scale,
                                                                        uint16_t* __restrict__ y, int M, int N,
                                                                        int K) {
  __shared__ f32x4_t part[kLinWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 15, q = lane >> 4;
  const int n0 = blockIdx.x * 16, m0 = blockIdx.y * 16;
  const int row = min(n0 + c, N - 1);
  const bool xvalid = (m0 + c) < M;
  const uint16_t* xrow = x + (int64_t)(xvalid ? m0 + c : 0) * K;
  const int ns = K / 128;
  const int s0 = (int)((int64_t)ns * wave / kLinWaves), s1 = (int)((int64_t)ns * (wave + 1) / kLinWaves);
  f32x4_t acc = tile_dot_a16(packed + (int64_t)row * (K / 2), scale + (int64_t)row * (K / 32), xrow, xvalid, q, s0,
                             s1);
  part[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    f32x4_t sum = part[0][lane];
    for (int w = 1; w < kLinWaves; ++w) sum += part[w][lane];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int mi = m0 + 4 * q + r;
      if (mi < M && n0 + c < N) y[(int64_t)mi * N + n0 + c] = f32_bf16(sum[r]);
    }
  }
}

// ----------------------------------------------------------- workspace -----
struct MoeWorkspace {
  int32_t *counts, *offsets, *perm, *perm_token, *sorted_ids, *inv_pos;
  float* perm_weight;
  int32_t *tile_expert, *tile_start, *tile_rows, *n_tiles;
  uint16_t* z;
  float* yp;
  int64_t tile_cap;
  size_t bytes;
};

static inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

static MoeWorkspace carve_moe_workspace(char* base, int64_t M, int64_t H, int64_t I, int64_t E, int64_t K,
                                        int has_shared, int block_m) {
  MoeWorkspace w{};
  const int64_t A = M * K + (has_shared ? M : 0);
  const int64_t Ee = E + (has_shared ? 1 : 0);
  const int64_t u = A < Ee ? A : Ee;
  w.tile_cap = (A + u * (block_m - 1)) / block_m;
  size_t off = 0;
  auto take = [&](size_t bytes) -> char* {
    char* p = base ? base + off : nullptr;
    off += align256(bytes);
    return p;
  };
  w.counts = (int32_t*)take(4 * (Ee + 1));
  w.offsets = (int32_t*)take(4 * (Ee + 2));
  w.perm = (int32_t*)take(4 * A);
  w.perm_token = (int32_t*)take(4 * A);
  w.perm_weight = (float*)take(4 * A);
  w.sorted_ids = (int32_t*)take(4 * A);
  w.inv_pos = (int32_t*)take(4 * A);
  w.tile_expert = (int32_t*)take(4 * w.tile_cap);
  w.tile_start = (int32_t*)take(4 * w.tile_cap);
  w.tile_rows = (int32_t*)take(4 * w.tile_cap);
  w.n_tiles = (int32_t*)take(4);
  w.z = (uint16_t*)take(2 * A * I);
  w.yp = (float*)take(4 * A * H);
  w.bytes = off;
  return w;
}

constexpr int kMoeBlockM = 16;

}  // namespace mosaic

using namespace mosaic;

extern "C" int mosaic_mx_linear_a16(const uint16_t* x, const uint8_t* packed, const uint8_t* scale, uint16_t* y,
                                    int64_t m, int64_t n, int64_t k, void* stream) {
  MOSAIC_CHECK_ARG(x && packed && scale && y, "mx_linear_a16: null pointer");
  MOSAIC_CHECK_ARG(k > 0 && k % 128 == 0, "mx_linear_a16: K=%lld must be a positive multiple of 128", (long long)k);
  MOSAIC_CHECK_ARG(m >= 0 && n >= 0 && m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 31),
                   "mx_linear_a16: shape out of range");
  if (m == 0 || n == 0) return kOk;
  dim3 grid((unsigned)((n + 15) / 16), (unsigned)((m + 15) / 16));
  hipLaunchKernelGGL(mx_linear_a16_kernel, grid, dim3(kLinWaves * 64), 0, (hipStream_t)stream, x, packed, scale, y,
                     (int)m, (int)n, (int)k);
  MOSAIC_RETURN_LAUNCH("mx_linear_a16");
}

extern "C" size_t mosaic_moe_a16_workspace_bytes(int64_t m, int64_t hidden, int64_t inter, int64_t n_experts,
                                                 int64_t top_k, int has_shared) {
  return carve_moe_workspace(nullptr, m, hidden, inter, n_experts, top_k, has_shared, kMoeBlockM).bytes;
}

extern "C" int mosaic_moe_a16_forward(const uint16_t* x, const float* logits, int32_t* ids, float* weights,
                                      const uint8_t* gu_packed, const uint8_t* gu_scale, const uint8_t* d_packed,
                                      const uint8_t* d_scale, const uint8_t* sh_gu_packed,
                                      const uint8_t* sh_gu_scale, const uint8_t* sh_d_packed,
                                      const uint8_t* sh_d_scale, uint16_t* y, int64_t m, int64_t hidden,
                                      int64_t inter, int64_t n_experts, int64_t top_k, int score_func, int renorm,
                                      float route_scale, const float* route_bias, float swiglu_limit,
                                      void* workspace, size_t workspace_bytes, void* stream) {
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
  MoeWorkspace w = carve_moe_workspace((char*)workspace, m, hidden, inter, n_experts, top_k, has_shared, kMoeBlockM);
  MOSAIC_CHECK_ARG(workspace_bytes >= w.bytes, "moe_a16_forward: workspace %zu < %zu bytes", workspace_bytes,
                   w.bytes);
  hipStream_t st = (hipStream_t)stream;
  LayoutOut lo{w.counts, w.offsets, w.perm, w.perm_token, w.perm_weight, w.sorted_ids, w.inv_pos,
               w.tile_expert, w.tile_start, w.tile_rows, w.n_tiles};
  int rc = launch_route_layout(logits, route_bias, ids, weights, m, n_experts, top_k, score_func, renorm,
                               route_scale, has_shared, kMoeBlockM, w.tile_cap, lo, st);
  if (rc != 0) return rc;
  const unsigned tcap = (unsigned)w.tile_cap;
  hipLaunchKernelGGL(moe_a16_gateup_kernel, dim3((unsigned)((inter + 31) / 32), tcap), dim3(256), 0, st, x,
                     gu_packed, gu_scale, sh_gu_packed, sh_gu_scale, w.tile_expert, w.tile_start, w.tile_rows,
                     w.n_tiles, w.offsets, w.perm_token, w.perm_weight, w.z, (int)hidden, (int)inter,
                     (int)n_experts, swiglu_limit);
  MOSAIC_LAUNCH_CHECK("moe_a16_gateup");
  hipLaunchKernelGGL(moe_a16_down_kernel, dim3((unsigned)((hidden + 63) / 64), tcap), dim3(256), 0, st, w.z,
                     d_packed, d_scale, sh_d_packed, sh_d_scale, w.tile_expert, w.tile_start, w.tile_rows,
                     w.n_tiles, w.offsets, w.yp, (int)hidden, (int)inter, (int)n_experts);
  MOSAIC_LAUNCH_CHECK("moe_a16_down");
  hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)((hidden + 255) / 256), (unsigned)m), dim3(256), 0, st,
                     w.yp, ids, w.inv_pos, y, (int)m, (int)top_k, (int)hidden, has_shared);
  MOSAIC_RETURN_LAUNCH("moe_combine");
}
