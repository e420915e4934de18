// A16 MXFP4 linear on the KN layout of the reference's skinny path
// (skinny_mxfp4_gemm, kernels/skinny_fp4.py:113-144, and the grouped
// _grouped_skinny_gemm of fused_moe_skinny, :237-322):
//   y [m, n] = x [m, k] . W,   W [k, n] = E2M1(packed [k, n/2]) * 2^(scale [k, n/32] - 127)
// bf16 x, fp32 accumulation, bf16 y.
//
// In KN, the 16 bytes of a row chunk are 32 N values at one k sharing one
// e8m0 byte: exactly one v_cvt_scalef32_pk_bf16_fp4 scale, so every chunk
// decodes to exact bf16 in registers.  The MFMA (v_mfma_f32_16x16x32_bf16)
// wants 8 consecutive K per lane at one column, so a wave writes its decoded
// [32 k][64 n] slice row-major into wave-private LDS and reads the B operands
// back with the gfx950 transposing read ds_read_b64_tr_b16: in each 16-lane
// group, lane l receives element l%4 of the 8-byte chunks of lanes l/4 + 4i
// (i = 0..3), which turns four 16-column rows into four K-consecutive values
// per column.  x (16 rows of the M tile) is staged once per workgroup.
//
// Work split: a workgroup of 4 waves owns 256 columns (whole 128-byte rows of
// the weight), one chunk of K (NS steps of 32 rows, NS in {4, 8, 16}) and one
// tile of at most 16 rows of x.  When K is split over several workgroups
// their fp32 partials go to a caller workspace and a second kernel sums them
// in chunk order (deterministic); with one chunk y is written directly.
#include <hip/hip_runtime.h>

#include "../../include/mosaic_amd.h"
#include "common.h"
#include "moe_internal.h"

namespace mosaic {
namespace {

typedef short v4s_t __attribute__((ext_vector_type(4)));

constexpr int kKnCols = 64;                 // columns per wave
constexpr int kKnWgCols = 4 * kKnCols;      // columns per workgroup
constexpr int kKnPitch = kKnCols * 2 + 16;  // LDS row pitch (bytes) of a wave's decoded slice
constexpr int kKnSlice = 32 * kKnPitch;     // one step's slice: 32 rows

struct KnTiles {  // optional tile list (grouped experts); null -> dense M tiles
  const int32_t* expert;
  const int32_t* rows;
  const int32_t* p0;
  const int32_t* n_tiles;
};

// grid (ceil(n / 256), ks, m tiles or tile_cap); 256 threads
template <int NS>
__global__ void __launch_bounds__(256) mx_kn_a16_kernel(const uint16_t* __restrict__ x,
                                                        const int32_t* __restrict__ x_rows,
                                                        const uint8_t* __restrict__ packed,
                                                        const uint8_t* __restrict__ scale, int64_t w_stride,
                                                        int64_t s_stride, KnTiles tl, float* __restrict__ part,
                                                        uint16_t* __restrict__ y, int M, int N, int K) {
  constexpr int KC = 32 * NS;
  __shared__ __attribute__((aligned(16))) uint16_t s_x[16][KC + 8];
  __shared__ __attribute__((aligned(16))) unsigned char s_w[4][2][kKnSlice];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ks = blockIdx.y, kbeg = ks * KC;
  // rows of this tile: [r0, r0 + nr) of the (gathered) x / y row space
  int r0, nr, e = 0;
  if (tl.expert) {
    const int t = blockIdx.z;
    if (t >= tl.n_tiles[0]) return;
    e = tl.expert[t];
    r0 = tl.p0[t];
    nr = tl.rows[t];
  } else {
    r0 = blockIdx.z * 16;
    nr = min(16, M - r0);
  }
  const uint8_t* wp = packed + (int64_t)e * w_stride;
  const uint8_t* sp = scale + (int64_t)e * s_stride;
  const int nb = blockIdx.x * kKnWgCols + wave * kKnCols;  // this wave's first column
  // weight loads of every step first (one 16-byte chunk + its scale byte per lane and step)
  const int rr = lane >> 1, half = lane & 1;
  const int col = nb + 32 * half;
  u32x4_t wv[NS];
  uint32_t sv[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int k = kbeg + 32 * s + rr;
    const bool ok = k < K && col < N;
    wv[s] = ok ? *reinterpret_cast<const u32x4_t*>(wp + (int64_t)k * (N / 2) + col / 2) : u32x4_t{0u, 0u, 0u, 0u};
    sv[s] = ok ? (uint32_t)sp[(int64_t)k * (N / 32) + col / 32] : 127u;
  }
  // x rows of the tile over this K chunk (bf16, zero past M / K)
  for (int i = tid; i < 16 * (KC / 8); i += 256) {
    const int r = i / (KC / 8), c8 = (i % (KC / 8)) * 8;
    u32x4_t v = {0u, 0u, 0u, 0u};
    if (r < nr && kbeg + c8 < K) {
      const int xr = x_rows ? x_rows[r0 + r] : r0 + r;
      v = *reinterpret_cast<const u32x4_t*>(x + (int64_t)xr * K + kbeg + c8);
    }
    *reinterpret_cast<u32x4_t*>(&s_x[r][c8]) = v;
  }
  __syncthreads();
  const int g = lane >> 4, c16 = lane & 15;
  f32x4_t acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    unsigned char* buf = s_w[wave][s & 1];
    // decode: 32 bf16 of row rr, columns 32*half .. +32 of the slice
    bf16x8_t d[4];
    mx_block_to_bf16(wv[s], e8m0_f32(sv[s]), d);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<bf16x8_t*>(buf + rr * kKnPitch + (32 * half + 8 * j) * 2) = d[j];
    wave_lds_fence();  // the slice is in LDS before any lane reads it
    // A: row c16 of the tile, K 8g .. 8g + 8 of this step
    const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(&s_x[c16][32 * s + 8 * g]);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      // B: column 16t + c16, K 8g .. 8g + 8, by two transposing reads of rows
      // 8g + c16/4 (+4), columns 16t + 4 (c16 % 4) .. +4
      const int boff = (8 * g + (c16 >> 2)) * kKnPitch + (16 * t + 4 * (c16 & 3)) * 2;
      const v4s_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) v4s_t*)(buf + boff));
      const v4s_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) v4s_t*)(buf + boff + 4 * kKnPitch));
      typedef short v8s_t __attribute__((ext_vector_type(8)));
      const v8s_t bs = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(bf16x8_t, bs), acc[t], 0, 0, 0);
    }
  }
  // acc[t][i]: tile row 4g + i, column nb + 16t + c16
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int n = nb + 16 * t + c16;
    if (n >= N) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * g + i;
      if (r >= nr) continue;
      const int64_t row = r0 + r;
      if (part)
        part[((int64_t)ks * M + row) * N + n] = acc[t][i];
      else
        y[row * N + n] = f32_bf16(acc[t][i]);
    }
  }
}

// y [m, n] = bf16(sum over ks of part[ks][m][n], in ks order)
__global__ void __launch_bounds__(256) kn_reduce_kernel(const float* __restrict__ part, uint16_t* __restrict__ y,
                                                        int64_t mn, int ks) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= mn) return;
  float s = 0.f;
  for (int j = 0; j < ks; ++j) s += part[(int64_t)j * mn + i];
  y[i] = f32_bf16(s);
}

int kn_steps(int64_t n, int64_t k, int64_t mtiles) {
  const int64_t ntiles = (n + kKnWgCols - 1) / kKnWgCols;
  for (int ns : {16, 8})
    if (ntiles * ((k + 32 * ns - 1) / (32 * ns)) * mtiles >= 384) return ns;
  return 4;
}

int launch_kn(const uint16_t* x, const int32_t* x_rows, const uint8_t* packed, const uint8_t* scale,
              int64_t w_stride, int64_t s_stride, KnTiles tl, int64_t zdim, float* ws, size_t ws_bytes, uint16_t* y,
              int64_t m, int64_t n, int64_t k, int ns, hipStream_t st) {
  const int64_t ks = (k + 32 * ns - 1) / (32 * ns);
  float* part = nullptr;
  if (ks > 1) {
    MOSAIC_CHECK_ARG(ws && ws_bytes >= (size_t)ks * m * n * 4, "mx_kn_linear_a16: workspace %zu < %zu bytes",
                     ws_bytes, (size_t)ks * m * n * 4);
    part = ws;
  }
  const dim3 grid((unsigned)((n + kKnWgCols - 1) / kKnWgCols), (unsigned)ks, (unsigned)zdim);
#define KN_LAUNCH(NSV)                                                                                              \
  MOSAIC_LAUNCH(mx_kn_a16_kernel<NSV>, grid, dim3(256), 0, st, x, x_rows, packed, scale, w_stride, s_stride, \
                     tl, part, y, (int)m, (int)n, (int)k)
  if (ns == 16)
    KN_LAUNCH(16);
  else if (ns == 8)
    KN_LAUNCH(8);
  else
    KN_LAUNCH(4);
#undef KN_LAUNCH
  MOSAIC_LAUNCH_CHECK("mx_kn_a16");
  if (part) {
    const int64_t mn = m * n;
    MOSAIC_LAUNCH(kn_reduce_kernel, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, st, part, y, mn, (int)ks);
    MOSAIC_LAUNCH_CHECK("mx_kn_reduce");
  }
  return kOk;
}

// fused_moe_skinny's torch epilogue in bf16 arithmetic
// (kernels/skinny_fp4.py:309-322): z = bf16(bf16(silu(gate)) * up) per row of
// gu [a, 2 * inter] (gate | up halves)
__global__ void __launch_bounds__(256) skinny_swiglu_kernel(const uint16_t* __restrict__ gu, uint16_t* __restrict__ z,
                                                            int64_t a, int inter) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a * inter) return;
  const int64_t r = i / inter, c = i % inter;
  const float gate = bf16_f32(gu[r * 2 * inter + c]);
  const float up = bf16_f32(gu[r * 2 * inter + inter + c]);
  const float sg = bf16_f32(f32_bf16(gate / (1.0f + expf(-gate))));
  z[i] = f32_bf16(sg * up);
}

// y [t] = sum over the token's assignments (flat order) of bf16(y_g[pos] * bf16(w)),
// accumulated in bf16 from 0 (index_add_ on a bf16 tensor, kernels/skinny_fp4.py:319-322)
__global__ void __launch_bounds__(256) skinny_combine_kernel(const uint16_t* __restrict__ yg,
                                                             const int32_t* __restrict__ inv_pos,
                                                             const float* __restrict__ w, uint16_t* __restrict__ y,
                                                             int m, int k, int h) {
  const int t = blockIdx.y;
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= h || t >= m) return;
  float acc = 0.f;
  for (int s = 0; s < k; ++s) {
    const int a = t * k + s;
    const int p = inv_pos[a];
    if (p < 0) continue;
    const float wb = bf16_f32(f32_bf16(w[a]));
    const float v = bf16_f32(f32_bf16(bf16_f32(yg[(int64_t)p * h + c]) * wb));
    acc = bf16_f32(f32_bf16(acc + v));
  }
  y[(int64_t)t * h + c] = f32_bf16(acc);
}

}  // namespace
}  // namespace mosaic

using namespace mosaic;

extern "C" size_t mosaic_mx_kn_linear_a16_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0) return 0;
  const int ns = kn_steps(n, k, (m + 15) / 16);
  const int64_t ks = (k + 32 * ns - 1) / (32 * ns);
  return ks > 1 ? (size_t)ks * m * n * 4 : 0;
}

extern "C" int mosaic_mx_kn_linear_a16(const uint16_t* x, const uint8_t* packed, const uint8_t* scale, uint16_t* y,
                                       int64_t m, int64_t n, int64_t k, void* workspace, size_t workspace_bytes,
                                       void* stream) {
  MOSAIC_CHECK_ARG(x && packed && scale && y, "mx_kn_linear_a16: null pointer");
  MOSAIC_CHECK_ARG(n > 0 && n % 32 == 0 && k > 0 && k % 32 == 0,
                   "mx_kn_linear_a16: N=%lld and K=%lld must be positive multiples of 32", (long long)n, (long long)k);
  MOSAIC_CHECK_ARG(m >= 0 && m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 31), "mx_kn_linear_a16: shape");
  if (m == 0) return kOk;
  const int64_t mt = (m + 15) / 16;
  MOSAIC_CHECK_ARG(mt <= 65535, "mx_kn_linear_a16: m=%lld too large", (long long)m);
  return launch_kn(x, nullptr, packed, scale, 0, 0, KnTiles{nullptr, nullptr, nullptr, nullptr}, mt, (float*)workspace,
                   workspace_bytes, y, m, n, k, kn_steps(n, k, mt), (hipStream_t)stream);
}

namespace {

// fused_moe_skinny workspace: the layout arrays of the MoE workspace (its z
// holds the bf16 SwiGLU output, its fp32 partial buffer the bf16 down
// outputs), gate/up outputs bf16 [A, 2 inter], fp32 split-K partials.
struct SkinnyWs {
  MoeWorkspace lw;
  uint16_t* gu;
  float* part;
  int ns_gu, ns_d;
  size_t bytes;
};

SkinnyWs carve_skinny(char* base, int64_t m, int64_t h, int64_t inter, int64_t e, int64_t k) {
  SkinnyWs w{};
  w.lw = carve_moe_workspace(base, m, h, inter, e, k, 0, kMoeBlockM, false);
  const int64_t a = m * k;
  size_t off = w.lw.bytes;
  w.gu = base ? (uint16_t*)(base + off) : nullptr;
  off += align256((size_t)a * 2 * inter * 2);
  w.ns_gu = kn_steps(2 * inter, h, w.lw.tile_cap);
  w.ns_d = kn_steps(h, inter, w.lw.tile_cap);
  const int64_t ks_gu = (h + 32 * w.ns_gu - 1) / (32 * w.ns_gu), ks_d = (inter + 32 * w.ns_d - 1) / (32 * w.ns_d);
  size_t pb = 0;
  if (ks_gu > 1) pb = (size_t)ks_gu * a * 2 * inter * 4;
  if (ks_d > 1 && (size_t)ks_d * a * h * 4 > pb) pb = (size_t)ks_d * a * h * 4;
  w.part = (base && pb) ? (float*)(base + off) : nullptr;
  off += align256(pb);
  w.bytes = off;
  return w;
}

}  // namespace

extern "C" size_t mosaic_moe_skinny_workspace_bytes(int64_t m, int64_t hidden, int64_t inter, int64_t n_experts,
                                                    int64_t top_k) {
  if (m <= 0 || hidden <= 0 || inter <= 0 || n_experts <= 0 || top_k <= 0) return 0;
  return carve_skinny(nullptr, m, hidden, inter, n_experts, top_k).bytes;
}

extern "C" int mosaic_moe_skinny_forward(const uint16_t* x, const int32_t* ids, const float* weights,
                                         const uint8_t* gu_packed, const uint8_t* gu_scale, const uint8_t* d_packed,
                                         const uint8_t* d_scale, uint16_t* y, int64_t m, int64_t hidden,
                                         int64_t inter, int64_t n_experts, int64_t top_k, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  MOSAIC_CHECK_ARG(x && ids && weights && gu_packed && gu_scale && d_packed && d_scale && y && workspace,
                   "moe_skinny_forward: null pointer");
  MOSAIC_CHECK_ARG(m >= 1 && top_k >= 1 && top_k <= 16 && n_experts >= 1 && n_experts <= 512,
                   "moe_skinny_forward: m=%lld top_k=%lld", (long long)m, (long long)top_k);
  MOSAIC_CHECK_ARG(hidden % 32 == 0 && inter % 32 == 0 && hidden > 0 && inter > 0,
                   "moe_skinny_forward: hidden and inter must be multiples of 32");
  SkinnyWs w = carve_skinny((char*)workspace, m, hidden, inter, n_experts, top_k);
  MOSAIC_CHECK_ARG(w.lw.tile_cap <= 65535, "moe_skinny_forward: %lld tiles", (long long)w.lw.tile_cap);
  MOSAIC_CHECK_ARG(workspace_bytes >= w.bytes, "moe_skinny_forward: workspace %zu < %zu bytes", workspace_bytes,
                   w.bytes);
  hipStream_t st = (hipStream_t)stream;
  const MoeWorkspace& l = w.lw;
  LayoutOut lo{l.counts, l.offsets, l.perm, l.perm_token, l.perm_weight, l.sorted_ids, l.inv_pos, l.combine_pos,
               l.tile_expert, l.tile_start, l.tile_rows, l.tile_p0, l.n_tiles, nullptr, 0, 0,
               l.chunk_counts, l.chunk_base};
  int rc = launch_route_layout(nullptr, nullptr, ids, weights, nullptr, nullptr, m, n_experts, top_k, 0, 0, 1.0f, 0,
                               kMoeBlockM, l.tile_cap, lo, st);
  if (rc != 0) return rc;
  const int64_t a = m * top_k;
  const KnTiles tl{l.tile_expert, l.tile_rows, l.tile_p0, l.n_tiles};
  // gate|up: rows of x gathered by token, outputs at sorted positions
  rc = launch_kn(x, l.perm_token, gu_packed, gu_scale, hidden * inter, hidden * (2 * inter / 32), tl, l.tile_cap,
                 w.part, (size_t)-1, w.gu, a, 2 * inter, hidden, w.ns_gu, st);
  if (rc != 0) return rc;
  MOSAIC_LAUNCH(skinny_swiglu_kernel, dim3((unsigned)((a * inter + 255) / 256)), dim3(256), 0, st, w.gu, l.z, a,
                     (int)inter);
  MOSAIC_LAUNCH_CHECK("moe_skinny_swiglu");
  uint16_t* yg = reinterpret_cast<uint16_t*>(l.yp);
  rc = launch_kn(l.z, nullptr, d_packed, d_scale, inter * hidden / 2, inter * (hidden / 32), tl, l.tile_cap, w.part,
                 (size_t)-1, yg, a, hidden, inter, w.ns_d, st);
  if (rc != 0) return rc;
  MOSAIC_LAUNCH(skinny_combine_kernel, dim3((unsigned)((hidden + 255) / 256), (unsigned)m), dim3(256), 0, st, yg,
                     l.inv_pos, weights, y, (int)m, (int)top_k, (int)hidden);
  MOSAIC_RETURN_LAUNCH("moe_skinny_combine");
}
