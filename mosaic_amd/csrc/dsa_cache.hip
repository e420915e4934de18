// DSA decode-step plumbing around the indexer and MLA decode:
//
// KV-cache writer (the kv rows of ExactAttention.forward / attention_core,
// mosaicvm/model/dsa_layers.py:550-553 and 579-582, stored as _core_body does
// at :510-534): a kv row is [d - rope non-rope dims | rope dims], bf16.  The
// non-rope dims go through act_quant_sim (mosaicvm/model/dsa.py:81-93): per 64
// values, s = 2^ceil(log2(max(amax, 1e-4) / 448)) (the quotient rounded once
// to fp32, the ceiling taken on its IEEE bits), codes = e4m3(clamp(x / s,
// +-448)) with torch's round-to-nearest-even cast; the stored value is
// e4m3 * s, exact in bf16.  The rope dims are kept as they are.  Two cache
// layouts:
//   bf16 cache [n, d]: the reference's own (kv_cache buffer, dsa_layers.py:397),
//     row = bf16(codes * s) | rope;
//   fp8 cache: codes [n, d - rope] e4m3, scales [n, (d - rope) / 64] fp32 and
//     rope [n, rope] bf16 -- the layout mosaic_mla_sparse_decode reads (it
//     decodes e4m3 * s to bf16, the same values).
// One wave per row: lanes 8b .. 8b + 7 own block b, 8 values each.
//
// Decode gather indices (window_topk_idxs and compress_topk_idxs_static,
// mosaicvm/model/dsa.py:185-212, concatenated as _core_body does at :479-481):
// per query row at absolute position p, the window part lists the ring slots
// of positions max(0, p - window + 1) .. p oldest first (slot = position %
// window; -1 pads rows with fewer than window positions), and the compressed
// part is either the row's indexer picks (already offset past the window) or
// the static list offset .. offset + (p + 1) / ratio - 1, -1 padded.
#include "common.h"
#include "../../include/mosaic_amd.h"

namespace mosaic {
namespace {

constexpr int kKvBlock = 64;

// 2^ceil(log2(max(amax, 1e-4) / 448)) with the quotient rounded once to fp32
__device__ __forceinline__ float kv_scale_pow2(float amax) {
  const float v = fmaxf(amax, 1e-4f) / 448.0f;
  const uint32_t vb = __float_as_uint(v);
  const int e = (int)((vb >> 23) & 0xFFu) - 127 + ((vb & 0x7FFFFFu) != 0u ? 1 : 0);
  return __uint_as_float((uint32_t)(e + 127) << 23);
}

// max over the 8 lanes of each aligned group (pair, quad, half-row mirrors)
__device__ __forceinline__ float group8_max(float v) {
  v = fmaxf(v, __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(v), 0xB1, 0xF)));
  v = fmaxf(v, __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(v), 0x4E, 0xF)));
  return fmaxf(v, __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(v), 0x141, 0xF)));
}

// grid: rows / 4 workgroups of 4 waves, one row a wave
__global__ void __launch_bounds__(256) dsa_kv_write_kernel(const uint16_t* __restrict__ kv,
                                                           const int32_t* __restrict__ slots, int rows, int d,
                                                           int rope, int n, uint16_t* __restrict__ cache_bf16,
                                                           uint8_t* __restrict__ codes, float* __restrict__ scales,
                                                           uint16_t* __restrict__ rope_cache) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int slot = slots ? slots[r] : r;
  if (slot < 0 || slot >= n) return;
  const int dn = d - rope, nb = dn / kKvBlock;
  const uint16_t* src = kv + (int64_t)r * d;
  const int blk = lane >> 3, col = kKvBlock * blk + 8 * (lane & 7);
  const bool act = blk < nb;
  u32x4_t raw = {0u, 0u, 0u, 0u};
  if (act) raw = *reinterpret_cast<const u32x4_t*>(src + col);
  float x[8], amax = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = __uint_as_float(raw[i] << 16);
    x[2 * i + 1] = __uint_as_float(raw[i] & 0xFFFF0000u);
    amax = fmaxf(amax, fmaxf(fabsf(x[2 * i]), fabsf(x[2 * i + 1])));
  }
  amax = group8_max(amax);
  const float s = kv_scale_pow2(amax);
  const float inv = 1.0f / s;  // exact: s is a power of two
  uint32_t c[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) c[i] = e4m3_hw(fminf(fmaxf(x[i] * inv, -448.f), 448.f));
  if (act) {
    if (cache_bf16) {
      // codes * s in bf16: the e4m3 value scaled by a power of two is exact
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x2_t dv = __builtin_amdgcn_cvt_pk_f32_fp8((int)(c[2 * i] | (c[2 * i + 1] << 8)), false);
        w[i] = (__float_as_uint(dv[0] * s) >> 16) | (__float_as_uint(dv[1] * s) & 0xFFFF0000u);
      }
      *reinterpret_cast<u32x4_t*>(cache_bf16 + (int64_t)slot * d + col) = u32x4_t{w[0], w[1], w[2], w[3]};
    } else {
      const uint32_t lo = c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24);
      const uint32_t hi = c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24);
      *reinterpret_cast<uint2*>(codes + (int64_t)slot * dn + col) = uint2{lo, hi};
      if ((lane & 7) == 0) scales[(int64_t)slot * nb + blk] = s;
    }
  }
  // rope dims: copied (8 values a lane)
  for (int j = 8 * lane; j < rope; j += 512) {
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(src + dn + j);
    if (cache_bf16)
      *reinterpret_cast<u32x4_t*>(cache_bf16 + (int64_t)slot * d + dn + j) = v;
    else
      *reinterpret_cast<u32x4_t*>(rope_cache + (int64_t)slot * rope + j) = v;
  }
}

// one thread per output index: row = blockIdx.y
__global__ void __launch_bounds__(256) dsa_decode_indices_kernel(const int32_t* __restrict__ pos, int window,
                                                                 const int32_t* __restrict__ cidx, int nc, int ratio,
                                                                 int offset, int32_t* __restrict__ out) {
  const int r = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
  const int width = window + nc;
  if (i >= width) return;
  const int p = pos[r];
  int v;
  if (i < window) {
    // window slot i holds position q = p - window + 1 + i (oldest first)
    const int q = p - window + 1 + i;
    v = q >= 0 ? q % window : -1;
    // rows that have not filled the ring list positions 0 .. p first
    if (p < window - 1) v = i <= p ? i : -1;
  } else {
    const int j = i - window;
    if (cidx)
      v = cidx[(int64_t)r * nc + j];
    else
      v = j < (p + 1) / ratio ? offset + j : -1;
  }
  out[(int64_t)r * width + i] = v;
}

}  // namespace
}  // namespace mosaic

using namespace mosaic;

extern "C" int mosaic_dsa_kv_write(const uint16_t* kv, const int32_t* slots, int64_t rows, int64_t d, int64_t rope,
                                   int64_t n, uint16_t* cache_bf16, uint8_t* codes, float* scales,
                                   uint16_t* rope_cache, void* stream) {
  MOSAIC_CHECK_ARG(kv, "dsa_kv_write: null kv");
  MOSAIC_CHECK_ARG(rows >= 0 && rows < (1ll << 31) && n >= 0 && n < (1ll << 31), "dsa_kv_write: shape out of range");
  MOSAIC_CHECK_ARG(rope >= 0 && rope % 8 == 0 && rope <= 512 && d > rope && (d - rope) % kKvBlock == 0 &&
                       d - rope <= 8 * kKvBlock,
                   "dsa_kv_write: dims %lld (rope %lld): the non-rope part must be a multiple of 64, at most 512",
                   (long long)d, (long long)rope);
  MOSAIC_CHECK_ARG((cache_bf16 != nullptr) != (codes != nullptr),
                   "dsa_kv_write: give either the bf16 cache or the fp8 codes");
  MOSAIC_CHECK_ARG(cache_bf16 || (scales && (rope == 0 || rope_cache)), "dsa_kv_write: fp8 cache needs scales/rope");
  if (rows == 0) return kOk;
  MOSAIC_LAUNCH(dsa_kv_write_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, (hipStream_t)stream, kv,
                     slots, (int)rows, (int)d, (int)rope, (int)n, cache_bf16, codes, scales, rope_cache);
  MOSAIC_RETURN_LAUNCH("dsa_kv_write");
}

extern "C" int mosaic_dsa_decode_indices(const int32_t* pos, int64_t rows, int64_t window, const int32_t* cidx,
                                         int64_t nc, int64_t ratio, int64_t offset, int32_t* out, void* stream) {
  MOSAIC_CHECK_ARG(pos && out, "dsa_decode_indices: null pointer");
  MOSAIC_CHECK_ARG(rows >= 0 && rows <= 65535 && window >= 1 && nc >= 0 && window + nc < (1ll << 24),
                   "dsa_decode_indices: shape out of range");
  MOSAIC_CHECK_ARG(cidx || nc == 0 || ratio >= 1, "dsa_decode_indices: the static list needs ratio >= 1");
  MOSAIC_CHECK_ARG(offset >= 0 && offset < (1ll << 31), "dsa_decode_indices: offset out of range");
  if (rows == 0) return kOk;
  const int64_t width = window + nc;
  MOSAIC_LAUNCH(dsa_decode_indices_kernel, dim3((unsigned)((width + 255) / 256), (unsigned)rows), dim3(256), 0,
                     (hipStream_t)stream, pos, (int)window, cidx, (int)nc, (int)(ratio > 0 ? ratio : 1), (int)offset,
                     out);
  MOSAIC_RETURN_LAUNCH("dsa_decode_indices");
}
