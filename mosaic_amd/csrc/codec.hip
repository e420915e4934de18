// Element-format kernels: MXFP4 dequant (through the same gfx950 FP4->bf16/f32
// converts the GEMMs use), MXFP4 quantizers (ceil and floor recipes), the
// 1xB E4M3 activation quantizer and an E4M3 decoder.
#include "common.h"
#include "../../include/mosaic_amd.h"

namespace mosaic {

// ------------------------------------------------------------- encoders ----
// E2M1 code from |q| (q already divided by the block scale), round to nearest
// even, saturating at 6; NaN -> 7.  Ties: .25->0 .75->1.0 1.25->1.0 1.75->2
// 2.5->2 3.5->4 5->4 (the even-mantissa neighbour).
__device__ __forceinline__ uint32_t e2m1_code_rne(float q) {
  uint32_t sign = (__float_as_uint(q) >> 28) & 0x8u;
  float a = fabsf(q);
  uint32_t c = 0;
  c = (a > 0.25f) ? 1u : c;
  c = (a >= 0.75f) ? 2u : c;
  c = (a > 1.25f) ? 3u : c;
  c = (a >= 1.75f) ? 4u : c;
  c = (a > 2.5f) ? 5u : c;
  c = (a >= 3.5f) ? 6u : c;
  c = (a > 5.0f) ? 7u : c;
  c = (a != a) ? 7u : c;
  return c | sign;
}

template <typename T> __device__ __forceinline__ float load_as_f32(const T* p, int64_t i);
template <> __device__ __forceinline__ float load_as_f32<float>(const float* p, int64_t i) { return p[i]; }
template <> __device__ __forceinline__ float load_as_f32<uint16_t>(const uint16_t* p, int64_t i) {
  return bf16_f32(p[i]);
}

// ------------------------------------------------------------- kernels -----
// One thread per (row, 32-element block).  recipe 0 = ceil (2^ceil(log2(amax/6))),
// recipe 1 = floor (2^(floor(log2 amax) - 2)).
template <typename T>
__global__ void __launch_bounds__(256) mx_quantize_kernel(const T* __restrict__ w, uint8_t* __restrict__ packed,
                                                          uint8_t* __restrict__ scale, int64_t n_blocks,
                                                          int64_t blocks_per_row, int recipe) {
  int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= n_blocks) return;
  const int64_t row = b / blocks_per_row;
  const int64_t kb = b % blocks_per_row;
  const int64_t base = row * blocks_per_row * 32 + kb * 32;
  float v[32];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    v[i] = load_as_f32<T>(w, base + i);
    amax = fmaxf(amax, fabsf(v[i]));  // fmaxf ignores NaN operands
  }
  bool any_nan = false;
#pragma unroll
  for (int i = 0; i < 32; ++i) any_nan |= (v[i] != v[i]);
  uint32_t biased;
  float s;
  if (recipe == 0) {
    float a = fmaxf(amax, 7.052966104933725e-38f);  // 6 * 2^-126
    float t = a * 0.16666667163372040f;            // fp32(1/6)
    uint32_t tb = __float_as_uint(t);
    int e = (int)((tb >> 23) & 0xFFu) - 127 + ((tb & 0x7FFFFFu) != 0u ? 1 : 0);
    biased = (uint32_t)(e + 127);
    s = __uint_as_float(biased << 23);
  } else {
    int e = (int)((__float_as_uint(amax) >> 23) & 0xFFu) - 127 - 2;
    e = e < -127 ? -127 : (e > 128 ? 128 : e);
    biased = any_nan ? 255u : (uint32_t)(e + 127);
    s = fmaxf(__uint_as_float(biased << 23), 1.1754943508222875e-38f);
  }
  uint32_t words[4] = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    float q = v[i] / s;
    if (recipe == 0) q = fminf(fmaxf(q, -6.0f), 6.0f);
    uint32_t c = e2m1_code_rne(q);
    words[i >> 3] |= c << (4 * (i & 7));
  }
  uint4* dst = reinterpret_cast<uint4*>(packed + row * blocks_per_row * 16 + kb * 16);
  *dst = make_uint4(words[0], words[1], words[2], words[3]);
  scale[row * blocks_per_row + kb] = (uint8_t)(biased & 0xFFu);
}

// One thread per MX block: 16 packed bytes + 1 scale byte -> 32 outputs, using
// the hardware FP4 converts (the same ones the GEMM kernels use).
__global__ void __launch_bounds__(256) mx_dequant_f32_kernel(const uint8_t* __restrict__ packed,
                                                             const uint8_t* __restrict__ scale,
                                                             float* __restrict__ out, int64_t n_blocks) {
  int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= n_blocks) return;
  const u32x4_t w = *reinterpret_cast<const u32x4_t*>(packed + b * 16);
  const float s = e8m0_f32(scale[b]);
  const uint32_t words[4] = {w[0], w[1], w[2], w[3]};
  float4* o = reinterpret_cast<float4*>(out + b * 32);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f32x2_t p0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[i], s, 0);
    f32x2_t p1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[i], s, 1);
    f32x2_t p2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[i], s, 2);
    f32x2_t p3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[i], s, 3);
    o[2 * i] = make_float4(p0[0], p0[1], p1[0], p1[1]);
    o[2 * i + 1] = make_float4(p2[0], p2[1], p3[0], p3[1]);
  }
}

__global__ void __launch_bounds__(256) mx_dequant_bf16_kernel(const uint8_t* __restrict__ packed,
                                                              const uint8_t* __restrict__ scale,
                                                              uint16_t* __restrict__ out, int64_t n_blocks) {
  int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= n_blocks) return;
  const u32x4_t w = *reinterpret_cast<const u32x4_t*>(packed + b * 16);
  const float s = e8m0_f32(scale[b]);
  bf16x8_t v[4];
  mx_block_to_bf16(w, s, v);
  bf16x8_t* o = reinterpret_cast<bf16x8_t*>(out + b * 32);
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = v[i];
}

// 1 x block activation quantizer: one wave per (row, block); lanes stride the block.
// mode 0: s = 2^ceil(log2(max(amax,1e-4) * fp32(1/448)))  (power of two)
// mode 1: s = max(amax,1e-4) * fp32(1/448)
// mode 2: s = amax / 448
// mode 3: s = amax / 448, and 1 where that is zero
template <typename T>
__global__ void __launch_bounds__(256) act_quant_kernel(const T* __restrict__ x, uint8_t* __restrict__ q,
                                                        float* __restrict__ s_out, int64_t rows, int64_t K,
                                                        int block, int mode) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t nb = K / block;
  if (wid >= rows * nb) return;
  const int64_t row = wid / nb, kb = wid % nb;
  const int64_t base = row * K + kb * block;
  float amax = 0.f;
  for (int i = lane; i < block; i += 64) amax = fmaxf(amax, fabsf(load_as_f32<T>(x, base + i)));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  float s;
  if (mode == 0) {
    s = act_scale_pow2(amax);
  } else if (mode == 1) {
    s = fmaxf(amax, 1e-4f) * 0.002232142925783992f;
  } else {
    s = amax / 448.0f;
    if (mode == 3 && s == 0.f) s = 1.0f;
  }
  // a power-of-two scale (mode 0) has an exact reciprocal: x * (1 / s) == x / s
  const float inv = mode == 0 ? 1.0f / s : 0.f;
  for (int i = lane; i < block; i += 64) {
    const float xv = load_as_f32<T>(x, base + i);
    float y = mode == 0 ? xv * inv : xv / s;
    y = fminf(fmaxf(y, -448.0f), 448.0f);
    q[base + i] = (uint8_t)e4m3_hw(y);
  }
  if (lane == 0) s_out[row * nb + kb] = s;
}

// 1x128 blocks, 16 lanes per block, 8 consecutive elements per lane (one
// 16- or 32-byte load, one 8-byte store); same arithmetic as act_quant_kernel.
template <typename T>
__device__ __forceinline__ void load8_f32(const T* p, float (&v)[8]);
template <>
__device__ __forceinline__ void load8_f32<uint16_t>(const uint16_t* p, float (&v)[8]) {
  const u32x4_t w = *reinterpret_cast<const u32x4_t*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
  }
}
template <>
__device__ __forceinline__ void load8_f32<float>(const float* p, float (&v)[8]) {
  const f32x4_t a = *reinterpret_cast<const f32x4_t*>(p), b = *reinterpret_cast<const f32x4_t*>(p + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[i] = a[i];
    v[4 + i] = b[i];
  }
}

template <typename T>
__global__ void __launch_bounds__(256) act_quant128_kernel(const T* __restrict__ x, uint8_t* __restrict__ q,
                                                           float* __restrict__ s_out, int64_t n_chunks, int mode) {
  const int64_t ch = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // 8-element chunk
  if (ch >= n_chunks) return;  // n_chunks is a multiple of 16: whole 16-lane groups leave together
  float v[8];
  load8_f32<T>(x + ch * 8, v);
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  // max over the chunk's 16-lane row on DPP moves (amax is never NaN: fmaxf drops NaN inputs)
  amax = fmaxf(amax, __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(amax), 0xB1, 0xF)));
  amax = fmaxf(amax, __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(amax), 0x4E, 0xF)));
  amax = fmaxf(amax, __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(amax), 0x141, 0xF)));
  amax = fmaxf(amax, __uint_as_float(MOSAIC_DPP(0u, __float_as_uint(amax), 0x140, 0xF)));
  float s;
  if (mode == 0) {
    s = act_scale_pow2(amax);
  } else if (mode == 1) {
    s = fmaxf(amax, 1e-4f) * 0.002232142925783992f;
  } else {
    s = amax / 448.0f;
    if (mode == 3 && s == 0.f) s = 1.0f;
  }
  // a power-of-two scale (mode 0) has an exact reciprocal: v * (1 / s) == v / s
  const float inv = mode == 0 ? 1.0f / s : 0.f;
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float y = mode == 0 ? v[i] * inv : v[i] / s;
    y = fminf(fmaxf(y, -448.0f), 448.0f);
    const uint32_t b = e4m3_hw(y);  // y clamped to [-448, 448] above
    if (i < 4) lo |= b << (8 * i);
    else hi |= b << (8 * (i - 4));
  }
  *reinterpret_cast<uint2*>(q + ch * 8) = uint2{lo, hi};
  if ((threadIdx.x & 15) == 0) s_out[ch / 16] = s;
}

// Every fp32 bit pattern once (grid-stride over 2^32): counts[0] = non-NaN
// inputs where bf16_round_hw differs from f32_bf16, counts[1] = inputs whose
// clamp to [-448, 448] encodes differently under e4m3_hw and e4m3_rne.
__global__ void __launch_bounds__(256) selfcheck_converters_kernel(unsigned long long* __restrict__ counts) {
  const uint64_t nt = (uint64_t)gridDim.x * blockDim.x;
  uint32_t bad_b = 0, bad_e = 0;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < (1ull << 32); i += nt) {
    const float f = __uint_as_float((uint32_t)i);
    if (f == f) {
      bad_b += __float_as_uint(bf16_round_hw(f)) != ((uint32_t)f32_bf16(f) << 16);
      const float y = fminf(fmaxf(f, -448.0f), 448.0f);
      bad_e += e4m3_hw(y) != e4m3_rne(y);
    }
  }
  if (bad_b) atomicAdd(&counts[0], (unsigned long long)bad_b);
  if (bad_e) atomicAdd(&counts[1], (unsigned long long)bad_e);
}

__global__ void __launch_bounds__(256) e4m3_decode_kernel(const uint8_t* __restrict__ in, float* __restrict__ out,
                                                          int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  f32x2_t v = __builtin_amdgcn_cvt_pk_f32_fp8((int)in[i], false);
  out[i] = v[0];
}

__global__ void __launch_bounds__(256) e4m3_encode_kernel(const float* __restrict__ in, uint8_t* __restrict__ out,
                                                          int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = (uint8_t)e4m3_rne(in[i]);
}


// ------------------------------------------------------- MXT16 prepack -----
// Tile layout for the 16-row MFMA tiles (bit-exact permutation of 16-byte MX
// blocks and of scale bytes; see mx_a16.hip):
//   packed_t[g][S][l][16 B] = packed[16g + l%16][16*(4S + l/16) .. +16]
//   scale_t [g][S4][l][s]   = scale[16g + l%16][4*(4*S4 + s) + l/16]  (0 past K)
// g = row group of 16, S = 128-K super-step, S4 = group of 4 super-steps.
__global__ void __launch_bounds__(256) mxt16_pack_kernel(const uint8_t* __restrict__ packed,
                                                         const uint8_t* __restrict__ scale, uint8_t* __restrict__ pt,
                                                         uint8_t* __restrict__ st, int64_t n_groups, int ns, int ns4,
                                                         int64_t kb, int inverse) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // one lane-slot
  const int64_t per_g = (int64_t)ns4 * 4 * 64;
  if (i >= n_groups * per_g) return;
  const int64_t g = i / per_g;
  const int64_t rem = i % per_g;
  const int S = (int)(rem / 64);
  const int l = (int)(rem % 64);
  const int c = l & 15, q = l >> 4;
  const int64_t row = 16 * g + c;
  const int blk = 4 * S + q;  // MX block index along K
  if (S < ns) {
    const int64_t src = row * (kb * 16) + (int64_t)blk * 16;
    const int64_t dst = (((int64_t)g * ns + S) * 64 + l) * 16;
    if (!inverse)
      *reinterpret_cast<u32x4_t*>(pt + dst) = *reinterpret_cast<const u32x4_t*>(packed + src);
    else
      *reinterpret_cast<u32x4_t*>(const_cast<uint8_t*>(packed) + src) = *reinterpret_cast<const u32x4_t*>(pt + dst);
  }
  const int S4 = S >> 2, s = S & 3;
  const int64_t sdst = (((int64_t)g * ns4 + S4) * 64 + l) * 4 + s;
  if (!inverse)
    st[sdst] = (S < ns) ? scale[row * kb + blk] : (uint8_t)0;
  else if (S < ns)
    const_cast<uint8_t*>(scale)[row * kb + blk] = st[sdst];
}

static inline unsigned grid1d(int64_t n, int threads) { return (unsigned)((n + threads - 1) / threads); }

}  // namespace mosaic

using namespace mosaic;

extern "C" int mosaic_mx_quantize(const void* w, int w_dtype, uint8_t* packed, uint8_t* scale, int64_t n,
                                  int64_t k, int recipe, void* stream) {
  MOSAIC_CHECK_ARG(w && packed && scale, "mx_quantize: null pointer");
  MOSAIC_CHECK_ARG(n >= 0 && k >= 0 && k % 32 == 0, "mx_quantize: K=%lld must be a multiple of 32", (long long)k);
  MOSAIC_CHECK_ARG(recipe == 0 || recipe == 1, "mx_quantize: recipe %d not in {0 ceil, 1 floor}", recipe);
  MOSAIC_CHECK_ARG(w_dtype == MOSAIC_DTYPE_F32 || w_dtype == MOSAIC_DTYPE_BF16, "mx_quantize: dtype %d", w_dtype);
  int64_t nb = n * (k / 32);
  if (nb == 0) return kOk;
  hipStream_t st = (hipStream_t)stream;
  if (w_dtype == MOSAIC_DTYPE_F32)
    MOSAIC_LAUNCH(mx_quantize_kernel<float>, dim3(grid1d(nb, 256)), dim3(256), 0, st, (const float*)w, packed,
                       scale, nb, k / 32, recipe);
  else
    MOSAIC_LAUNCH(mx_quantize_kernel<uint16_t>, dim3(grid1d(nb, 256)), dim3(256), 0, st, (const uint16_t*)w,
                       packed, scale, nb, k / 32, recipe);
  MOSAIC_RETURN_LAUNCH("mx_quantize");
}

extern "C" int mosaic_mx_dequant(const uint8_t* packed, const uint8_t* scale, void* out, int out_dtype, int64_t n,
                                 int64_t k, void* stream) {
  MOSAIC_CHECK_ARG(packed && scale && out, "mx_dequant: null pointer");
  MOSAIC_CHECK_ARG(n >= 0 && k >= 0 && k % 32 == 0, "mx_dequant: K=%lld must be a multiple of 32", (long long)k);
  int64_t nb = n * (k / 32);
  if (nb == 0) return kOk;
  hipStream_t st = (hipStream_t)stream;
  if (out_dtype == MOSAIC_DTYPE_F32)
    MOSAIC_LAUNCH(mx_dequant_f32_kernel, dim3(grid1d(nb, 256)), dim3(256), 0, st, packed, scale, (float*)out, nb);
  else if (out_dtype == MOSAIC_DTYPE_BF16)
    MOSAIC_LAUNCH(mx_dequant_bf16_kernel, dim3(grid1d(nb, 256)), dim3(256), 0, st, packed, scale,
                       (uint16_t*)out, nb);
  else
    MOSAIC_CHECK_ARG(false, "mx_dequant: out dtype %d", out_dtype);
  MOSAIC_RETURN_LAUNCH("mx_dequant");
}

extern "C" int mosaic_act_quant(const void* x, int x_dtype, uint8_t* q, float* s, int64_t m, int64_t k, int block,
                                int mode, void* stream) {
  MOSAIC_CHECK_ARG(x && q && s, "act_quant: null pointer");
  MOSAIC_CHECK_ARG(block > 0 && k % block == 0, "act_quant: K=%lld must be a multiple of block %d", (long long)k,
                   block);
  MOSAIC_CHECK_ARG(mode >= 0 && mode <= 3, "act_quant: mode %d", mode);
  MOSAIC_CHECK_ARG(x_dtype == MOSAIC_DTYPE_F32 || x_dtype == MOSAIC_DTYPE_BF16, "act_quant: dtype %d", x_dtype);
  int64_t waves = m * (k / block);
  if (waves == 0) return kOk;
  hipStream_t st = (hipStream_t)stream;
  if (block == 128 && ((uintptr_t)x & 15u) == 0 && ((uintptr_t)q & 7u) == 0) {
    const int64_t chunks = m * k / 8;
    const unsigned g = grid1d(chunks, 256);
    if (x_dtype == MOSAIC_DTYPE_F32)
      MOSAIC_LAUNCH(act_quant128_kernel<float>, dim3(g), dim3(256), 0, st, (const float*)x, q, s, chunks, mode);
    else
      MOSAIC_LAUNCH(act_quant128_kernel<uint16_t>, dim3(g), dim3(256), 0, st, (const uint16_t*)x, q, s, chunks,
                         mode);
    MOSAIC_RETURN_LAUNCH("act_quant");
  }
  unsigned grid = grid1d(waves * 64, 256);
  if (x_dtype == MOSAIC_DTYPE_F32)
    MOSAIC_LAUNCH(act_quant_kernel<float>, dim3(grid), dim3(256), 0, st, (const float*)x, q, s, m, k, block,
                       mode);
  else
    MOSAIC_LAUNCH(act_quant_kernel<uint16_t>, dim3(grid), dim3(256), 0, st, (const uint16_t*)x, q, s, m, k,
                       block, mode);
  MOSAIC_RETURN_LAUNCH("act_quant");
}

extern "C" int mosaic_selfcheck_converters(unsigned long long* counts, void* stream) {
  MOSAIC_CHECK_ARG(counts, "selfcheck_converters: null pointer");
  MOSAIC_LAUNCH(selfcheck_converters_kernel, dim3(4096), dim3(256), 0, (hipStream_t)stream, counts);
  MOSAIC_RETURN_LAUNCH("selfcheck_converters");
}

extern "C" int mosaic_e4m3_decode(const uint8_t* in, float* out, int64_t n, void* stream) {
  MOSAIC_CHECK_ARG(in && out, "e4m3_decode: null pointer");
  if (n == 0) return kOk;
  MOSAIC_LAUNCH(e4m3_decode_kernel, dim3(grid1d(n, 256)), dim3(256), 0, (hipStream_t)stream, in, out, n);
  MOSAIC_RETURN_LAUNCH("e4m3_decode");
}

extern "C" int mosaic_e4m3_encode(const float* in, uint8_t* out, int64_t n, void* stream) {
  MOSAIC_CHECK_ARG(in && out, "e4m3_encode: null pointer");
  if (n == 0) return kOk;
  MOSAIC_LAUNCH(e4m3_encode_kernel, dim3(grid1d(n, 256)), dim3(256), 0, (hipStream_t)stream, in, out, n);
  MOSAIC_RETURN_LAUNCH("e4m3_encode");
}

extern "C" int mosaic_mxt16_prepack(const uint8_t* packed, const uint8_t* scale, uint8_t* packed_t, uint8_t* scale_t,
                                    int64_t n, int64_t k, void* stream) {
  MOSAIC_CHECK_ARG(packed && scale && packed_t && scale_t, "mxt16_prepack: null pointer");
  MOSAIC_CHECK_ARG(n > 0 && n % 16 == 0, "mxt16_prepack: N=%lld must be a positive multiple of 16", (long long)n);
  MOSAIC_CHECK_ARG(k > 0 && k % 128 == 0, "mxt16_prepack: K=%lld must be a positive multiple of 128", (long long)k);
  const int ns = (int)(k / 128), ns4 = (ns + 3) / 4;
  const int64_t total = (n / 16) * (int64_t)ns4 * 4 * 64;
  MOSAIC_LAUNCH(mxt16_pack_kernel, dim3(grid1d(total, 256)), dim3(256), 0, (hipStream_t)stream, packed, scale,
                     packed_t, scale_t, n / 16, ns, ns4, k / 32, 0);
  MOSAIC_RETURN_LAUNCH("mxt16_prepack");
}

extern "C" int mosaic_mxt16_unpack(const uint8_t* packed_t, const uint8_t* scale_t, uint8_t* packed, uint8_t* scale,
                                   int64_t n, int64_t k, void* stream) {
  MOSAIC_CHECK_ARG(packed && scale && packed_t && scale_t, "mxt16_unpack: null pointer");
  MOSAIC_CHECK_ARG(n > 0 && n % 16 == 0, "mxt16_unpack: N=%lld must be a positive multiple of 16", (long long)n);
  MOSAIC_CHECK_ARG(k > 0 && k % 128 == 0, "mxt16_unpack: K=%lld must be a positive multiple of 128", (long long)k);
  const int ns = (int)(k / 128), ns4 = (ns + 3) / 4;
  const int64_t total = (n / 16) * (int64_t)ns4 * 4 * 64;
  MOSAIC_LAUNCH(mxt16_pack_kernel, dim3(grid1d(total, 256)), dim3(256), 0, (hipStream_t)stream, packed, scale,
                     const_cast<uint8_t*>(packed_t), const_cast<uint8_t*>(scale_t), n / 16, ns, ns4, k / 32, 1);
  MOSAIC_RETURN_LAUNCH("mxt16_unpack");
}
