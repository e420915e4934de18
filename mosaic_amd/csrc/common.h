// Shared device/host helpers for the gfx950 quantized-weight matrix path.
//
// Element formats (OCP MX): E2M1 nibbles packed two per byte, low nibble =
// even K; E8M0 scale byte b decodes to 2^(b-127) by writing b into the fp32
// exponent field; E4M3 is OCP e4m3fn (max 448, 0x7F/0xFF NaN).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mosaic {

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(2))) float f32x2_t;
typedef __attribute__((ext_vector_type(8))) int i32x8_t;
typedef __attribute__((ext_vector_type(4))) int i32x4_t;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4_t;

// ----------------------------------------------------------- status ABI ----
// 0 = OK, <0 = invalid argument, >0 = hipError_t of the failing launch.
enum : int { kOk = 0, kInvalid = -1, kUnsupported = -2, kTooLarge = -3 };

void set_last_error(const char* fmt, ...);

// Counts kernel launches made by this library on the calling thread
// (mosaic_launch_count); every launch site goes through MOSAIC_LAUNCH.
void note_launch();

#define MOSAIC_LAUNCH(...)         \
  do {                             \
    ::mosaic::note_launch();       \
    hipLaunchKernelGGL(__VA_ARGS__); \
  } while (0)

#define MOSAIC_CHECK_ARG(cond, ...)                     \
  do {                                                  \
    if (!(cond)) {                                      \
      ::mosaic::set_last_error(__VA_ARGS__);            \
      return ::mosaic::kInvalid;                        \
    }                                                   \
  } while (0)

#define MOSAIC_RETURN_LAUNCH(name)                                           \
  do {                                                                       \
    hipError_t _e = hipGetLastError();                                       \
    if (_e != hipSuccess) {                                                  \
      ::mosaic::set_last_error("%s: launch failed: %s", name,                \
                               hipGetErrorString(_e));                       \
      return (int)_e;                                                        \
    }                                                                        \
    return ::mosaic::kOk;                                                    \
  } while (0)

#define MOSAIC_LAUNCH_CHECK(name)                                            \
  do {                                                                       \
    hipError_t _e = hipGetLastError();                                       \
    if (_e != hipSuccess) {                                                  \
      ::mosaic::set_last_error("%s: launch failed: %s", name,                \
                               hipGetErrorString(_e));                       \
      return (int)_e;                                                        \
    }                                                                        \
  } while (0)

// ----------------------------------------------------------- bit helpers ---
__device__ __forceinline__ float bits_f32(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f32_bits(float f) { return __float_as_uint(f); }

// e8m0 byte -> fp32 2^(b-127) (0x00 -> 0.0, 0xFF -> +inf)
__device__ __forceinline__ float e8m0_f32(uint32_t b) { return __uint_as_float(b << 23); }

__device__ __forceinline__ float bf16_f32(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// fp32 -> bf16 bits, round-to-nearest-even (NaN kept quiet)
__device__ __forceinline__ uint16_t f32_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// LDS written by some lanes of a wave and read back by other lanes of the same
// wave, with no workgroup barrier between: wait for the wave's LDS operations
// and keep the compiler from moving the reads above the writes (without the
// fence it may, since another lane's write is invisible to the C++ model).
__device__ __forceinline__ void wave_lds_fence() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// 128-bit streaming load that bypasses cache allocation (read-once data)
__device__ __forceinline__ u32x4_t load_nt_u32x4(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
}

// 8-bit MFMA operand of one 128-byte K block for v_mfma_scale_f32_16x16x128_f8f6f4:
// lane (c = l%16, q = l/16) holds bytes [16q, 16q+16) and [64+16q, 64+16q+16)
// of row c (the same lane->K map on the A and B sides).
__device__ __forceinline__ i32x8_t load_fp8_operand(const uint8_t* __restrict__ row, int kb, int q) {
  const u32x4_t lo = *reinterpret_cast<const u32x4_t*>(row + (int64_t)kb * 128 + 16 * q);
  const u32x4_t hi = *reinterpret_cast<const u32x4_t*>(row + (int64_t)kb * 128 + 64 + 16 * q);
  return i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

__device__ __forceinline__ i32x8_t load_fp8_operand_nt(const uint8_t* __restrict__ row, int kb, int q) {
  const u32x4_t lo = load_nt_u32x4(row + (int64_t)kb * 128 + 16 * q);
  const u32x4_t hi = load_nt_u32x4(row + (int64_t)kb * 128 + 64 + 16 * q);
  return i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

// Two E2M1 nibbles of byte `sel` of `word` -> two bf16 scaled by `scale`
// (gfx950 v_cvt_scalef32_pk_bf16_fp4; low nibble -> element 0).
#define MOSAIC_CVT_FP4_BF16(word, scale, sel) \
  __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4((word), (scale), (sel))

// 16 packed bytes (32 E2M1 values, one MX block) -> 4 x bf16x8 scaled
__device__ __forceinline__ void mx_block_to_bf16(const u32x4_t w, float scale, bf16x8_t out[4]) {
  const uint32_t words[4] = {w[0], w[1], w[2], w[3]};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bf16x2_t p0 = MOSAIC_CVT_FP4_BF16(words[i], scale, 0);
    bf16x2_t p1 = MOSAIC_CVT_FP4_BF16(words[i], scale, 1);
    bf16x2_t p2 = MOSAIC_CVT_FP4_BF16(words[i], scale, 2);
    bf16x2_t p3 = MOSAIC_CVT_FP4_BF16(words[i], scale, 3);
    out[i][0] = p0[0]; out[i][1] = p0[1];
    out[i][2] = p1[0]; out[i][3] = p1[1];
    out[i][4] = p2[0]; out[i][5] = p2[1];
    out[i][6] = p3[0]; out[i][7] = p3[1];
  }
}

// fp32 -> e4m3fn byte, round to nearest even; beyond 448 after rounding, inf
// and NaN give 0x7F | sign (the behaviour of torch's float8_e4m3fn cast).
__device__ __forceinline__ uint32_t e4m3_rne(float v) {
  uint32_t u = __float_as_uint(v);
  uint32_t sign = (u >> 24) & 0x80u;
  float a = fabsf(v);
  if (!(a < 464.0f)) {
    if (a == 464.0f) return sign | 0x7Eu;  // tie between 448 and 480: even -> 448
    return sign | 0x7Fu;                   // overflow, inf, NaN
  }
  if (a < 0.015625f) {  // below 2^-6: subnormal step 2^-9
    float q = rintf(a * 512.0f);
    return sign | (uint32_t)q;
  }
  uint32_t au = __float_as_uint(a);
  int e = (int)(au >> 23) - 127;
  uint32_t mant = au & 0x7FFFFFu;
  uint32_t m3 = mant >> 20;
  uint32_t rem = mant & 0xFFFFFu;
  if (rem > 0x80000u || (rem == 0x80000u && (m3 & 1u))) m3++;
  if (m3 == 8u) { m3 = 0; e++; }
  uint32_t code = ((uint32_t)(e + 7) << 3) | m3;
  if (code > 0x7Eu) code = 0x7Fu;
  return sign | code;
}

// The same roundings on gfx950's converters (one instruction each).  Both
// round to nearest even; mosaic_selfcheck_converters compares them with the
// software versions above over every fp32 input (bf16: every non-NaN input;
// e4m3: every input after the clamp to [-448, 448] these callers apply).
__device__ __forceinline__ float bf16_round_hw(float f) {  // f finite or inf
  return (float)(__bf16)f;
}
__device__ __forceinline__ uint16_t f32_bf16_hw(float f) {  // f not NaN
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ uint32_t e4m3_hw(float v) {  // v in [-448, 448]
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v, v, 0, false) & 0xFFu;
}

// power-of-two 1x128 activation scale: 2^ceil(log2(max(amax, 1e-4) * fp32(1/448)))
// by IEEE bits (act_quant_ref, kernels/fp4_source.py:110-129)
__device__ __forceinline__ float act_scale_pow2(float amax) {
  const float a = fmaxf(amax, 1e-4f) * 0.002232142925783992f;  // fp32(1/448)
  const uint32_t ab = __float_as_uint(a);
  const int e = (int)((ab >> 23) & 0xFFu) - 127 + ((ab & 0x7FFFFFu) != 0u ? 1 : 0);
  return __uint_as_float((uint32_t)(e + 127) << 23);
}

// ---------------------------------------------------- DPP wave primitives ----
// gfx9 DPP controls: quad_perm [1,0,3,2] / [2,3,0,1], row_half_mirror,
// row_mirror, row_shr:n, row_bcast:15, row_bcast:31.
#define MOSAIC_DPP(old, v, ctrl, rmask) \
  ((uint32_t)__builtin_amdgcn_update_dpp((int)(old), (int)(v), (ctrl), (rmask), 0xF, false))

// max over the 64 lanes (all lanes active), broadcast to every lane
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, MOSAIC_DPP(0u, v, 0xB1, 0xF));
  v = max(v, MOSAIC_DPP(0u, v, 0x4E, 0xF));
  v = max(v, MOSAIC_DPP(0u, v, 0x141, 0xF));
  v = max(v, MOSAIC_DPP(0u, v, 0x140, 0xF));
  v = max(v, MOSAIC_DPP(0u, v, 0x142, 0xA));
  v = max(v, MOSAIC_DPP(0u, v, 0x143, 0xC));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

__device__ __forceinline__ float wave_max_f32(float v) {
  // order-preserving map of floats to unsigned (NaN-free input)
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  u = wave_max_u32(u);
  u = (u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u;
  return __uint_as_float(u);
}

// inclusive prefix sum over the 64 lanes (all lanes active)
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
  v += MOSAIC_DPP(0u, v, 0x111, 0xF);
  v += MOSAIC_DPP(0u, v, 0x112, 0xF);
  v += MOSAIC_DPP(0u, v, 0x114, 0xF);
  v += MOSAIC_DPP(0u, v, 0x118, 0xF);
  v += MOSAIC_DPP(0u, v, 0x142, 0xA);
  v += MOSAIC_DPP(0u, v, 0x143, 0xC);
  return v;
}

__device__ __forceinline__ uint32_t wave_bcast_u32(uint32_t v, int lane) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, lane);
}

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + __expf(-g)); }

__device__ __forceinline__ float swiglu_f32(float gate, float up, float limit) {
  if (limit > 0.f) {
    gate = fminf(gate, limit);
    up = fmaxf(fminf(up, limit), -limit);
  }
  return (gate / (1.0f + expf(-gate))) * up;
}

// The same SwiGLU on the hardware exp2 and reciprocal (a few ulp of fp32
// instead of correctly rounded expf and division; about 5 VALU instead of 25),
// for the prefill epilogues that evaluate 64 values a lane.  A large negative
// gate gives gate * rcp(inf) = -0, as the accurate form does.
__device__ __forceinline__ float swiglu_fast_f32(float gate, float up, float limit) {
  if (limit > 0.f) {
    gate = fminf(gate, limit);
    up = fmaxf(fminf(up, limit), -limit);
  }
  const float e = __builtin_amdgcn_exp2f(-gate * 1.4426950408889634f);
  return gate * __builtin_amdgcn_rcpf(1.0f + e) * up;
}

}  // namespace mosaic
