// Shared device helpers for the gfx950 (CDNA4) MoE expert-path kernels.
//
// Storage conventions used by every kernel in this library:
//   * bf16 values travel as raw uint16_t (round-to-nearest-even on writes);
//   * weights sit in HBM in the "P16" panel layout built once at weight load:
//       a [N rows][K] matrix is cut into panels of 16 rows; each panel into
//       super-blocks of 4 x 16 bytes along K per row; the 1 KiB of one
//       (panel, super-block) is stored [4 chunk q][16 row r][16 byte], so one
//       wave64 reading 16 bytes per lane (lane = 16*q + r) fetches one
//       contiguous KiB.  A chunk is 32 e2m1 codes (fp4), 16 e4m3 bytes (fp8)
//       or 8 bf16 values;
//   * fp4 scales: e8m0 [N/16][K/128][4 q][16 r] (MXFP4, one per 32 k) or e4m3
//     [N/16][K/128][4 q][16 r][2] (NVFP4, one per 16 k) -- the lane that reads
//     a weight chunk reads its scale(s) at the same (q, r);
//   * fp8 block scales stay [N/128][K/128] fp32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace xtu {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

enum WeightFormat : int { kBF16 = 0, kFP8 = 1, kMXFP4 = 2, kNVFP4 = 3 };

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// e4m3fn byte -> fp32 (normal: exponent rebias by +120; subnormal m * 2^-9).
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
  const uint32_t e = (b >> 3) & 15u, m = b & 7u;
  float v = (e == 0) ? (float)m * 1.953125e-03f : __uint_as_float(((e + 120u) << 23) | (m << 20));
  return (b & 0x80u) ? -v : v;
}

// e8m0 byte -> 2^(b-127) as fp32 (b = 0 gives 2^-127, a subnormal; b = 255 inf).
__device__ __forceinline__ float e8m0_to_f32(uint32_t b) {
  b &= 255u;
  const float v = __uint_as_float(b << 23);   // 255 -> +inf
  return b == 0 ? __uint_as_float(0x00400000u) : v;
}

// ---------------------------------------------------------------------------
// exp / sigmoid with a fixed fp32 operation sequence (bit-reproducible on the
// host).  Cody-Waite reduction x = k*ln2 + r, degree-7 Taylor polynomial in r
// by fused multiply-add Horner steps, scale by 2^k through two exponent-field
// factors.  Contraction is disabled so the compiler cannot fuse other steps.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float xtu_expf(float x) {
#pragma clang fp contract(off)
  if (!(x == x)) return x;
  if (x > 88.5f) return __uint_as_float(0x7f800000u);
  if (x < -87.0f) return 0.0f;
  const float kLog2e = 1.44269504088896341f;
  const float kLn2Hi = 0.693145751953125f;
  const float kLn2Lo = 1.42860682030941723e-06f;
  const float k = __builtin_rintf(x * kLog2e);
  float r = __builtin_fmaf(-k, kLn2Hi, x);
  r = __builtin_fmaf(-k, kLn2Lo, r);
  float p = 1.98412698412698413e-04f;
  p = __builtin_fmaf(p, r, 1.38888888888888889e-03f);
  p = __builtin_fmaf(p, r, 8.33333333333333333e-03f);
  p = __builtin_fmaf(p, r, 4.16666666666666667e-02f);
  p = __builtin_fmaf(p, r, 1.66666666666666667e-01f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const int ki = (int)k;
  const int k1 = ki / 2, k2 = ki - k1;
  const float s1 = __uint_as_float((uint32_t)(k1 + 127) << 23);
  const float s2 = __uint_as_float((uint32_t)(k2 + 127) << 23);
  return (p * s1) * s2;
}

__device__ __forceinline__ float xtu_sigmoid(float x) {
#pragma clang fp contract(off)
  return __fdiv_rn(1.0f, 1.0f + xtu_expf(-x));
}

// Clamped gated SiLU of the expert MLP: gate clamped above only, up on both
// sides (limit <= 0 disables), act = g * sigmoid(alpha*g) * (u + beta).
__device__ __forceinline__ float silu_gate(float g, float u, float limit, float alpha,
                                           float beta) {
  if (limit > 0.f) {
    g = fminf(g, limit);
    u = fminf(fmaxf(u, -limit), limit);
  }
  return (g / (1.f + __expf(-alpha * g))) * (u + beta);
}

// ---------------------------------------------------------------------------
// Chunk dequantisation to bf16 pairs on gfx950's scaled converters.
// Each returns 16 packed dwords (32 bf16) for fp4, or 8 for fp8.
// ---------------------------------------------------------------------------

// 8 e2m1 codes in one dword (byte b holds k = 2b (low nibble), 2b+1) times a
// power-of-two `scale` -> 4 dwords of bf16 pairs in k order.
__device__ __forceinline__ void fp4x8_to_bf16(uint32_t w, float scale, uint32_t* out) {
  out[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0));
  out[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1));
  out[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2));
  out[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3));
}

// 32 e2m1 codes (16 bytes, low nibble = even k) times `scale` -> 32 bf16.
__device__ __forceinline__ void fp4x32_to_bf16(const u32x4_t w, float scale, uint32_t out[16]) {
#pragma unroll
  for (int d = 0; d < 4; ++d) fp4x8_to_bf16(w[d], scale, out + 4 * d);
}

// 8 e2m1 codes times an arbitrary fp32 `scale` whose products are exact in
// bf16 (NVFP4: 2-bit x 4-bit significands): decode to fp32, multiply, keep the
// high half (exact because the product is representable).
__device__ __forceinline__ void fp4x8_to_bf16_mul(uint32_t w, float scale, uint32_t* out) {
  f32x2_t v0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 0);
  f32x2_t v1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 1);
  f32x2_t v2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 2);
  f32x2_t v3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 3);
  const f32x2_t vv[4] = {v0, v1, v2, v3};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = __float_as_uint(vv[i][0] * scale);
    const uint32_t hi = __float_as_uint(vv[i][1] * scale);
    out[i] = (lo >> 16) | (hi & 0xffff0000u);
  }
}

// NVFP4: the first 16 codes (bytes 0..7) use s0, the last 16 use s1.
__device__ __forceinline__ void fp4x32_to_bf16_2s(const u32x4_t w, float s0, float s1,
                                                  uint32_t out[16]) {
#pragma unroll
  for (int d = 0; d < 4; ++d) fp4x8_to_bf16_mul(w[d], d < 2 ? s0 : s1, out + 4 * d);
}

// 16 e4m3 bytes -> 16 bf16 (exact).
__device__ __forceinline__ void fp8x16_to_bf16(const u32x4_t w, uint32_t out[8]) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    bf16x2_t lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[d], 1.0f, false);
    bf16x2_t hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[d], 1.0f, true);
    out[d * 2 + 0] = __builtin_bit_cast(uint32_t, lo);
    out[d * 2 + 1] = __builtin_bit_cast(uint32_t, hi);
  }
}

__device__ __forceinline__ bf16x8_t as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  u32x4_t v = {a, b, c, d};
  return __builtin_bit_cast(bf16x8_t, v);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(const u32x4_t v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

}  // namespace xtu

#define XTU_CHECK_ARG(cond)                 \
  do {                                      \
    if (!(cond)) return hipErrorInvalidValue; \
  } while (0)
