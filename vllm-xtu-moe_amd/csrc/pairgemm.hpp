// Exact activation pairs (shared by fp8pair.hip and pairgemm.hip).
//
// A bf16 row is cut into blocks of 32 k and every block is written as two
// e4m3 vectors with one e8m0 scale sa,
//   x = hi * 2^(sa-127) + lo * 2^(sl-127),   sl = max(sa - 4, 0),
// sa putting the block maximum at <= 448 (the largest e4m3 normal), hi the
// round-to-nearest-even e4m3 of x / 2^(sa-127) and lo the e4m3 of 16x the
// remainder.
#pragma once
#include "weight_format.hpp"

namespace xtu {

// Exponent e of the block scale 2^e: the smallest e with amax / 2^e <= 448.
__device__ __forceinline__ int pair_exponent(float amax) {
  const uint32_t u = __float_as_uint(amax);
  const int ex = (int)((u >> 23) & 0xff);
  if (ex == 0) return -127;                 // zero or subnormal block
  int e = ex - 127 - 8 + ((u & 0x7fffffu) > 0x600000u ? 1 : 0);   // 448 = 1.75 * 2^8
  return e < -127 ? -127 : (e > 127 ? 127 : e);
}

__device__ __forceinline__ float pow2f(int e) {   // 2^e for e in [-126, 127]
  return __uint_as_float((uint32_t)(e + 127) << 23);
}

// One 32-k block of bf16 values (64 bytes at src, 16-byte aligned) -> hi and
// lo e4m3 codes (32 bytes each, k order) and the e8m0 byte sa.
__device__ __forceinline__ int pair_split32(const uint16_t* src, uint32_t hw[8], uint32_t lw[8]) {
  float v[32];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const u32x4_t p = *reinterpret_cast<const u32x4_t*>(src + 8 * j);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      v[8 * j + 2 * w] = __uint_as_float(p[w] << 16);
      v[8 * j + 2 * w + 1] = __uint_as_float(p[w] & 0xffff0000u);
    }
  }
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
  const int e = pair_exponent(amax);
  // x / 2^e in two exact power-of-two steps (e may be -127)
  const float inv1 = pow2f(-(e / 2)), inv2 = pow2f(-(e - e / 2));
#pragma unroll
  for (int j = 0; j < 32; j += 2) {
    const float a = (v[j] * inv1) * inv2, b = (v[j + 1] * inv1) * inv2;
    const int h = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    const float ra = (a - __builtin_amdgcn_cvt_f32_fp8(h, 0)) * 16.0f;
    const float rb = (b - __builtin_amdgcn_cvt_f32_fp8(h, 1)) * 16.0f;
    const int lv = __builtin_amdgcn_cvt_pk_fp8_f32(ra, rb, 0, false);
    const int wi = j / 4, sh = (j % 4) * 8;
    if ((j % 4) == 0) {
      hw[wi] = 0u;
      lw[wi] = 0u;
    }
    hw[wi] |= ((uint32_t)h & 0xffffu) << sh;
    lw[wi] |= ((uint32_t)lv & 0xffffu) << sh;
  }
  return e + 127;
}

}  // namespace xtu
