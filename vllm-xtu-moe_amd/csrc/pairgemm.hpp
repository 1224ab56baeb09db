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

// ---------------------------------------------------------------------------
// Activation triples (pairgemm.hip, the double-rate fp6/fp4 MFMA).  A bf16
// block of 32 k is written as three pieces with one e8m0 byte s = e + 127,
//   x ~= 2^e (p1 + p2 / 16 + p3 / 256),
// p1, p2 e2m3 (fp6) and p3 e2m1 (fp4), each the round-to-nearest-even of
// the remainder left by the previous pieces (IEEE conversions: a negative
// value that rounds to zero is -0), scaled by 16: e is the
// smallest exponent with amax <= 7.5 * 2^e, so |x / 2^e| <= 7.5 and each
// remainder, at most half a grid step (<= 0.25), scales to <= 4.  The
// error is at most half a grid step of p3, 2^(e-9), below 2^-10.9 of the
// block maximum (typically 2^-14 of it).  A piece whose scale byte would
// fall below 0 (s < 4, s < 8: blocks below 2^-119) is zero.
// ---------------------------------------------------------------------------

// Exponent e of the triple scale 2^e: the smallest e with amax <= 7.5 * 2^e.
__device__ __forceinline__ int tri_exponent(float amax) {
  const uint32_t u = __float_as_uint(amax);
  const int ex = (int)((u >> 23) & 0xff);
  if (ex == 0) return -127;                 // zero or subnormal block
  int e = ex - 127 - 2 + ((u & 0x7fffffu) > 0x700000u ? 1 : 0);   // 7.5 = 1.875 * 2^2
  return e < -127 ? -127 : (e > 127 ? 127 : e);
}

// One 32-k block of bf16 values (64 bytes at src, 16-byte aligned) -> the
// pieces p1, p2 (6 dwords each, code j at bits 6j..6j+5) and p3 (4 dwords,
// code j at bits 4j..4j+3), the layout the 32x32x64 MFMA reads for an fp6 /
// fp4 A operand lane; returns the e8m0 byte s.  The roundings are the
// hardware's fp32 -> e2m3 / e2m1 conversions (round to nearest even, scale
// 1), the remainders exact fp32 arithmetic on the converted-back values.
__device__ __forceinline__ int tri_split32(const uint16_t* src, uint32_t p1[6], uint32_t p2[6],
                                           uint32_t p3[4]) {
  typedef float f32x16v __attribute__((ext_vector_type(16)));
  typedef float f32x32v __attribute__((ext_vector_type(32)));
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
  const int e = tri_exponent(amax);
  const int s = e + 127;
  // x / 2^e in two exact power-of-two steps (e may be -127)
  const float inv1 = pow2f(-(e / 2)), inv2 = pow2f(-(e - e / 2));
  // the 2 x 16 converter packs code 2i from its first operand's element i
  // and code 2i + 1 from its second's: even k first, odd k second
  float y[32];
#pragma unroll
  for (int j = 0; j < 32; ++j) y[j] = (v[j] * inv1) * inv2;
  auto to_fp6 = [&]() {
    f32x16v ev, od;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      ev[i] = y[2 * i];
      od[i] = y[2 * i + 1];
    }
    return __builtin_amdgcn_cvt_scalef32_2xpk16_fp6_f32(ev, od, 1.0f);
  };
  // remainder of each value after its rounded piece, times 16 (exact)
  auto next = [&](const f32x32v& q) {
#pragma unroll
    for (int j = 0; j < 32; ++j) y[j] = (y[j] - q[j]) * 16.f;
  };
  const auto c1 = to_fp6();
  next(__builtin_amdgcn_cvt_scalef32_pk32_f32_fp6(c1, 1.0f));
  const auto c2 = to_fp6();
  next(__builtin_amdgcn_cvt_scalef32_pk32_f32_fp6(c2, 1.0f));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t w = 0u;
    w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, y[8 * i + 0], y[8 * i + 1], 1.0f, 0);
    w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, y[8 * i + 2], y[8 * i + 3], 1.0f, 1);
    w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, y[8 * i + 4], y[8 * i + 5], 1.0f, 2);
    w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, y[8 * i + 6], y[8 * i + 7], 1.0f, 3);
    p3[i] = s >= 8 ? w : 0u;
  }
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    p1[i] = (uint32_t)c1[i];
    p2[i] = s >= 4 ? (uint32_t)c2[i] : 0u;
  }
  return s;
}

// ---------------------------------------------------------------------------
// pieces of the LDS-staged pair GEMM (pairgemm.hip)
// ---------------------------------------------------------------------------

// Memory-to-LDS loads (saddr form: a wave-uniform 64-bit base plus a 32-bit
// lane offset; M0 holds the LDS address that lane 0's bytes go to).  Written
// as asm so that the compiler does not make every later LDS read wait for
// all of them; the pipelines wait with explicit vmcnt counts and barriers.
__device__ __forceinline__ void dma16(const uint8_t* base, uint32_t off, const uint8_t* dst) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(off), "s"(base), "{m0}"((uint32_t)(uintptr_t)dst) : "memory");
}
__device__ __forceinline__ void dma4(const uint8_t* base, uint32_t off, const uint8_t* dst) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, %1"
               :: "v"(off), "s"(base), "{m0}"((uint32_t)(uintptr_t)dst) : "memory");
}

// s_waitcnt immediate for vmcnt(n) lgkmcnt(0) (gfx9 encoding: vmcnt in bits
// 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
__host__ __device__ constexpr int wait_vm_lgkm0(int n) {
  return 0x0070 | (n & 15) | ((n >> 4) << 14);
}

// LDS row stride of a tile's activation scales: K/32 bytes padded to an odd
// number of dwords (conflict-free byte reads of 32 consecutive rows), and the
// area of `rows` rows rounded up to whole 256-byte load chunks
__host__ __device__ constexpr int asc_stride(int K) { return ((K / 32 + 4) / 8) * 8 + 4; }
__host__ __device__ constexpr int asc_bytes(int K, int rows) {
  return (rows * asc_stride(K) + 255) / 256 * 256;
}

}  // namespace xtu
