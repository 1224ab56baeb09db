// Test-only probe kernels (built into tests/probes/libxtu_probes.so, not the
// product library): in-bounds checks of the device builtins the product
// kernels rely on -- converter byte/nibble order and scale handling, MFMA
// operand/result lane layouts, the fixed-sequence exp -- against host-side
// expectations in tests/test_gpu_probes.py.
#include "weight_format.hpp"

namespace xtu {
namespace {

__global__ void probe_fp4_kernel(const float* __restrict__ scales, int nscale,
                                 uint32_t* __restrict__ out) {
  // out[s*256 + b] = bf16 pair of byte b converted with scales[s]
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nscale * 256) return;
  const int s = i / 256, b = i % 256;
  uint32_t words[4];
  fp4x8_to_bf16((uint32_t)b, scales[s], words);
  out[i] = words[0];
}

__global__ void probe_fp4_mul_kernel(const float* __restrict__ scales, int nscale,
                                     uint32_t* __restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nscale * 256) return;
  const int s = i / 256, b = i % 256;
  uint32_t words[4];
  fp4x8_to_bf16_mul((uint32_t)b, scales[s], words);
  out[i] = words[0];
}

__global__ void probe_fp8_kernel(uint32_t* __restrict__ out) {
  // out[b] = bf16 of e4m3 byte b in the low half
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= 256) return;
  u32x4_t w = {(uint32_t)b, 0u, 0u, 0u};
  uint32_t words[8];
  fp8x16_to_bf16(w, words);
  out[b] = words[0];
}

// one wave: C[16][16] = A[16][32] * B[32][16] with this library's lane
// conventions (A lane l: row l%16, k 8*(l/16)+i; B lane l: col l%16, same k;
// C lane l: rows 4*(l/16)+i, col l%16)
__global__ void probe_mfma16_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                                    float* __restrict__ C) {
  const int l = threadIdx.x;
  uint32_t av[4], bv[4];
  for (int j = 0; j < 4; ++j) {
    const int k = 8 * (l / 16) + 2 * j;
    av[j] = (uint32_t)A[(l % 16) * 32 + k] | ((uint32_t)A[(l % 16) * 32 + k + 1] << 16);
    bv[j] = (uint32_t)B[k * 16 + (l % 16)] | ((uint32_t)B[(k + 1) * 16 + (l % 16)] << 16);
  }
  f32x4_t c = {0.f, 0.f, 0.f, 0.f};
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av[0], av[1], av[2], av[3]),
                                             as_bf16x8(bv[0], bv[1], bv[2], bv[3]), c, 0, 0, 0);
  for (int i = 0; i < 4; ++i) C[(4 * (l / 16) + i) * 16 + (l % 16)] = c[i];
}

// one wave: C[32][32] = A[32][16] * B[16][32]; A lane l: row l%32, k 8*(l/32)+i;
// C lane l: col l%32, rows 8*(i/4) + 4*(l/32) + i%4
__global__ void probe_mfma32_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                                    float* __restrict__ C) {
  const int l = threadIdx.x;
  uint32_t av[4], bv[4];
  for (int j = 0; j < 4; ++j) {
    const int k = 8 * (l / 32) + 2 * j;
    av[j] = (uint32_t)A[(l % 32) * 16 + k] | ((uint32_t)A[(l % 32) * 16 + k + 1] << 16);
    bv[j] = (uint32_t)B[k * 32 + (l % 32)] | ((uint32_t)B[(k + 1) * 32 + (l % 32)] << 16);
  }
  f32x16_t c;
  for (int i = 0; i < 16; ++i) c[i] = 0.f;
  c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(av[0], av[1], av[2], av[3]),
                                             as_bf16x8(bv[0], bv[1], bv[2], bv[3]), c, 0, 0, 0);
  for (int i = 0; i < 16; ++i)
    C[(8 * (i / 4) + 4 * (l / 32) + (i % 4)) * 32 + (l % 32)] = c[i];
}

// one wave: int32 C[32][32] = A[32][32] * B[32][32] (int8), k 16*(l/32)+i
__global__ void probe_mfma_i8_kernel(const int8_t* __restrict__ A, const int8_t* __restrict__ B,
                                     int32_t* __restrict__ C) {
  const int l = threadIdx.x;
  int8_t a[16], b[16];
  for (int i = 0; i < 16; ++i) {
    const int k = 16 * (l / 32) + i;
    a[i] = A[(l % 32) * 32 + k];
    b[i] = B[k * 32 + (l % 32)];
  }
  i32x4_t av = __builtin_bit_cast(i32x4_t, a);
  i32x4_t bv = __builtin_bit_cast(i32x4_t, b);
  i32x16_t c;
  for (int i = 0; i < 16; ++i) c[i] = 0;
  c = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, c, 0, 0, 0);
  for (int i = 0; i < 16; ++i)
    C[(8 * (i / 4) + 4 * (l / 32) + (i % 4)) * 32 + (l % 32)] = c[i];
}

__global__ void probe_exp_kernel(const float* __restrict__ x, int n, float* __restrict__ e,
                                 float* __restrict__ s) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  e[i] = xtu_expf(x[i]);
  s[i] = xtu_sigmoid(x[i]);
}

typedef int i32x8_t __attribute__((ext_vector_type(8)));

// one wave: raw per-lane operands and scale bytes of one
// v_mfma_scale_f32_16x16x128_f8f6f4 with an fp8 (e4m3) A and an fp4 (e2m1)
// B; C lane l holds rows 4*(l/16)+i of column l%16
__global__ void probe_mfma_scaled_fp4b_kernel(const int* __restrict__ A, const int* __restrict__ B,
                                              const uint8_t* __restrict__ sa,
                                              const uint8_t* __restrict__ sb,
                                              float* __restrict__ C) {
  const int l = threadIdx.x;
  i32x8_t a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = A[l * 8 + i];
    b[i] = B[l * 8 + i];
  }
  f32x4_t c = {0.f, 0.f, 0.f, 0.f};
  c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 4, 0, sa[l], 0, sb[l]);
  for (int i = 0; i < 4; ++i) C[l * 4 + i] = c[i];
}

}  // namespace
}  // namespace xtu

using namespace xtu;

extern "C" {

hipError_t xtu_probe_fp4(const float* scales, int nscale, uint32_t* out, hipStream_t stream) {
  XTU_CHECK_ARG(scales && out && nscale > 0 && nscale <= 4096);
  (void)hipGetLastError();
  probe_fp4_kernel<<<(nscale * 256 + 255) / 256, 256, 0, stream>>>(scales, nscale, out);
  return hipPeekAtLastError();
}

hipError_t xtu_probe_fp4_mul(const float* scales, int nscale, uint32_t* out, hipStream_t stream) {
  XTU_CHECK_ARG(scales && out && nscale > 0 && nscale <= 4096);
  (void)hipGetLastError();
  probe_fp4_mul_kernel<<<(nscale * 256 + 255) / 256, 256, 0, stream>>>(scales, nscale, out);
  return hipPeekAtLastError();
}

hipError_t xtu_probe_fp8(uint32_t* out, hipStream_t stream) {
  XTU_CHECK_ARG(out);
  (void)hipGetLastError();
  probe_fp8_kernel<<<1, 256, 0, stream>>>(out);
  return hipPeekAtLastError();
}

hipError_t xtu_probe_mfma(int which, const void* A, const void* B, void* C, hipStream_t stream) {
  XTU_CHECK_ARG(A && B && C && which >= 0 && which <= 2);
  (void)hipGetLastError();
  if (which == 0)
    probe_mfma16_kernel<<<1, 64, 0, stream>>>((const uint16_t*)A, (const uint16_t*)B, (float*)C);
  else if (which == 1)
    probe_mfma32_kernel<<<1, 64, 0, stream>>>((const uint16_t*)A, (const uint16_t*)B, (float*)C);
  else
    probe_mfma_i8_kernel<<<1, 64, 0, stream>>>((const int8_t*)A, (const int8_t*)B, (int32_t*)C);
  return hipPeekAtLastError();
}

hipError_t xtu_probe_mfma_scaled_fp4b(const int* A, const int* B, const uint8_t* sa,
                                     const uint8_t* sb, float* C, hipStream_t stream) {
  XTU_CHECK_ARG(A && B && sa && sb && C);
  (void)hipGetLastError();
  probe_mfma_scaled_fp4b_kernel<<<1, 64, 0, stream>>>(A, B, sa, sb, C);
  return hipPeekAtLastError();
}

hipError_t xtu_probe_exp(const float* x, int n, float* e, float* s, hipStream_t stream) {
  XTU_CHECK_ARG(n >= 0 && (n == 0 || (x && e && s)));
  if (n == 0) return hipSuccess;
  (void)hipGetLastError();
  probe_exp_kernel<<<(n + 255) / 256, 256, 0, stream>>>(x, n, e, s);
  return hipPeekAtLastError();
}

}  // extern "C"
