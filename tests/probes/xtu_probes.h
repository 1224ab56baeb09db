/*
 * xtu_probes.h -- test-only library (tests/probes/libxtu_probes.so): probe
 * kernels that check, in bounds, the device builtins the product kernels rely
 * on.  Not part of the product ABI (include/xtu_moe_amd.h).
 */
#ifndef XTU_PROBES_H
#define XTU_PROBES_H

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* scaled fp4/fp8 converters, MFMA lane layouts, the fixed-sequence
 * exp/sigmoid, compared with host expectations by tests/test_gpu_probes.py */
hipError_t xtu_probe_fp4(const float* scales, int nscale, uint32_t* out, hipStream_t stream);
hipError_t xtu_probe_fp4_mul(const float* scales, int nscale, uint32_t* out, hipStream_t stream);
hipError_t xtu_probe_fp8(uint32_t* out, hipStream_t stream);
hipError_t xtu_probe_mfma(int which, const void* A, const void* B, void* C, hipStream_t stream);
hipError_t xtu_probe_exp(const float* x, int n, float* e, float* s, hipStream_t stream);
/* one v_mfma_scale_f32_16x16x128_f8f6f4, fp8 A x fp4 B: raw lane operands A,
 * B [64][8] dwords, per-lane scale bytes sa, sb [64]; C [64][4] raw lanes */
hipError_t xtu_probe_mfma_scaled_fp4b(const int* A, const int* B, const uint8_t* sa,
                                     const uint8_t* sb, float* C, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* XTU_PROBES_H */
