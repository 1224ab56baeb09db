// Per-format description of one 16-byte weight chunk in the P16 panel layout
// and its conversion to bf16 MFMA operands (exact for every format).
#pragma once

#include "xtu_common.hpp"

namespace xtu {

template <int FMT>
struct WFmt;

// fp4 scale groups: per panel, the scales of kUG consecutive super-blocks
// are stored [64 lanes][16 bytes] (lane = 16q + r: chunk q of row r), so one
// 16-byte load gives a lane the scales of kUG super-blocks.  Groups per panel:
// ceil((K/128) / kUG); the last group is zero-padded.
__host__ __device__ constexpr long scale_groups(long K, int ug) { return (K / 128 + ug - 1) / ug; }

// MXFP4: 32 e2m1 codes per chunk, one e8m0 byte per chunk.
template <>
struct WFmt<kMXFP4> {
  static constexpr int kCK = 32;       // k per chunk
  static constexpr int kWords = 16;    // bf16 pairs per chunk
  static constexpr int kSB = 128;      // k per super-block (4 chunks)
  static constexpr int kSPU = 1;       // super-blocks per 128-k unit
  static constexpr int kSBY = 1;       // scale bytes per chunk
  static constexpr int kUG = 16;       // super-blocks per scale group
  static __host__ __device__ constexpr long w_bytes(long N, long K) { return N * K / 2; }
  static __host__ __device__ constexpr long s_bytes(long N, long K) {
    return N / 16 * scale_groups(K, kUG) * 1024;
  }
};

// NVFP4: 32 e2m1 codes per chunk, two e4m3 bytes (one per 16 k) per chunk,
// plus a per-expert fp32 global scale applied to the GEMM result.
template <>
struct WFmt<kNVFP4> {
  static constexpr int kCK = 32;
  static constexpr int kWords = 16;
  static constexpr int kSB = 128;
  static constexpr int kSPU = 1;
  static constexpr int kSBY = 2;
  static constexpr int kUG = 8;
  static __host__ __device__ constexpr long w_bytes(long N, long K) { return N * K / 2; }
  static __host__ __device__ constexpr long s_bytes(long N, long K) {
    return N / 16 * scale_groups(K, kUG) * 1024;
  }
};

// FP8 e4m3: 16 codes per chunk; one fp32 scale per 128x128 block.
template <>
struct WFmt<kFP8> {
  static constexpr int kCK = 16;
  static constexpr int kWords = 8;
  static constexpr int kSB = 64;
  static constexpr int kSPU = 2;
  static constexpr int kSBY = 0;
  static constexpr int kUG = 1;
  static __host__ __device__ constexpr long w_bytes(long N, long K) { return N * K; }
  static __host__ __device__ constexpr long s_bytes(long N, long K) { return (N / 128) * (K / 128) * 4; }
};

// BF16: 8 values per chunk, no scale.
template <>
struct WFmt<kBF16> {
  static constexpr int kCK = 8;
  static constexpr int kWords = 4;
  static constexpr int kSB = 32;
  static constexpr int kSPU = 4;
  static constexpr int kSBY = 0;
  static constexpr int kUG = 1;
  static __host__ __device__ constexpr long w_bytes(long N, long K) { return N * K * 2; }
  static __host__ __device__ constexpr long s_bytes(long, long) { return 0; }
};

// Byte offset of the scale(s) of chunk `lane` (= 16q + r) of super-block sb
// of a panel inside an expert's fp4 scale array (K = the row length).
template <int FMT>
__host__ __device__ __forceinline__ long scale_offset(long panel, long sb, int lane, long K) {
  using F = WFmt<FMT>;
  const long g = panel * scale_groups(K, F::kUG) + sb / F::kUG;
  return (g * 64 + lane) * 16 + (sb % F::kUG) * F::kSBY;
}

// Raw scale bits of one chunk (no use of the value, so the load does not
// stall the issue of the loads that follow it).  `sc` points at this expert's
// fp4 scale array.
template <int FMT>
__device__ __forceinline__ uint32_t load_chunk_scale_raw(const uint8_t* __restrict__ sc,
                                                         long panel, long sb, int lane, long K) {
  if constexpr (FMT == kMXFP4) {
    return sc[scale_offset<FMT>(panel, sb, lane, K)];
  } else if constexpr (FMT == kNVFP4) {
    return *reinterpret_cast<const uint16_t*>(sc + scale_offset<FMT>(panel, sb, lane, K));
  } else {
    return 0u;
  }
}

// Branch-free decode of the raw scale bits into the chunk's scale(s).
template <int FMT>
__device__ __forceinline__ void chunk_scale(uint32_t raw, float& s0, float& s1) {
  if constexpr (FMT == kMXFP4) {
    s0 = e8m0_to_f32(raw);
    s1 = s0;
  } else if constexpr (FMT == kNVFP4) {
    s0 = e4m3_to_f32(raw & 0xffu);
    s1 = e4m3_to_f32((raw >> 8) & 0xffu);
  } else {
    s0 = s1 = 1.0f;
  }
}

template <int FMT>
__device__ __forceinline__ void decode_chunk(const u32x4_t raw, float s0, float s1,
                                             uint32_t* words) {
  if constexpr (FMT == kMXFP4) {
    fp4x32_to_bf16(raw, s0, words);
  } else if constexpr (FMT == kNVFP4) {
    fp4x32_to_bf16_2s(raw, s0, s1, words);
  } else if constexpr (FMT == kFP8) {
    fp8x16_to_bf16(raw, words);
  } else {
    words[0] = raw[0];
    words[1] = raw[1];
    words[2] = raw[2];
    words[3] = raw[3];
  }
}

}  // namespace xtu
