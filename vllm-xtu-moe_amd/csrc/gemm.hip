// Grouped expert GEMMs for prefill-sized batches, and the weighted combine.
//
// Tile list: seg_scan_kernel cuts each expert's contiguous segment of sorted
// pairs into M tiles of BM rows; blockIdx.x walks that list (entries past
// n_tiles exit at once), blockIdx.y walks 256-row blocks of the weight.
//
// Per K step (BK = 64) a workgroup of four waves stages
//   A: BM activation rows (gathered through sorted_tok for gate/up, the
//      contiguous act rows for down) as bf16, and
//   B: 256 weight rows read from the P16 panel layout (each panel's K slice is
//      one contiguous run of bytes), dequantised exactly to bf16 while being
//      written to LDS,
// then each wave runs v_mfma_f32_32x32x16_bf16 over its BM x 64 sub-tile.
// Global loads of step k+1 are issued before the MFMAs of step k.
//
// Scale handling, all exact: MXFP4 e8m0 and NVFP4 e4m3 scales are folded into
// the bf16 operand (products are representable); NVFP4's per-expert global
// scale multiplies the fp32 result; FP8's 128x128 fp32 block scales multiply
// a per-128-k partial accumulator (fp32 promotion, no operand rounding).
//
// gate/up blocks hold 128 gate rows and the matching 128 up rows, so each
// lane owns (g, u) of the same output element and the epilogue writes the
// clamped-SwiGLU activation as bf16.  down writes fp32 y rows; the combine
// kernel adds them per token in top-k order.
#include "weight_format.hpp"

namespace xtu {
namespace {

constexpr int kBK = 64;
constexpr int kBN = 256;
constexpr int kLDK = kBK + 8;   // LDS row pitch in bf16 (16-byte pad)

struct GemmArgs {
  const uint16_t* a;          // gate/up: x [T][K]; down: act [A][K]
  const int32_t* sorted_tok;  // gate/up row gather
  const uint8_t* w;
  const uint8_t* s;
  const float* gs;
  const int32_t* seg_start;
  const int32_t* tile_expert;
  const int32_t* tile_row0;
  const int32_t* tile_lo;     // m-tile range [*tile_lo, *tile_hi) of the tile list
  const int32_t* tile_hi;
  const int32_t* slot_map;    // expert -> weight slot (null: identity)
  void* out;                  // gate/up: act bf16 [A][I]; down: y fp32 [A][H]
  int H, I;
  long w_estride, s_estride;
  float limit, alpha, beta;
};

template <int FMT, int BM, bool GU>
__global__ __launch_bounds__(256) void moe_gemm_kernel(GemmArgs a) {
  using F = WFmt<FMT>;
  constexpr int MT = BM / 32;                     // 32-row MFMA tiles per wave
  constexpr int A_CH = BM * kBK / 8 / 256;        // 16-byte A chunks per thread
  constexpr int CPP = (kBK / F::kCK) * 16;        // B chunks per panel per K step
  constexpr int B_CH = 16 * CPP / 256;            // B chunks per thread
  constexpr bool kIsFP8 = (FMT == kFP8);
  __shared__ __attribute__((aligned(16))) uint16_t As[BM * kLDK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[kBN * kLDK];

  const int tile = a.tile_lo[0] + blockIdx.x;
  if (tile >= a.tile_hi[0]) return;
  const int e = a.tile_expert[tile];
  const int ws = a.slot_map ? a.slot_map[e] : e;
  const int row0 = a.tile_row0[tile];
  const int rows = min(BM, a.seg_start[e + 1] - row0);
  const int nb = blockIdx.y;
  const int K = GU ? a.H : a.I;
  const int tid = threadIdx.x, w = tid / 64, lane = tid % 64;
  const long nsbk = K / F::kSB;
  const uint8_t* wexp = a.w + (long)ws * a.w_estride;
  const uint8_t* sexp = a.s ? a.s + (long)ws * a.s_estride : nullptr;

  // A source row of each chunk this thread loads (constant over K)
  const uint16_t* asrc[A_CH];
#pragma unroll
  for (int i = 0; i < A_CH; ++i) {
    const int c = i * 256 + tid, r = c / 8;
    if (r < rows) {
      const long src = GU ? (long)a.sorted_tok[row0 + r] : (long)(row0 + r);
      asrc[i] = a.a + src * K + (c % 8) * 8;
    } else {
      asrc[i] = nullptr;
    }
  }
  // B: weight panel and in-region offset of each chunk this thread loads
  long bpanel[B_CH];
  int boff[B_CH];
#pragma unroll
  for (int i = 0; i < B_CH; ++i) {
    const int c = i * 256 + tid, pl = c / CPP;
    boff[i] = c % CPP;
    if (GU) bpanel[i] = pl < 8 ? (long)nb * 8 + pl : (long)(a.I / 16) + nb * 8 + (pl - 8);
    else bpanel[i] = (long)nb * 16 + pl;
  }

  u32x4_t areg[A_CH];
  u32x4_t breg[B_CH];
  uint32_t bsraw[B_CH];

  auto gload = [&](int kk) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      u32x4_t v = {0u, 0u, 0u, 0u};
      if (asrc[i]) v = *reinterpret_cast<const u32x4_t*>(asrc[i] + kk);
      areg[i] = v;
    }
    const long sb = kk / F::kSB;
    const int qbase = (kk % F::kSB) / F::kCK;
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      const uint8_t* region = wexp + (bpanel[i] * nsbk + sb) * 1024 + qbase * 256;
      breg[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(region + boff[i] * 16));
      const int lane_eq = qbase * 16 + boff[i];   // (q, r) position inside the super-block
      bsraw[i] = load_chunk_scale_raw<FMT>(sexp, bpanel[i], sb, lane_eq, K);
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int c = i * 256 + tid;
      *reinterpret_cast<u32x4_t*>(&As[(c / 8) * kLDK + (c % 8) * 8]) = areg[i];
    }
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      const int c = i * 256 + tid, pl = c / CPP;
      const int r = boff[i] % 16, qr = boff[i] / 16;
      uint32_t words[F::kWords];
      float s0, s1;
      chunk_scale<FMT>(bsraw[i], s0, s1);
      decode_chunk<FMT>(breg[i], s0, s1, words);
      uint16_t* dst = &Bs[(pl * 16 + r) * kLDK + qr * F::kCK];
#pragma unroll
      for (int j = 0; j < F::kWords / 4; ++j) {
        u32x4_t v = {words[4 * j], words[4 * j + 1], words[4 * j + 2], words[4 * j + 3]};
        *reinterpret_cast<u32x4_t*>(dst + 8 * j) = v;
      }
    }
  };

  // wave's two 32-column tiles inside the 256-row B block
  const int jt0 = GU ? 32 * w : 64 * w;
  const int jt1 = GU ? 128 + 32 * w : 64 * w + 32;

  f32x16_t acc[MT][2];
  f32x16_t part[kIsFP8 ? MT : 1][2];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int n = 0; n < 2; ++n) {
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[m][n][i] = 0.f;
    }
  if constexpr (kIsFP8) {
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int i = 0; i < 16; ++i) part[m][n][i] = 0.f;
  }

  const int nk = K / kBK;
  gload(0);
  for (int kt = 0; kt < nk; ++kt) {
    __syncthreads();
    lstore();
    __syncthreads();
    if (kt + 1 < nk) gload((kt + 1) * kBK);
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      const int kofs = ks * 16 + (lane / 32) * 8;
      const bf16x8_t b0 = as_bf16x8(*reinterpret_cast<const u32x4_t*>(&Bs[(jt0 + lane % 32) * kLDK + kofs]));
      const bf16x8_t b1 = as_bf16x8(*reinterpret_cast<const u32x4_t*>(&Bs[(jt1 + lane % 32) * kLDK + kofs]));
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const bf16x8_t av = as_bf16x8(*reinterpret_cast<const u32x4_t*>(&As[(m * 32 + lane % 32) * kLDK + kofs]));
        if constexpr (kIsFP8) {
          part[m][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, b0, part[m][0], 0, 0, 0);
          part[m][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, b1, part[m][1], 0, 0, 0);
        } else {
          acc[m][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, b0, acc[m][0], 0, 0, 0);
          acc[m][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, b1, acc[m][1], 0, 0, 0);
        }
      }
    }
    if constexpr (kIsFP8) {
      if ((kt & 1) == 1) {   // a 128-k block is complete: fold its fp32 scale
        const float* bsc = reinterpret_cast<const float*>(sexp);
        const long kb = (long)(kt / 2);
        long rb0, rb1;
        if (GU) {
          rb0 = (long)nb;                      // gate rows nb*128 + ...
          rb1 = (long)(a.I / 128) + nb;        // up rows I + nb*128 + ...
        } else {
          rb0 = ((long)nb * 256 + jt0) / 128;
          rb1 = ((long)nb * 256 + jt1) / 128;
        }
        const float s0 = bsc[rb0 * (K / 128) + kb];
        const float s1 = bsc[rb1 * (K / 128) + kb];
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            acc[m][0][i] = __builtin_fmaf(s0, part[m][0][i], acc[m][0][i]);
            acc[m][1][i] = __builtin_fmaf(s1, part[m][1][i], acc[m][1][i]);
            part[m][0][i] = 0.f;
            part[m][1][i] = 0.f;
          }
      }
    }
  }

  float gsv = 1.0f;
  if constexpr (FMT == kNVFP4) gsv = a.gs ? a.gs[ws] : 1.0f;
  const int ncol = lane % 32;
  if constexpr (GU) {
    uint16_t* act = reinterpret_cast<uint16_t*>(a.out);
    const long col = (long)nb * 128 + 32 * w + ncol;
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = m * 32 + (i / 4) * 8 + (lane / 32) * 4 + (i % 4);
        if (r < rows) {
          const float g = acc[m][0][i] * gsv, u = acc[m][1][i] * gsv;
          act[(long)(row0 + r) * a.I + col] = f32_to_bf16(silu_gate(g, u, a.limit, a.alpha, a.beta));
        }
      }
  } else {
    float* y = reinterpret_cast<float*>(a.out);
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = m * 32 + (i / 4) * 8 + (lane / 32) * 4 + (i % 4);
        if (r < rows) {
          float* yr = y + (long)(row0 + r) * a.H + (long)nb * 256;
          yr[jt0 + ncol] = acc[m][0][i] * gsv;
          yr[jt1 + ncol] = acc[m][1][i] * gsv;
        }
      }
  }
}

// out[t][h] = sum_k w[t,k] * y[inv[t*K+k]][h] over the pairs that were not
// sent to the trash bucket (sorted position < *trash_start) and have a
// non-zero weight, in k order, + sum_s y[inv[T*K + t*NS + s]][h]
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ y,
                                                      const int32_t* __restrict__ inv,
                                                      const float* __restrict__ wts,
                                                      const int32_t* __restrict__ trash_start,
                                                      int T, int K, int NS, int H, void* out,
                                                      int out_bf16) {
  const int t = blockIdx.y;
  const int h = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (h >= H) return;
  const int trash = trash_start[0];
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int k = 0; k < K; ++k) {
    const int pos = inv[t * K + k];
    const float w = wts[t * K + k];
    if (pos >= trash || w == 0.f) continue;
    const f32x4_t v = *reinterpret_cast<const f32x4_t*>(y + (long)pos * H + h);
    acc += w * v;
  }
  for (int s = 0; s < NS; ++s) {
    const f32x4_t v = *reinterpret_cast<const f32x4_t*>(y + (long)inv[T * K + t * NS + s] * H + h);
    acc += v;
  }
  if (out_bf16) {
    uint16_t* o = reinterpret_cast<uint16_t*>(out) + (long)t * H + h;
    const uint32_t lo = f32_to_bf16(acc[0]) | ((uint32_t)f32_to_bf16(acc[1]) << 16);
    const uint32_t hi = f32_to_bf16(acc[2]) | ((uint32_t)f32_to_bf16(acc[3]) << 16);
    *reinterpret_cast<uint2*>(o) = make_uint2(lo, hi);
  } else {
    *reinterpret_cast<f32x4_t*>(reinterpret_cast<float*>(out) + (long)t * H + h) = acc;
  }
}

template <int FMT, int BM>
hipError_t launch_gemm(bool gu, GemmArgs a, int max_tiles, hipStream_t stream) {
  using F = WFmt<FMT>;
  if (gu) {
    if (!a.w_estride) a.w_estride = F::w_bytes(2L * a.I, a.H);
    if (!a.s_estride) a.s_estride = F::s_bytes(2L * a.I, a.H);
    dim3 grid(max_tiles, a.I / 128);
    moe_gemm_kernel<FMT, BM, true><<<grid, 256, 0, stream>>>(a);
  } else {
    if (!a.w_estride) a.w_estride = F::w_bytes(a.H, a.I);
    if (!a.s_estride) a.s_estride = F::s_bytes(a.H, a.I);
    dim3 grid(max_tiles, a.H / 256);
    moe_gemm_kernel<FMT, BM, false><<<grid, 256, 0, stream>>>(a);
  }
  return hipPeekAtLastError();
}

}  // namespace
}  // namespace xtu

using namespace xtu;

extern "C" {

int xtu_gemm_tile_m(int fmt) { return fmt == kFP8 ? 64 : 128; }

hipError_t xtu_gemm_gate_up(int fmt, const void* x, const int32_t* sorted_tok, int H, int I,
                            const void* w13, const void* s13, const float* gs13,
                            long w_estride, long s_estride, const int32_t* slot_map,
                            const int32_t* seg_start, const int32_t* tile_expert,
                            const int32_t* tile_row0, const int32_t* tile_lo,
                            const int32_t* tile_hi, int max_tiles, void* act, float limit,
                            float alpha, float beta, hipStream_t stream) {
  XTU_CHECK_ARG(fmt >= 0 && fmt <= 3 && H > 0 && I > 0 && H % 256 == 0 && I % 128 == 0);
  XTU_CHECK_ARG(max_tiles >= 0 && max_tiles < (1 << 30) && w_estride >= 0 && s_estride >= 0);
  XTU_CHECK_ARG(x && sorted_tok && w13 && (fmt == kBF16 || s13) && seg_start && tile_expert &&
                tile_row0 && tile_lo && tile_hi && act);
  if (max_tiles == 0) return hipSuccess;
  (void)hipGetLastError();
  GemmArgs a{(const uint16_t*)x, sorted_tok, (const uint8_t*)w13, (const uint8_t*)s13, gs13,
             seg_start, tile_expert, tile_row0, tile_lo, tile_hi, slot_map, act, H, I,
             w_estride, s_estride, limit, alpha, beta};
  switch (fmt) {
    case kMXFP4: return launch_gemm<kMXFP4, 128>(true, a, max_tiles, stream);
    case kNVFP4: return launch_gemm<kNVFP4, 128>(true, a, max_tiles, stream);
    case kFP8: return launch_gemm<kFP8, 64>(true, a, max_tiles, stream);
    case kBF16: return launch_gemm<kBF16, 128>(true, a, max_tiles, stream);
  }
  return hipErrorInvalidValue;
}

hipError_t xtu_gemm_down(int fmt, const void* act, int H, int I, const void* w2, const void* s2,
                         const float* gs2, long w_estride, long s_estride,
                         const int32_t* slot_map, const int32_t* seg_start,
                         const int32_t* tile_expert, const int32_t* tile_row0,
                         const int32_t* tile_lo, const int32_t* tile_hi, int max_tiles, float* y,
                         hipStream_t stream) {
  XTU_CHECK_ARG(fmt >= 0 && fmt <= 3 && H > 0 && I > 0 && H % 256 == 0 && I % 128 == 0);
  XTU_CHECK_ARG(max_tiles >= 0 && max_tiles < (1 << 30) && w_estride >= 0 && s_estride >= 0);
  XTU_CHECK_ARG(act && w2 && (fmt == kBF16 || s2) && seg_start && tile_expert && tile_row0 &&
                tile_lo && tile_hi && y);
  if (max_tiles == 0) return hipSuccess;
  (void)hipGetLastError();
  GemmArgs a{(const uint16_t*)act, nullptr, (const uint8_t*)w2, (const uint8_t*)s2, gs2,
             seg_start, tile_expert, tile_row0, tile_lo, tile_hi, slot_map, y, H, I, w_estride,
             s_estride, 0.f, 1.f, 0.f};
  switch (fmt) {
    case kMXFP4: return launch_gemm<kMXFP4, 128>(false, a, max_tiles, stream);
    case kNVFP4: return launch_gemm<kNVFP4, 128>(false, a, max_tiles, stream);
    case kFP8: return launch_gemm<kFP8, 64>(false, a, max_tiles, stream);
    case kBF16: return launch_gemm<kBF16, 128>(false, a, max_tiles, stream);
  }
  return hipErrorInvalidValue;
}

hipError_t xtu_combine(const float* y, const int32_t* inv, const float* topk_weights,
                       const int32_t* trash_start, int T, int K, int n_shared, int H, void* out,
                       int out_bf16, hipStream_t stream) {
  XTU_CHECK_ARG(T >= 0 && T <= 65535 && K >= 0 && n_shared >= 0 && H > 0 && H % 4 == 0);
  XTU_CHECK_ARG(T == 0 || (y && inv && out && trash_start && (K == 0 || topk_weights)));
  if (T == 0) return hipSuccess;
  (void)hipGetLastError();
  dim3 grid((H / 4 + 255) / 256, T);
  combine_kernel<<<grid, 256, 0, stream>>>(y, inv, topk_weights, trash_start, T, K, n_shared, H,
                                           out, out_bf16);
  return hipPeekAtLastError();
}

}  // extern "C"
