// Skinny-M (decode) expert kernels: a handful of tokens per expert, so the
// layer is a weight stream.  Every wave reads one contiguous KiB of its
// panel per step (16 bytes per lane, the P16 layout), dequantises it in
// registers to bf16 and feeds v_mfma_f32_16x16x32_bf16 with the expert's
// tokens as the 16-row A operand (rows beyond the expert's token count are
// zero).  The K range of a panel is split over KSPLIT waves of the same
// workgroup and reduced through LDS in a fixed order, so results are
// deterministic.  Empty expert slots (beyond n_active) exit at once; experts
// nobody routed to (or only with zero weight) are never read.
//
// gate/up: one workgroup per (gate panel p, active expert); waves [0,KSPLIT)
//   stream gate rows 16p.., waves [KSPLIT, 2KSPLIT) the matching up rows
//   I+16p.., so the SwiGLU of row n is formed in the reduction step and only
//   the bf16 activation row is written.
// down:    one workgroup per (PPB panels of W2, active expert); y is fp32.
#include "weight_format.hpp"

namespace xtu {
namespace {

constexpr int kWave = 64;

struct DecodeArgs {
  const uint16_t* x;         // gate/up: hidden rows [T][H]; down: act rows [A][I]
  const uint8_t* w;          // packed weights, expert-major
  const uint8_t* s;          // fp4 scales (packed) or fp8 block scales (fp32)
  const float* gs;           // NVFP4 per-expert global scale (may be null)
  const int32_t* sorted_tok;
  const int32_t* seg_start;
  const int32_t* active;
  const int32_t* n_active;
  const int32_t* slot_map;   // expert -> weight slot (null: identity)
  void* out;                 // gate/up: act bf16 [A][I]; down: y fp32 [A][H]
  int H, I;
  long w_estride, s_estride;
  float limit, alpha, beta;
};

// Accumulate a 16 x 16 output tile (tokens x panel rows) over 128-k units
// [u0, u1) of one panel with K = K_total.
template <int FMT>
__device__ __forceinline__ f32x4_t panel_gemv(const DecodeArgs& a, int ws, int panel, int K_total,
                                              const uint16_t* __restrict__ arow, int u0, int u1,
                                              int lane) {
  using F = WFmt<FMT>;
  const int q = lane / 16;
  const long nsbk = K_total / F::kSB;   // super-blocks per panel row
  const uint8_t* wp = a.w + (long)ws * a.w_estride + ((long)panel * nsbk) * 1024 + lane * 16;
  const uint8_t* sp = a.s + (long)ws * a.s_estride;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int u = u0; u < u1; ++u) {
    f32x4_t part = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < F::kSPU; ++j) {
      const long sb = (long)u * F::kSPU + j;
      const u32x4_t raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wp + sb * 1024));
      float s0, s1;
      load_chunk_scale<FMT>(sp, (long)panel * nsbk + sb, lane, s0, s1);
      uint32_t words[F::kWords];
      decode_chunk<FMT>(raw, s0, s1, words);
#pragma unroll
      for (int st = 0; st < F::kWords / 4; ++st) {
        u32x4_t av = {0u, 0u, 0u, 0u};
        if (arow) av = *reinterpret_cast<const u32x4_t*>(arow + sb * F::kSB + q * F::kCK + 8 * st);
        const bf16x8_t bv = as_bf16x8(words[4 * st], words[4 * st + 1], words[4 * st + 2],
                                      words[4 * st + 3]);
        if constexpr (FMT == kFP8)
          part = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av), bv, part, 0, 0, 0);
        else
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av), bv, acc, 0, 0, 0);
      }
    }
    if constexpr (FMT == kFP8) {
      // one fp32 block scale per (128 rows, 128 k): exact fp32 promotion
      const float* bs = reinterpret_cast<const float*>(a.s + (long)ws * a.s_estride);
      const float sc = bs[(long)(panel / 8) * (K_total / 128) + u];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(sc, part[i], acc[i]);
    }
  }
  return acc;
}

template <int FMT, int KSPLIT>
__global__ __launch_bounds__(128 * KSPLIT) void decode_gate_up_kernel(DecodeArgs a) {
  __shared__ f32x4_t red[2 * KSPLIT][kWave];
  const int slot = blockIdx.y;
  if (slot >= a.n_active[0]) return;           // uniform over the workgroup
  const int e = a.active[slot];
  const int r0 = a.seg_start[e];
  const int na = min(a.seg_start[e + 1] - r0, 16);
  const int p = blockIdx.x;
  const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int half = w / KSPLIT, ks = w % KSPLIT;
  const int panel = half ? (a.I / 16 + p) : p;
  const int nunits = a.H / 128;
  const int u0 = ks * nunits / KSPLIT, u1 = (ks + 1) * nunits / KSPLIT;
  const int tslot = lane % 16;
  const uint16_t* arow = tslot < na ? a.x + (long)a.sorted_tok[r0 + tslot] * a.H : nullptr;
  const int ws = a.slot_map ? a.slot_map[e] : e;
  red[w][lane] = panel_gemv<FMT>(a, ws, panel, a.H, arow, u0, u1, lane);
  __syncthreads();
  const int t = threadIdx.x;
  if (t < 256) {
    const int m = t / 16, n = t % 16;
    if (m < na) {
      const int l = (m / 4) * 16 + n, i = m % 4;
      float g = 0.f, u = 0.f;
#pragma unroll
      for (int k = 0; k < KSPLIT; ++k) {
        g += red[k][l][i];
        u += red[KSPLIT + k][l][i];
      }
      if constexpr (FMT == kNVFP4) {
        const float gsv = a.gs ? a.gs[ws] : 1.0f;
        g *= gsv;
        u *= gsv;
      }
      uint16_t* act = reinterpret_cast<uint16_t*>(a.out);
      act[(long)(r0 + m) * a.I + 16 * p + n] = f32_to_bf16(silu_gate(g, u, a.limit, a.alpha, a.beta));
    }
  }
}

template <int FMT, int KSPLIT, int PPB>
__global__ __launch_bounds__(64 * KSPLIT * PPB) void decode_down_kernel(DecodeArgs a) {
  __shared__ f32x4_t red[KSPLIT * PPB][kWave];
  const int slot = blockIdx.y;
  if (slot >= a.n_active[0]) return;
  const int e = a.active[slot];
  const int r0 = a.seg_start[e];
  const int na = min(a.seg_start[e + 1] - r0, 16);
  const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int pp = w / KSPLIT, ks = w % KSPLIT;
  const int panel = blockIdx.x * PPB + pp;
  const int nunits = a.I / 128;
  const int u0 = ks * nunits / KSPLIT, u1 = (ks + 1) * nunits / KSPLIT;
  const int tslot = lane % 16;
  const uint16_t* arow = tslot < na ? a.x + (long)(r0 + tslot) * a.I : nullptr;
  const int ws = a.slot_map ? a.slot_map[e] : e;
  red[w][lane] = panel_gemv<FMT>(a, ws, panel, a.I, arow, u0, u1, lane);
  __syncthreads();
  float gsv = 1.0f;
  if constexpr (FMT == kNVFP4) gsv = a.gs ? a.gs[ws] : 1.0f;
  float* y = reinterpret_cast<float*>(a.out);
  for (int t = threadIdx.x; t < PPB * 256; t += 64 * KSPLIT * PPB) {
    const int pq = t / 256, m = (t % 256) / 16, n = t % 16;
    if (m < na) {
      const int l = (m / 4) * 16 + n, i = m % 4;
      float v = 0.f;
#pragma unroll
      for (int k = 0; k < KSPLIT; ++k) v += red[pq * KSPLIT + k][l][i];
      y[(long)(r0 + m) * a.H + 16 * (blockIdx.x * PPB + pq) + n] = v * gsv;
    }
  }
}

template <int FMT>
hipError_t launch_decode(int which, DecodeArgs a, int max_active, hipStream_t stream) {
  using F = WFmt<FMT>;
  if (which == 0) {
    if (!a.w_estride) a.w_estride = F::w_bytes(2L * a.I, a.H);
    if (!a.s_estride) a.s_estride = F::s_bytes(2L * a.I, a.H);
    dim3 grid(a.I / 16, max_active);
    decode_gate_up_kernel<FMT, 2><<<grid, 256, 0, stream>>>(a);
  } else {
    if (!a.w_estride) a.w_estride = F::w_bytes(a.H, a.I);
    if (!a.s_estride) a.s_estride = F::s_bytes(a.H, a.I);
    dim3 grid(a.H / 16 / 2, max_active);
    decode_down_kernel<FMT, 2, 2><<<grid, 256, 0, stream>>>(a);
  }
  return hipPeekAtLastError();
}

hipError_t dispatch_decode(int fmt, int which, DecodeArgs a, int max_active, hipStream_t stream) {
  switch (fmt) {
    case kMXFP4: return launch_decode<kMXFP4>(which, a, max_active, stream);
    case kNVFP4: return launch_decode<kNVFP4>(which, a, max_active, stream);
    case kFP8: return launch_decode<kFP8>(which, a, max_active, stream);
    case kBF16: return launch_decode<kBF16>(which, a, max_active, stream);
  }
  return hipErrorInvalidValue;
}

bool shape_ok(int fmt, int H, int I) {
  if (H <= 0 || I <= 0 || H % 128 || I % 128) return false;
  if (fmt == kFP8 && ((2 * I) % 128 || H % 128)) return false;
  return fmt >= 0 && fmt <= 3;
}

}  // namespace
}  // namespace xtu

using namespace xtu;

extern "C" {

hipError_t xtu_decode_gate_up(int fmt, const void* x, int H, int I, const void* w13,
                              const void* s13, const float* gs13, long w_estride,
                              long s_estride, const int32_t* slot_map,
                              const int32_t* sorted_tok, const int32_t* seg_start,
                              const int32_t* active, const int32_t* n_active, int max_active,
                              void* act, float limit, float alpha, float beta,
                              hipStream_t stream) {
  XTU_CHECK_ARG(shape_ok(fmt, H, I) && max_active >= 0 && max_active <= 65535);
  XTU_CHECK_ARG(w_estride >= 0 && s_estride >= 0);
  XTU_CHECK_ARG(x && w13 && (fmt == kBF16 || s13) && sorted_tok && seg_start && active &&
                n_active && act);
  if (max_active == 0) return hipSuccess;
  (void)hipGetLastError();
  DecodeArgs a{(const uint16_t*)x, (const uint8_t*)w13, (const uint8_t*)s13, gs13, sorted_tok,
               seg_start, active, n_active, slot_map, act, H, I, w_estride, s_estride, limit,
               alpha, beta};
  return dispatch_decode(fmt, 0, a, max_active, stream);
}

hipError_t xtu_decode_down(int fmt, const void* act, int H, int I, const void* w2,
                           const void* s2, const float* gs2, long w_estride, long s_estride,
                           const int32_t* slot_map, const int32_t* seg_start,
                           const int32_t* active, const int32_t* n_active, int max_active,
                           float* y, hipStream_t stream) {
  XTU_CHECK_ARG(shape_ok(fmt, H, I) && max_active >= 0 && max_active <= 65535 &&
                (H / 16) % 2 == 0);
  XTU_CHECK_ARG(w_estride >= 0 && s_estride >= 0);
  XTU_CHECK_ARG(act && w2 && (fmt == kBF16 || s2) && seg_start && active && n_active && y);
  if (max_active == 0) return hipSuccess;
  (void)hipGetLastError();
  DecodeArgs a{(const uint16_t*)act, (const uint8_t*)w2, (const uint8_t*)s2, gs2, nullptr,
               seg_start, active, n_active, slot_map, y, H, I, w_estride, s_estride, 0.f, 1.f,
               0.f};
  return dispatch_decode(fmt, 1, a, max_active, stream);
}

}  // extern "C"
