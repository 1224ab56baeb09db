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
  const float* sorted_wts;   // down+combine: pair weight per sorted row
  int lds_rows;              // activation rows staged in LDS (<= kLdsRows)
};

// Activation rows of one expert staged in LDS: rows m < min(na, kLdsRows) of
// length K (bf16); rows kLdsRows <= m < na are read from global memory.
constexpr int kLdsRows = 4;

// launch shape (waves per workgroup split K; D = 128-k units in flight per wave)
#ifndef XTU_GU_KSPLIT
#define XTU_GU_KSPLIT 4
#endif
#ifndef XTU_GU_D
#define XTU_GU_D 4
#endif
#ifndef XTU_GU_MAXGRID
#define XTU_GU_MAXGRID 1024
#endif
#ifndef XTU_DN_KSPLIT
#define XTU_DN_KSPLIT 2
#endif
#ifndef XTU_DN_PPB
#define XTU_DN_PPB 2
#endif
#ifndef XTU_DN_D
#define XTU_DN_D 4
#endif
#ifndef XTU_DN_MAXGRID
#define XTU_DN_MAXGRID 2048
#endif

// One batch of D 128-k units of a panel held in registers: weight chunks, raw
// scale bits, and (FP8) the block scale of each unit.
template <int FMT, int D>
struct WBatch {
  u32x4_t raw[D][WFmt<FMT>::kSPU];
  uint32_t sraw[D][WFmt<FMT>::kSPU];
  float bsc[D];
};

// Stream position of one wave inside one panel of one expert.
struct PanelPos {
  const uint8_t* wp;   // this lane's bytes in (panel, super-block 0)
  const uint8_t* sp;   // expert's scale array
  long sbase;          // panel * super-blocks per row
  int panel, K_total;
};

template <int FMT>
__device__ __forceinline__ PanelPos panel_pos(const DecodeArgs& a, int ws, int panel, int K_total,
                                              int lane) {
  using F = WFmt<FMT>;
  const long nsbk = K_total / F::kSB;
  PanelPos p;
  p.wp = a.w + (long)ws * a.w_estride + ((long)panel * nsbk) * 1024 + lane * 16;
  p.sp = a.s + (long)ws * a.s_estride;
  p.sbase = (long)panel * nsbk;
  p.panel = panel;
  p.K_total = K_total;
  return p;
}

// Issue the loads of units [ub, ub + D) (units >= u1 re-read unit ub, unused).
template <int FMT, int D>
__device__ __forceinline__ void issue_batch(WBatch<FMT, D>& b, const PanelPos& p, int ub, int u1,
                                            int lane) {
  using F = WFmt<FMT>;
#pragma unroll
  for (int i = 0; i < D; ++i) {
    const int u = (ub + i < u1) ? ub + i : ub;
#pragma unroll
    for (int j = 0; j < F::kSPU; ++j) {
      const long sb = (long)u * F::kSPU + j;
      b.raw[i][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p.wp + sb * 1024));
      b.sraw[i][j] = load_chunk_scale_raw<FMT>(p.sp, p.sbase + sb, lane);
    }
    if constexpr (FMT == kFP8)
      b.bsc[i] = reinterpret_cast<const float*>(p.sp)[(long)(p.panel / 8) * (p.K_total / 128) + u];
  }
}

// MFMA the batch into acc.  The activation fragment of lane (q, m) for unit
// u, step st is row m, k = u*128 + q*kCK + 8*st (fp4; likewise for the other
// formats through kSB / kCK): from LDS (LDS_ONLY: row index clamped to the
// zero row) or, for rows beyond the staged ones, from global memory.
template <int FMT, int D, bool LDS_ONLY>
__device__ __forceinline__ void compute_batch(const WBatch<FMT, D>& b, f32x4_t& acc,
                                              const uint16_t* __restrict__ arow_z,
                                              const uint16_t* __restrict__ arow_l,
                                              const uint16_t* __restrict__ arow_g, int ub, int u1,
                                              int q) {
  using F = WFmt<FMT>;
  constexpr int ST = F::kWords / 4;
#pragma unroll
  for (int i = 0; i < D; ++i) {
    const int u = ub + i;
    if (u >= u1) break;
    f32x4_t part = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < F::kSPU; ++j) {
      const long sb = (long)u * F::kSPU + j;
      uint32_t words[F::kWords];
      float s0, s1;
      chunk_scale<FMT>(b.sraw[i][j], s0, s1);
      decode_chunk<FMT>(b.raw[i][j], s0, s1, words);
#pragma unroll
      for (int st = 0; st < ST; ++st) {
        const long k = sb * F::kSB + q * F::kCK + 8 * st;
        u32x4_t av = {0u, 0u, 0u, 0u};
        if constexpr (LDS_ONLY) {
          av = *reinterpret_cast<const u32x4_t*>(arow_z + k);
        } else {
          if (arow_l) av = *reinterpret_cast<const u32x4_t*>(arow_l + k);
          else if (arow_g) av = *reinterpret_cast<const u32x4_t*>(arow_g + k);
        }
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
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = __builtin_fmaf(b.bsc[i], part[r], acc[r]);
    }
  }
}

// Finish a panel whose first batch (units [u0, u0 + D)) is already in flight
// in b0: a two-buffer pipeline keeps the next batch's loads issued while the
// current one is computed.
template <int FMT, int D, bool LDS_ONLY>
__device__ __forceinline__ f32x4_t panel_finish(WBatch<FMT, D>& b0, const PanelPos& p,
                                                const DecodeArgs& a, const uint16_t* xs,
                                                const uint16_t* xg, int na, int u0, int u1,
                                                int lane) {
  const int q = lane / 16, m = lane % 16;
  const uint16_t* arow_z = xs + (m < na ? m : a.lds_rows) * p.K_total;
  const uint16_t* arow_l = (m < na && m < a.lds_rows) ? xs + m * p.K_total : nullptr;
  const uint16_t* arow_g = (m < na && m >= a.lds_rows) ? xg + (long)m * p.K_total : nullptr;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  WBatch<FMT, D> b1;
  for (int ub = u0; ub < u1; ub += 2 * D) {
    if (ub + D < u1) issue_batch<FMT, D>(b1, p, ub + D, u1, lane);
    compute_batch<FMT, D, LDS_ONLY>(b0, acc, arow_z, arow_l, arow_g, ub, u1, q);
    if (ub + 2 * D < u1) issue_batch<FMT, D>(b0, p, ub + 2 * D, u1, lane);
    if (ub + D < u1) compute_batch<FMT, D, LDS_ONLY>(b1, acc, arow_z, arow_l, arow_g, ub + D, u1, q);
  }
  return acc;
}

// Copy rows src_row(r), r < nr, each K bf16 long, into xs; row zero_row is zero.
template <typename RowFn>
__device__ __forceinline__ void stage_rows(uint16_t* xs, int nr, int zero_row, int K,
                                           RowFn src_row) {
  const int per_row = K / 8;   // 16-byte pieces
  for (int c = threadIdx.x; c < nr * per_row; c += blockDim.x) {
    const int r = c / per_row, k = (c % per_row) * 8;
    *reinterpret_cast<u32x4_t*>(xs + r * K + k) = *reinterpret_cast<const u32x4_t*>(src_row(r) + k);
  }
  const u32x4_t z = {0u, 0u, 0u, 0u};
  for (int c = threadIdx.x; c < per_row; c += blockDim.x)
    *reinterpret_cast<u32x4_t*>(xs + zero_row * K + c * 8) = z;
}

template <int FMT, int KSPLIT, int D>
__global__ __launch_bounds__(128 * KSPLIT) void decode_gate_up_kernel(DecodeArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs_dyn[];   // kLdsRows x H
  __shared__ f32x4_t red[2 * KSPLIT][kWave];
  const int npan = a.I / 16;
  const int items = a.n_active[0] * npan;   // (active expert, gate panel) pairs
  const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int half = w / KSPLIT, ks = w % KSPLIT;
  const int nunits = a.H / 128;
  const int u0 = ks * nunits / KSPLIT, u1 = (ks + 1) * nunits / KSPLIT;
  int cur_e = -1;
  for (int it = blockIdx.x; it < items; it += gridDim.x) {   // uniform loop bound
    const int slot = it / npan, p = it % npan;
    const int e = a.active[slot];
    const int r0 = a.seg_start[e];
    const int na = min(a.seg_start[e + 1] - r0, 16);
    const int panel = half ? (npan + p) : p;
    const int ws = a.slot_map ? a.slot_map[e] : e;
    const PanelPos pos = panel_pos<FMT>(a, ws, panel, a.H, lane);
    WBatch<FMT, D> b0;
    issue_batch<FMT, D>(b0, pos, u0, u1, lane);   // in flight while the rows are staged
    if (e != cur_e) {   // uniform: stage this expert's token rows once
      __syncthreads();
      stage_rows(xs_dyn, min(na, a.lds_rows), a.lds_rows, a.H,
                 [&](int r) { return a.x + (long)a.sorted_tok[r0 + r] * a.H; });
      __syncthreads();
      cur_e = e;
    }
    const int m = lane % 16;
    const uint16_t* xg = (m < na && m >= a.lds_rows) ? a.x + (long)a.sorted_tok[r0 + m] * a.H - (long)m * a.H : nullptr;
    if (na <= a.lds_rows)   // uniform per item
      red[w][lane] = panel_finish<FMT, D, true>(b0, pos, a, xs_dyn, xg, na, u0, u1, lane);
    else
      red[w][lane] = panel_finish<FMT, D, false>(b0, pos, a, xs_dyn, xg, na, u0, u1, lane);
    __syncthreads();
    const int t = threadIdx.x;
    if (t < 256) {
      const int mm = t / 16, n = t % 16;
      if (mm < na) {
        const int l = (mm / 4) * 16 + n, i = mm % 4;
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
        act[(long)(r0 + mm) * a.I + 16 * p + n] = f32_to_bf16(silu_gate(g, u, a.limit, a.alpha, a.beta));
      }
    }
    __syncthreads();   // red is rewritten by the next item
  }
}

template <int FMT, int KSPLIT, int PPB, int D>
__global__ __launch_bounds__(64 * KSPLIT * PPB) void decode_down_kernel(DecodeArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs_dyn[];   // kLdsRows x I
  __shared__ f32x4_t red[KSPLIT * PPB][kWave];
  const int npb = a.H / 16 / PPB;
  const int items = a.n_active[0] * npb;
  const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int pp = w / KSPLIT, ks = w % KSPLIT;
  const int nunits = a.I / 128;
  const int u0 = ks * nunits / KSPLIT, u1 = (ks + 1) * nunits / KSPLIT;
  int cur_e = -1;
  for (int it = blockIdx.x; it < items; it += gridDim.x) {
    const int slot = it / npb, pb = it % npb;
    const int e = a.active[slot];
    const int r0 = a.seg_start[e];
    const int na = min(a.seg_start[e + 1] - r0, 16);
    const int ws = a.slot_map ? a.slot_map[e] : e;
    const int panel = pb * PPB + pp;
    const PanelPos pos = panel_pos<FMT>(a, ws, panel, a.I, lane);
    WBatch<FMT, D> b0;
    issue_batch<FMT, D>(b0, pos, u0, u1, lane);
    if (e != cur_e) {
      __syncthreads();
      stage_rows(xs_dyn, min(na, a.lds_rows), a.lds_rows, a.I,
                 [&](int r) { return a.x + (long)(r0 + r) * a.I; });
      __syncthreads();
      cur_e = e;
    }
    const uint16_t* xg = a.x + (long)r0 * a.I;
    if (na <= a.lds_rows)
      red[w][lane] = panel_finish<FMT, D, true>(b0, pos, a, xs_dyn, xg, na, u0, u1, lane);
    else
      red[w][lane] = panel_finish<FMT, D, false>(b0, pos, a, xs_dyn, xg, na, u0, u1, lane);
    __syncthreads();
    float gsv = 1.0f;
    if constexpr (FMT == kNVFP4) gsv = a.gs ? a.gs[ws] : 1.0f;
    float* y = reinterpret_cast<float*>(a.out);
    for (int t = threadIdx.x; t < PPB * 256; t += 64 * KSPLIT * PPB) {
      const int pq = t / 256, mm = (t % 256) / 16, n = t % 16;
      if (mm < na) {
        const int l = (mm / 4) * 16 + n, i = mm % 4;
        float v = 0.f;
#pragma unroll
        for (int k = 0; k < KSPLIT; ++k) v += red[pq * KSPLIT + k][l][i];
        y[(long)(r0 + mm) * a.H + 16 * (pb * PPB + pq) + n] = v * gsv;
      }
    }
    __syncthreads();
  }
}

template <int FMT, int NW, int UNR>
__global__ __launch_bounds__(64 * NW) void decode_down_combine_kernel(DecodeArgs a, int T,
                                                                      int out_bf16) {
  using F = WFmt<FMT>;
  constexpr int ST = F::kWords / 4;
  __shared__ float acc_s[NW][16][16];
  const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int panel = blockIdx.x;
  for (int i = threadIdx.x; i < NW * 256; i += 64 * NW) (&acc_s[0][0][0])[i] = 0.f;
  __syncthreads();
  const int nu = a.I / 128;
  const int items = a.n_active[0] * nu;
  const int q = lane / 16, tslot = lane % 16;
  const long nsbk = a.I / F::kSB;
  for (int jb = w; jb < items; jb += NW * UNR) {
    u32x4_t raw[UNR][F::kSPU];
    uint32_t sraw[UNR][F::kSPU];
    u32x4_t av[UNR][F::kSPU][ST];
    float bsc[UNR];
    int tok[UNR][4];
    float wt[UNR][4];
#pragma unroll
    for (int b = 0; b < UNR; ++b) {
      const int j = jb + b * NW;
      const bool ok = j < items;
      const int slot = ok ? j / nu : 0, u = ok ? j % nu : 0;
      const int e = a.active[slot];
      const int r0 = a.seg_start[e];
      const int na = ok ? min(a.seg_start[e + 1] - r0, 16) : 0;
      const int ws = a.slot_map ? a.slot_map[e] : e;
      const uint8_t* wp = a.w + (long)ws * a.w_estride + ((long)panel * nsbk) * 1024 + lane * 16;
      const uint8_t* sp = a.s + (long)ws * a.s_estride;
      const uint16_t* arow = tslot < na ? a.x + (long)(r0 + tslot) * a.I : nullptr;
#pragma unroll
      for (int jj = 0; jj < F::kSPU; ++jj) {
        const long sb = (long)u * F::kSPU + jj;
        const u32x4_t z = {0u, 0u, 0u, 0u};
        raw[b][jj] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wp + sb * 1024));
        if (!ok) raw[b][jj] = z;
        sraw[b][jj] = load_chunk_scale_raw<FMT>(sp, (long)panel * nsbk + sb, lane);
#pragma unroll
        for (int st = 0; st < ST; ++st) {
          av[b][jj][st] = z;
          if (arow) av[b][jj][st] = *reinterpret_cast<const u32x4_t*>(arow + sb * F::kSB + q * F::kCK + 8 * st);
        }
      }
      bsc[b] = 1.0f;
      if constexpr (FMT == kFP8)
        if (ok) bsc[b] = reinterpret_cast<const float*>(sp)[(long)(panel / 8) * (a.I / 128) + u];
      float gsv = 1.0f;
      if constexpr (FMT == kNVFP4) gsv = (ok && a.gs) ? a.gs[ws] : 1.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = 4 * q + i;
        tok[b][i] = (m < na) ? a.sorted_tok[r0 + m] : -1;
        wt[b][i] = (m < na) ? a.sorted_wts[r0 + m] * gsv : 0.f;
      }
    }
#pragma unroll
    for (int b = 0; b < UNR; ++b) {
      f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int jj = 0; jj < F::kSPU; ++jj) {
        uint32_t words[F::kWords];
        float s0, s1;
        chunk_scale<FMT>(sraw[b][jj], s0, s1);
        decode_chunk<FMT>(raw[b][jj], s0, s1, words);
#pragma unroll
        for (int st = 0; st < ST; ++st)
          c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              as_bf16x8(av[b][jj][st]),
              as_bf16x8(words[4 * st], words[4 * st + 1], words[4 * st + 2], words[4 * st + 3]),
              c, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (tok[b][i] >= 0) acc_s[w][tok[b][i]][lane % 16] += wt[b][i] * (bsc[b] * c[i]);
    }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < 256; t += 64 * NW) {
    const int m = t / 16, n = t % 16;
    if (m < T) {
      float v = 0.f;
#pragma unroll
      for (int k = 0; k < NW; ++k) v += acc_s[k][m][n];
      const long o = (long)m * a.H + 16 * panel + n;
      if (out_bf16) reinterpret_cast<uint16_t*>(a.out)[o] = f32_to_bf16(v);
      else reinterpret_cast<float*>(a.out)[o] = v;
    }
  }
}

template <int FMT>
hipError_t launch_decode(int which, DecodeArgs a, int max_active, hipStream_t stream) {
  using F = WFmt<FMT>;
  if (which == 0) {
    if (!a.w_estride) a.w_estride = F::w_bytes(2L * a.I, a.H);
    if (!a.s_estride) a.s_estride = F::s_bytes(2L * a.I, a.H);
    const int items = max_active * (a.I / 16);
    constexpr int D = FMT == kBF16 ? 2 : (FMT == kFP8 ? XTU_GU_D / 2 : XTU_GU_D);
    const size_t lds = (size_t)(a.lds_rows + 1) * a.H * sizeof(uint16_t);
    decode_gate_up_kernel<FMT, XTU_GU_KSPLIT, D>
        <<<dim3(items < XTU_GU_MAXGRID ? items : XTU_GU_MAXGRID), 128 * XTU_GU_KSPLIT, lds, stream>>>(a);
  } else {
    if (!a.w_estride) a.w_estride = F::w_bytes(a.H, a.I);
    if (!a.s_estride) a.s_estride = F::s_bytes(a.H, a.I);
    const int items = max_active * (a.H / 16 / XTU_DN_PPB);
    constexpr int D = FMT == kBF16 ? 2 : (FMT == kFP8 ? XTU_DN_D / 2 : XTU_DN_D);
    const size_t lds = (size_t)(a.lds_rows + 1) * a.I * sizeof(uint16_t);
    decode_down_kernel<FMT, XTU_DN_KSPLIT, XTU_DN_PPB, D>
        <<<dim3(items < XTU_DN_MAXGRID ? items : XTU_DN_MAXGRID), 64 * XTU_DN_KSPLIT * XTU_DN_PPB,
           lds, stream>>>(a);
  }
  return hipPeekAtLastError();
}

template <int FMT>
hipError_t launch_down_combine(DecodeArgs a, int T, int out_bf16, hipStream_t stream) {
  using F = WFmt<FMT>;
  if (!a.w_estride) a.w_estride = F::w_bytes(a.H, a.I);
  if (!a.s_estride) a.s_estride = F::s_bytes(a.H, a.I);
  constexpr int UNR = FMT == kBF16 ? 2 : 4;
  decode_down_combine_kernel<FMT, 8, UNR><<<dim3(a.H / 16), 512, 0, stream>>>(a, T, out_bf16);
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
  if (H <= 0 || I <= 0 || H % 128 || I % 128 || H > 16384 || I > 16384) return false;
  if (fmt == kFP8 && ((2 * I) % 128 || H % 128)) return false;
  return fmt >= 0 && fmt <= 3;
}

}  // namespace
}  // namespace xtu

using namespace xtu;

extern "C" {

hipError_t xtu_decode_gate_up(int fmt, const void* x, int T, int H, int I, const void* w13,
                              const void* s13, const float* gs13, long w_estride,
                              long s_estride, const int32_t* slot_map,
                              const int32_t* sorted_tok, const int32_t* seg_start,
                              const int32_t* active, const int32_t* n_active, int max_active,
                              void* act, float limit, float alpha, float beta,
                              hipStream_t stream) {
  XTU_CHECK_ARG(shape_ok(fmt, H, I) && max_active >= 0 && max_active <= 65535 && T >= 0 &&
                T <= 16);
  XTU_CHECK_ARG(w_estride >= 0 && s_estride >= 0);
  XTU_CHECK_ARG(x && w13 && (fmt == kBF16 || s13) && sorted_tok && seg_start && active &&
                n_active && act);
  if (max_active == 0) return hipSuccess;
  (void)hipGetLastError();
  DecodeArgs a{(const uint16_t*)x, (const uint8_t*)w13, (const uint8_t*)s13, gs13, sorted_tok,
               seg_start, active, n_active, slot_map, act, H, I, w_estride, s_estride, limit,
               alpha, beta};
  a.lds_rows = T < kLdsRows ? T : kLdsRows;
  return dispatch_decode(fmt, 0, a, max_active, stream);
}

hipError_t xtu_decode_down(int fmt, const void* act, int T, int H, int I, const void* w2,
                           const void* s2, const float* gs2, long w_estride, long s_estride,
                           const int32_t* slot_map, const int32_t* seg_start,
                           const int32_t* active, const int32_t* n_active, int max_active,
                           float* y, hipStream_t stream) {
  XTU_CHECK_ARG(shape_ok(fmt, H, I) && max_active >= 0 && max_active <= 65535 &&
                (H / 16) % XTU_DN_PPB == 0 && T >= 0 && T <= 16);
  XTU_CHECK_ARG(w_estride >= 0 && s_estride >= 0);
  XTU_CHECK_ARG(act && w2 && (fmt == kBF16 || s2) && seg_start && active && n_active && y);
  if (max_active == 0) return hipSuccess;
  (void)hipGetLastError();
  DecodeArgs a{(const uint16_t*)act, (const uint8_t*)w2, (const uint8_t*)s2, gs2, nullptr,
               seg_start, active, n_active, slot_map, y, H, I, w_estride, s_estride, 0.f, 1.f,
               0.f};
  a.lds_rows = T < kLdsRows ? T : kLdsRows;
  return dispatch_decode(fmt, 1, a, max_active, stream);
}

hipError_t xtu_decode_down_combine(int fmt, const void* act, int T, int H, int I, const void* w2,
                                   const void* s2, const float* gs2, long w_estride,
                                   long s_estride, const int32_t* slot_map,
                                   const int32_t* sorted_tok, const float* sorted_wts,
                                   const int32_t* seg_start, const int32_t* active,
                                   const int32_t* n_active, void* out, int out_bf16,
                                   hipStream_t stream) {
  XTU_CHECK_ARG(shape_ok(fmt, H, I) && T >= 0 && T <= 16 && w_estride >= 0 && s_estride >= 0);
  XTU_CHECK_ARG(act && w2 && (fmt == kBF16 || s2) && sorted_tok && sorted_wts && seg_start &&
                active && n_active && out);
  if (T == 0) return hipSuccess;
  (void)hipGetLastError();
  DecodeArgs a{(const uint16_t*)act, (const uint8_t*)w2, (const uint8_t*)s2, gs2, sorted_tok,
               seg_start, active, n_active, slot_map, out, H, I, w_estride, s_estride, 0.f, 1.f,
               0.f};
  a.sorted_wts = sorted_wts;
  switch (fmt) {
    case kMXFP4: return launch_down_combine<kMXFP4>(a, T, out_bf16, stream);
    case kNVFP4: return launch_down_combine<kNVFP4>(a, T, out_bf16, stream);
    case kFP8: return launch_down_combine<kFP8>(a, T, out_bf16, stream);
    case kBF16: return launch_down_combine<kBF16>(a, T, out_bf16, stream);
  }
  return hipErrorInvalidValue;
}

}  // extern "C"
