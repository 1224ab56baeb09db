// Skinny-M (decode) expert kernels: a handful of tokens per expert, so the
// layer is a weight stream.  A wave owns a contiguous range of 128-k units of
// one 16-row panel; it issues the loads of up to NU units at once (one
// contiguous KiB per format chunk: 16 bytes per lane, the P16 layout), then
// consumes them in issue order: dequantise in registers to bf16 and feed
// v_mfma_f32_16x16x32_bf16 with the expert's tokens as the 16-row A operand
// (from LDS).  The code of one round is straight-line, so every wait is for
// exactly the unit about to be used.
//
// One workgroup per work item: (active expert, gate panel) for gate/up,
// (active expert, PPB panels of W2) for down.  Expert slots beyond n_active
// exit at once; experts nobody routed to (or only with zero weight) are never
// read.  The K range of a panel is split over KSPLIT waves and reduced through
// LDS in a fixed order, so results are deterministic.  A lane whose token
// slot is empty reads any staged row: MFMA output row m depends on A row m
// only, and rows beyond the expert's token count are never written.
//
// gate/up: waves [0,KSPLIT) stream gate rows 16p.., waves [KSPLIT, 2KSPLIT)
//   the matching up rows I+16p.., so the SwiGLU of row n is formed in the
//   reduction step and only the bf16 activation row is written.
// down: y is fp32; with KSPLIT = 1 each wave writes its panel directly.
#pragma once
#include "route_tiny.hpp"
#include "weight_format.hpp"
#include <algorithm>

namespace xtu {
namespace {

constexpr int kWave = 64;
constexpr int kMaxTok = 16;             // tokens per expert on this path
constexpr int kLdsBudget = 72 * 1024;   // bytes of staged rows per workgroup
constexpr int kRegChunks = 4;           // 16-byte row pieces per thread staged through registers

struct DecodeArgs {
  const uint16_t* x;         // gate/up: hidden rows [T][H]; down: act rows [A][I]
  const uint8_t* w;          // packed weights, expert-major
  const uint8_t* s;          // fp4 scales (packed) or fp8 block scales (fp32)
  const float* gs;           // NVFP4 second-level scales: gate/up [slot][2], down [slot] (may be null)
  const int32_t* sorted_tok;
  const int32_t* seg_start;
  const int32_t* active;     // work slots: active experts, or the 16-row tiles' experts
  const int32_t* n_active;   // number of work slots
  const int32_t* slot_map;   // expert -> weight slot (null: identity)
  void* out;                 // gate/up: act bf16 [A][I]; down: y fp32 [A][H]
  const int32_t* tile_row0;  // null: slot = whole expert from seg_start; else its first row
  int T, H, I;
  long w_estride, s_estride;
  float limit, alpha, beta;
  int rows;                  // rows the LDS stage holds
  int ksplit, ppb;           // waves per panel K range; panels per workgroup (down)
  int skip;                  // gate/up fast path: trailing active slots left out
  const int32_t* pair_of;    // down: null = y row per sorted position; else y row
                             // pair_of[position] (the flat pair index)
};

// Units issued per round: about 80 VGPRs of weights in flight per wave, and
// fewer than 64 outstanding vector-memory instructions.
template <int FMT>
constexpr int round_units() {
  return FMT == kBF16 ? 4 : (FMT == kFP8 ? 8 : 16);
}

__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
}

// Buffer resource dword 3 for raw (untyped, stride-0) buffers on gfx9-class
// parts.  Loads past num_records return zero instead of touching memory.
constexpr int kRawBufferFlags = 0x00020000;
constexpr int kAuxNontemporal = 2;

// Wave-uniform buffer descriptors of one panel's weight stream.
template <int FMT>
struct Stream {
  __amdgpu_buffer_rsrc_t w;   // the panel's super-blocks
  __amdgpu_buffer_rsrc_t s;   // fp4: the panel's scale groups; fp8: its block-scale row
};

// live = false: zero-length ranges (loads return 0 without touching memory).
template <int FMT>
__device__ __forceinline__ Stream<FMT> make_stream(const DecodeArgs& a, int ws, int panel, int K,
                                                   bool live = true) {
  using F = WFmt<FMT>;
  const long nsb = K / F::kSB;
  const uint8_t* sx = a.s + (long)ws * a.s_estride;
  Stream<FMT> st;
  st.w = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.w + (long)ws * a.w_estride + (long)panel * nsb * 1024), 0,
      live ? (int)(nsb * 1024) : 0, kRawBufferFlags);
  if constexpr (FMT == kMXFP4 || FMT == kNVFP4) {
    const long gbytes = scale_groups(K, F::kUG) * 1024;
    st.s = __builtin_amdgcn_make_buffer_rsrc((void*)(sx + (long)panel * gbytes), 0,
                                             live ? (int)gbytes : 0, kRawBufferFlags);
  } else if constexpr (FMT == kFP8) {
    st.s = __builtin_amdgcn_make_buffer_rsrc((void*)(sx + (long)(panel / 8) * (K / 128) * 4), 0,
                                             live ? (K / 128) * 4 : 0, kRawBufferFlags);
  } else {
    st.s = st.w;
  }
  return st;
}

// One round of one lane: the weight chunks of NU units and their scales.
// fp4: the 16-byte scale groups covering the round, rotated so that unit i's
// scale sits at byte i * kSBY of sw; fp8: lane l holds the block scale of
// unit ub + l.
template <int FMT, int NU>
struct Round {
  using F = WFmt<FMT>;
  static constexpr int kGroups = F::kSBY ? (15 + NU * F::kSBY + 15) / 16 : 0;
  u32x4_t w[NU][F::kSPU];
  uint32_t sw[kGroups > 0 ? 4 * kGroups : 1];
  float bsv;
};

// Loads of the round [ub, min(ub + NU, u1)): scales first, then weights, all
// unconditional (an index past the range re-reads unit u1 - 1, which is never
// consumed twice), so the wait counts stay exact.
template <int FMT, int NU>
__device__ __forceinline__ void issue_round(Round<FMT, NU>& r, const Stream<FMT>& st, int ub,
                                            int u1, uint32_t lane) {
  using F = WFmt<FMT>;
  if constexpr (Round<FMT, NU>::kGroups > 0) {
    const int g0 = ub / F::kUG;
#pragma unroll
    for (int j = 0; j < Round<FMT, NU>::kGroups; ++j) {
      const u32x4_t v = __builtin_bit_cast(
          u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(st.s, (int)lane * 16, (g0 + j) * 1024,
                                                         kAuxNontemporal));
      r.sw[4 * j] = v[0];
      r.sw[4 * j + 1] = v[1];
      r.sw[4 * j + 2] = v[2];
      r.sw[4 * j + 3] = v[3];
    }
  } else if constexpr (FMT == kFP8) {
    r.bsv = __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(st.s, (int)lane * 4, ub * 4, 0));
  }
#pragma unroll
  for (int i = 0; i < NU; ++i) {
    const int u = ub + i < u1 ? ub + i : u1 - 1;
#pragma unroll
    for (int j = 0; j < F::kSPU; ++j)
      r.w[i][j] = __builtin_bit_cast(
          u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(st.w, (int)lane * 16,
                                                         (u * F::kSPU + j) * 1024,
                                                         kAuxNontemporal));
  }
}

// Shift the scale words down by `off` bytes (wave-uniform, 0..15).
template <int N>
__device__ __forceinline__ void shift_bytes_down(uint32_t (&v)[N], int off) {
  if (off & 4) {
#pragma unroll
    for (int j = 0; j < N - 1; ++j) v[j] = v[j + 1];
    v[N - 1] = 0u;
  }
  if (off & 8) {
#pragma unroll
    for (int j = 0; j < N - 2; ++j) v[j] = v[j + 2];
    v[N - 2] = v[N - 1] = 0u;
  }
  const int b = off & 3;
  if (b) {
#pragma unroll
    for (int j = 0; j < N - 1; ++j) v[j] = __builtin_amdgcn_alignbyte(v[j + 1], v[j], b);
    v[N - 1] >>= 8 * b;
  }
}

// acc += x_rows (16 x 128) * W_unit^T (128 x 16) for unit u.  The A fragment
// of lane (q, m) for step st of super-block j is row m at k = kb + q*kCK +
// 8*st; xa points at that row's k = q*kCK in LDS, xg (if set) at the same
// place in global memory for a row the stage does not hold.
template <int FMT, bool LDS_ONLY>
__device__ __forceinline__ void mma_unit(const u32x4_t (&w)[WFmt<FMT>::kSPU], uint32_t sraw,
                                         float bs, f32x4_t& acc, int u, const uint16_t* xa,
                                         const uint16_t* xg) {
  using F = WFmt<FMT>;
  constexpr int ST = F::kWords / 4;
  f32x4_t part = {0.f, 0.f, 0.f, 0.f};
  float s0, s1;
  chunk_scale<FMT>(sraw, s0, s1);
#pragma unroll
  for (int j = 0; j < F::kSPU; ++j) {
    uint32_t words[F::kWords];
    decode_chunk<FMT>(w[j], s0, s1, words);
    const int kb = (u * F::kSPU + j) * F::kSB;
#pragma unroll
    for (int st = 0; st < ST; ++st) {
      u32x4_t av;
      if constexpr (LDS_ONLY) {
        av = *reinterpret_cast<const u32x4_t*>(xa + kb + 8 * st);
      } else {
        if (xg) av = *reinterpret_cast<const u32x4_t*>(xg + kb + 8 * st);
        else av = *reinterpret_cast<const u32x4_t*>(xa + kb + 8 * st);
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
    for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(bs, part[i], acc[i]);
  }
}

template <int FMT, int NU, bool LDS_ONLY>
__device__ __forceinline__ void consume_round(Round<FMT, NU>& r, f32x4_t& acc, int ub, int u1,
                                              const uint16_t* xa, const uint16_t* xg) {
  using F = WFmt<FMT>;
  if constexpr (Round<FMT, NU>::kGroups > 0) shift_bytes_down(r.sw, (ub % F::kUG) * F::kSBY);
#pragma unroll
  for (int i = 0; i < NU; ++i) {
    if (ub + i < u1) {
      uint32_t sraw = 0u;
      float bs = 1.0f;
      if constexpr (FMT == kMXFP4) sraw = r.sw[i / 4] >> (8 * (i % 4));
      else if constexpr (FMT == kNVFP4) sraw = r.sw[i / 2] >> (16 * (i % 2));
      else if constexpr (FMT == kFP8)
        bs = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, r.bsv), i));
      mma_unit<FMT, LDS_ONLY>(r.w[i], sraw, bs, acc, ub + i, xa, xg);
    }
  }
}

// Rounds after the first (shapes with more than NU units per wave).
template <int FMT, int NU, bool LDS_ONLY>
__device__ __forceinline__ f32x4_t more_rounds(f32x4_t acc, const Stream<FMT>& st, int ub, int u1,
                                               uint32_t lane, const uint16_t* xa,
                                               const uint16_t* xg) {
  for (; ub < u1; ub += NU) {
    Round<FMT, NU> r;
    issue_round<FMT, NU>(r, st, ub, u1, lane);
    consume_round<FMT, NU, LDS_ONLY>(r, acc, ub, u1, xa, xg);
  }
  return acc;
}

struct Item {
  int e, r0, na, ws, sub;
};

__device__ __forceinline__ Item item_at(const DecodeArgs& a, int it, int per_expert) {
  Item c;
  const int slot = it / per_expert;
  c.sub = it - slot * per_expert;
  c.e = a.active[slot];
  c.r0 = a.tile_row0 ? a.tile_row0[slot] : a.seg_start[c.e];
  c.na = min(a.seg_start[c.e + 1] - c.r0, kMaxTok);
  c.ws = a.slot_map ? a.slot_map[c.e] : c.e;
  return c;
}

// Store the register-staged row pieces (piece index threadIdx.x + j*blockDim)
// and copy any remaining pieces directly.
template <typename SrcFn>
__device__ __forceinline__ void finish_stage(uint16_t* xs, const u32x4_t (&xv)[kRegChunks],
                                             int nchunks, SrcFn src) {
#pragma unroll
  for (int j = 0; j < kRegChunks; ++j) {
    const int c = threadIdx.x + j * blockDim.x;
    if (c < nchunks) *reinterpret_cast<u32x4_t*>(xs + c * 8) = xv[j];
  }
  for (int c = threadIdx.x + kRegChunks * blockDim.x; c < nchunks; c += blockDim.x)
    *reinterpret_cast<u32x4_t*>(xs + c * 8) = *reinterpret_cast<const u32x4_t*>(src(c));
}

// Reduce the gate (waves [0, ksplit)) and up (waves [ksplit, 2 ksplit)) K
// splits in a fixed order and write the expert's na SwiGLU rows of panel sub.
// COH: device-coherent stores (read by other workgroups in the same launch).
template <int FMT, bool COH = false>
__device__ __forceinline__ void gate_up_epilogue(const DecodeArgs& a, f32x4_t (*red)[kWave],
                                                 f32x4_t acc, int w, uint32_t lane, int r0,
                                                 int na, int ws, int sub) {
  red[w][lane] = acc;
  __syncthreads();
  for (int t = threadIdx.x; t < 256; t += blockDim.x) {   // 16 rows x 16 columns
    const int mm = t / 16, n = t % 16;
    if (mm < na) {
      const int l = (mm / 4) * 16 + n, i = mm % 4;
      float g = 0.f, u = 0.f;
      for (int k = 0; k < a.ksplit; ++k) {
        g += red[k][l][i];
        u += red[a.ksplit + k][l][i];
      }
      if constexpr (FMT == kNVFP4) {   // second-level scales [slot][2]: gate, up
        if (a.gs) {
          g *= a.gs[2 * ws];
          u *= a.gs[2 * ws + 1];
        }
      }
      uint16_t* act = reinterpret_cast<uint16_t*>(a.out);
      const uint16_t v = f32_to_bf16(silu_gate(g, u, a.limit, a.alpha, a.beta));
      if constexpr (COH)
        __hip_atomic_store(act + (long)(r0 + mm) * a.I + 16 * sub + n, v, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      else
        act[(long)(r0 + mm) * a.I + 16 * sub + n] = v;
    }
  }
}

// GENERIC: more than one round per wave, or token rows beyond the stage; the
// fast instantiation holds neither (the host checks the shape) and stages the
// batch's T rows through XC register pieces per thread.
template <int FMT, bool GENERIC, int XC>
__global__ __launch_bounds__(512) void decode_gate_up_kernel(DecodeArgs a) {
  using F = WFmt<FMT>;
  constexpr int NU = round_units<FMT>();
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];   // rows x H
  __shared__ f32x4_t red[8][kWave];
  const int npan = a.I / 16;
  const int ksplit = a.ksplit;
  const int w = wave_id();
  const uint32_t lane = threadIdx.x % kWave;
  const int half = w / ksplit, ks = w - half * ksplit;
  const int nunits = a.H / 128;
  const int u0 = ks * nunits / ksplit, u1 = (ks + 1) * nunits / ksplit;
  const int q = lane / 16, m = lane % 16;
  const int per_row = a.H / 8;        // 16-byte pieces per row
  Round<FMT, NU> r;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  if constexpr (!GENERIC) {
    // Every token row of the batch is staged (x rows 0..T-1 are contiguous).
    // Issue order: the active count and the slot's expert (scalar, one
    // level), the rows, the weights (zero-length ranges for a slot past the
    // active count, which then exits), then the expert's row range and lane
    // m's token; the row stores wait for the rows only and the units are
    // consumed as they arrive.
    const int slot = blockIdx.x / npan, sub = blockIdx.x - slot * npan;
    const int nact = a.n_active[0];
    const int e_raw = a.active[slot];
    const int nchunks = a.T * per_row;
    u32x4_t xv[XC];
#pragma unroll
    for (int j = 0; j < XC; ++j) {
      const int cc = min((int)threadIdx.x + j * (int)blockDim.x, nchunks - 1);
      xv[j] = *reinterpret_cast<const u32x4_t*>(a.x + (long)cc * 8);
    }
    const bool live = slot < nact - a.skip;
    const int e = live ? e_raw : 0;
    const int ws = live && a.slot_map ? a.slot_map[e] : e;
    const Stream<FMT> st = make_stream<FMT>(a, ws, half ? npan + sub : sub, a.H, live);
    __builtin_amdgcn_sched_barrier(0);
    issue_round<FMT, NU>(r, st, u0, u1, lane);
    __builtin_amdgcn_sched_barrier(0);
    if (!live) return;   // whole workgroup
    const int r0 = a.tile_row0 ? a.tile_row0[slot] : a.seg_start[e];
    const int na = min(a.seg_start[e + 1] - r0, kMaxTok);
    const int tok = a.sorted_tok[r0 + min(m, na - 1)];
#pragma unroll
    for (int j = 0; j < XC; ++j) {
      const int cc = threadIdx.x + j * blockDim.x;
      if (cc < nchunks) *reinterpret_cast<u32x4_t*>(xs + cc * 8) = xv[j];
    }
    __syncthreads();
    consume_round<FMT, NU, true>(r, acc, u0, u1, xs + tok * a.H + q * F::kCK, nullptr);
    gate_up_epilogue<FMT>(a, red, acc, w, lane, r0, na, ws, sub);
    return;
  } else {
    if ((int)blockIdx.x >= a.n_active[0] * npan) return;   // whole workgroup
    const Item c = item_at(a, blockIdx.x, npan);
    const Stream<FMT> st = make_stream<FMT>(a, c.ws, half ? npan + c.sub : c.sub, a.H);
    // the expert's first `rows` token rows are staged, the rest read from
    // global memory; more than one round per wave when K needs it
    const int nr = min(c.na, a.rows);
    const int nchunks = nr * per_row;
    int trow[kRegChunks];
#pragma unroll
    for (int j = 0; j < kRegChunks; ++j) {
      const int cc = min((int)threadIdx.x + j * (int)blockDim.x, nchunks - 1);
      trow[j] = a.sorted_tok[c.r0 + cc / per_row];
    }
    __builtin_amdgcn_sched_barrier(0);   // keep the issue order: ids, weights, rows
    issue_round<FMT, NU>(r, st, u0, u1, lane);
    __builtin_amdgcn_sched_barrier(0);
    u32x4_t xv[kRegChunks];
#pragma unroll
    for (int j = 0; j < kRegChunks; ++j) {
      const int cc = min((int)threadIdx.x + j * (int)blockDim.x, nchunks - 1);
      xv[j] = *reinterpret_cast<const u32x4_t*>(a.x + (long)trow[j] * a.H + (cc % per_row) * 8);
    }
    finish_stage(xs, xv, nchunks, [&](int cc) {
      return a.x + (long)a.sorted_tok[c.r0 + cc / per_row] * a.H + (cc % per_row) * 8;
    });
    __syncthreads();
    const uint16_t* xa = xs + (m < nr ? m : 0) * a.H + q * F::kCK;
    if (c.na <= nr) {   // uniform: every token row is staged
      consume_round<FMT, NU, true>(r, acc, u0, u1, xa, nullptr);
      if (u0 + NU < u1) acc = more_rounds<FMT, NU, true>(acc, st, u0 + NU, u1, lane, xa, nullptr);
    } else {
      const uint16_t* xg =
          (m < c.na && m >= nr) ? a.x + (long)a.sorted_tok[c.r0 + m] * a.H + q * F::kCK : nullptr;
      consume_round<FMT, NU, false>(r, acc, u0, u1, xa, xg);
      if (u0 + NU < u1) acc = more_rounds<FMT, NU, false>(acc, st, u0 + NU, u1, lane, xa, xg);
    }
    gate_up_epilogue<FMT>(a, red, acc, w, lane, c.r0, c.na, c.ws, c.sub);
  }
}

// Routing + segmentation (workgroup 0, tiny::route_segment_block) and the
// shared experts' gate/up (workgroups 1.., one per (shared expert, gate
// panel)) in one launch: a shared expert needs no routing, so its weight
// stream runs beside the router instead of after it.  Its act rows go to
// act_sh [n_shared][T][I] (token order), since their sorted positions are
// known only once the batch is routed; the routed gate/up then leaves the
// shared slots out (DecodeArgs::skip) and the fused down reads them from
// act_sh.  The gate/up part is decode_gate_up_kernel's fast path with all T
// rows of the batch as the expert's rows.
template <int FMT, int MODE, int EPL, int XC>
__global__ __launch_bounds__(512) void decode_route_shared_kernel(tiny::SmallArgs ra,
                                                                  DecodeArgs a) {
  using F = WFmt<FMT>;
  constexpr int NU = round_units<FMT>();
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];   // T rows x H
  __shared__ f32x4_t red[8][kWave];
  __shared__ __attribute__((aligned(16))) tiny::TinySmem g;
  if (blockIdx.x == 0) {
    tiny::route_segment_block<MODE, EPL>(ra, g);
    return;
  }
  const int npan = a.I / 16;
  const int item = blockIdx.x - 1;
  const int sh = item / npan, sub = item - sh * npan;
  const int e = ra.E + sh;
  const int ws = a.slot_map ? a.slot_map[e] : e;
  const int ksplit = a.ksplit;
  const int w = wave_id();
  const uint32_t lane = threadIdx.x % kWave;
  const int half = w / ksplit, ks = w - half * ksplit;
  const int nunits = a.H / 128;
  const int u0 = ks * nunits / ksplit, u1 = (ks + 1) * nunits / ksplit;
  const int q = lane / 16, m = lane % 16;
  const int nchunks = a.T * (a.H / 8);
  u32x4_t xv[XC];
#pragma unroll
  for (int j = 0; j < XC; ++j) {
    const int cc = min((int)threadIdx.x + j * (int)blockDim.x, nchunks - 1);
    xv[j] = *reinterpret_cast<const u32x4_t*>(a.x + (long)cc * 8);
  }
  const Stream<FMT> st = make_stream<FMT>(a, ws, half ? npan + sub : sub, a.H);
  Round<FMT, NU> r;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  __builtin_amdgcn_sched_barrier(0);
  issue_round<FMT, NU>(r, st, u0, u1, lane);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < XC; ++j) {
    const int cc = threadIdx.x + j * blockDim.x;
    if (cc < nchunks) *reinterpret_cast<u32x4_t*>(xs + cc * 8) = xv[j];
  }
  __syncthreads();
  const int tok = min(m, a.T - 1);
  consume_round<FMT, NU, true>(r, acc, u0, u1, xs + tok * a.H + q * F::kCK, nullptr);
  gate_up_epilogue<FMT>(a, red, acc, w, lane, sh * a.T, a.T, ws, sub);
}

// Routing, segmentation and every gate/up of a decode batch in one launch.
// Workgroups [0, n_sh): the shared experts' gate/up panels when they are
// split off (rows to act_sh, as decode_route_shared_kernel writes them); the
// rest route and segment the whole batch for themselves in LDS
// (tiny::route_segment_block with STORE = false; the first one also stores
// the routing and the segmentation for the down pass), stage the batch's x
// rows once, then take (16-row tile, gate panel) work items item0, item0 +
// stride, ... of the batch, each streamed as decode_gate_up_kernel's fast
// path does.  Launched with about one resident round of these workgroups,
// so the routing is done once per workgroup, beside the first weight
// streams, and the routing launch and its boundary are gone.  skip: tiles at
// the end of the tile list left out (the split-off shared experts' own).
// ROUTE_ALL: the shared-expert workgroups route the batch too, after their
// gate/up item (the one-launch layer's down phase reads the routing from
// every workgroup's LDS).
template <int FMT, int MODE, int EPL, int XC, bool ROUTE_ALL>
__device__ __forceinline__ void route_gate_up_phase(const tiny::SmallArgs& ra, DecodeArgs a,
                                                    void* act_sh, int n_sh, int skip,
                                                    uint16_t* xs, f32x4_t (*red)[kWave],
                                                    tiny::TinySmem& g) {
  using F = WFmt<FMT>;
  constexpr int NU = round_units<FMT>();
  const int npan = a.I / 16;
  const int ksplit = a.ksplit;
  const int w = wave_id();
  const uint32_t lane = threadIdx.x % kWave;
  const int half = w / ksplit, ks = w - half * ksplit;
  const int nunits = a.H / 128;
  const int u0 = ks * nunits / ksplit, u1 = (ks + 1) * nunits / ksplit;
  const int q = lane / 16, m = lane % 16;
  const int nchunks = a.T * (a.H / 8);
  // The batch's rows, all pieces in flight at once.  A shared-expert
  // workgroup stores them to LDS before its weight stream (their registers
  // are then free for it); a routed one keeps up to two pieces per thread in
  // flight during the routing and stores them after it (more, or NVFP4's
  // wider dequantisation beside them, would cost a wave per SIMD).  They are
  // read only after a barrier.
  constexpr bool kLateX = XC <= 2 && FMT != kNVFP4;
  u32x4_t xv[XC];
#pragma unroll
  for (int j = 0; j < XC; ++j) {
    const int cc = min((int)threadIdx.x + j * (int)blockDim.x, nchunks - 1);
    xv[j] = *reinterpret_cast<const u32x4_t*>(a.x + (long)cc * 8);
  }
  auto stage_x = [&]() {
#pragma unroll
    for (int j = 0; j < XC; ++j) {
      const int cc = threadIdx.x + j * blockDim.x;
      if (cc < nchunks) *reinterpret_cast<u32x4_t*>(xs + cc * 8) = xv[j];
    }
  };
  if constexpr (!kLateX) stage_x();
  if ((int)blockIdx.x < n_sh) {
    if constexpr (kLateX) stage_x();
    // a shared expert: all T rows of the batch, in token order, no routing
    const int sh = blockIdx.x / npan, sub = blockIdx.x - sh * npan;
    const int e = ra.E + sh;
    const int ws = a.slot_map ? a.slot_map[e] : e;
    const Stream<FMT> st = make_stream<FMT>(a, ws, half ? npan + sub : sub, a.H);
    Round<FMT, NU> r;
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    __builtin_amdgcn_sched_barrier(0);
    issue_round<FMT, NU>(r, st, u0, u1, lane);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    consume_round<FMT, NU, true>(r, acc, u0, u1, xs + min(m, a.T - 1) * a.H + q * F::kCK,
                                 nullptr);
    a.out = act_sh;
    gate_up_epilogue<FMT, ROUTE_ALL>(a, red, acc, w, lane, sh * a.T, a.T, ws, sub);
    if constexpr (ROUTE_ALL) tiny::route_segment_block<MODE, EPL, false>(ra, g);
    return;
  }
  const int first = blockIdx.x - n_sh, stride = gridDim.x - n_sh;
  if (first == 0) tiny::route_segment_block<MODE, EPL, true>(ra, g);
  else tiny::route_segment_block<MODE, EPL, false>(ra, g);
  const int items = (g.act_t[g.n_act] - skip) * npan;
  if (first >= items) return;   // whole workgroup
  if constexpr (kLateX) stage_x();
  // The next item's weights are issued before this item's epilogue, whose
  // row stores would otherwise sit in front of them in the wave's in-order
  // memory counter.
  auto issue = [&](Round<FMT, NU>& rr, int it, int& ws_out) {
    const int slot = it / npan, sub = it - slot * npan;
    const int e = g.tile_e[slot];
    ws_out = a.slot_map ? a.slot_map[e] : e;
    const Stream<FMT> st = make_stream<FMT>(a, ws_out, half ? npan + sub : sub, a.H);
    __builtin_amdgcn_sched_barrier(0);
    issue_round<FMT, NU>(rr, st, u0, u1, lane);
    __builtin_amdgcn_sched_barrier(0);
  };
  Round<FMT, NU> r;
  int item = first, ws = 0;
  issue(r, item, ws);
  __syncthreads();   // the staged rows
  while (true) {
    const int slot = item / npan, sub = item - slot * npan;
    const int r0 = g.tile_r[slot], na = g.tile_n[slot];
    const int tok = g.stok[r0 + min(m, na - 1)];
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    consume_round<FMT, NU, true>(r, acc, u0, u1, xs + tok * a.H + q * F::kCK, nullptr);
    const int next = item + stride, ws_cur = ws;
    if (next < items) issue(r, next, ws);
    gate_up_epilogue<FMT, ROUTE_ALL>(a, red, acc, w, lane, r0, na, ws_cur, sub);
    if (next >= items) break;
    __syncthreads();   // red is read back before the next item writes it
    item = next;
  }
}

template <int FMT, int MODE, int EPL, int XC>
__global__ __launch_bounds__(512) void decode_route_gate_up_kernel(tiny::SmallArgs ra,
                                                                   DecodeArgs a, void* act_sh,
                                                                   int n_sh, int skip) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];   // T rows x H
  __shared__ f32x4_t red[8][kWave];
  __shared__ __attribute__((aligned(16))) tiny::TinySmem g;
  route_gate_up_phase<FMT, MODE, EPL, XC, false>(ra, a, act_sh, n_sh, skip, xs, red, g);
}

template <int FMT, bool GENERIC>
__global__ __launch_bounds__(256) void decode_down_kernel(DecodeArgs a) {
  using F = WFmt<FMT>;
  constexpr int NU = round_units<FMT>();
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];   // rows x I
  __shared__ f32x4_t red[4][kWave];
  const int ppb = a.ppb, ksplit = a.ksplit;
  const int npb = a.H / 16 / ppb;
  if ((int)blockIdx.x >= a.n_active[0] * npb) return;
  const int w = wave_id();
  const uint32_t lane = threadIdx.x % kWave;
  const int pp = w / ksplit, ks = w - pp * ksplit;
  const int nunits = a.I / 128;
  const int u0 = ks * nunits / ksplit, u1 = (ks + 1) * nunits / ksplit;
  const int q = lane / 16, m = lane % 16;
  const Item c = item_at(a, blockIdx.x, npb);
  const int nr = min(c.na, a.rows);
  const int nchunks = nr * (a.I / 8);   // the expert's rows are contiguous
  const uint16_t* xsrc = a.x + (long)c.r0 * a.I;

  u32x4_t xv[kRegChunks];
#pragma unroll
  for (int j = 0; j < kRegChunks; ++j) {
    const int cc = min((int)threadIdx.x + j * (int)blockDim.x, nchunks - 1);
    xv[j] = *reinterpret_cast<const u32x4_t*>(xsrc + cc * 8);
  }
  // y row of each of the tile's rows, loaded with the rows (before the
  // weights, so waiting for it does not wait for them)
  __shared__ int yrow[kMaxTok];
  int yr = c.r0 + (int)threadIdx.x;
  if (a.pair_of && (int)threadIdx.x < c.na) yr = a.pair_of[c.r0 + threadIdx.x];
  const int panel = c.sub * ppb + pp;
  const Stream<FMT> st = make_stream<FMT>(a, c.ws, panel, a.I);
  Round<FMT, NU> r;
  __builtin_amdgcn_sched_barrier(0);   // keep the issue order: rows, weights
  issue_round<FMT, NU>(r, st, u0, u1, lane);
  __builtin_amdgcn_sched_barrier(0);
  finish_stage(xs, xv, nchunks, [&](int cc) { return xsrc + cc * 8; });
  if (threadIdx.x < kMaxTok) yrow[threadIdx.x] = yr;
  __syncthreads();

  const uint16_t* xa = xs + (m < nr ? m : 0) * a.I + q * F::kCK;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  if (!GENERIC && c.na <= nr) {   // one round, every row staged
    consume_round<FMT, NU, true>(r, acc, u0, u1, xa, nullptr);
  } else if (c.na <= nr) {
    consume_round<FMT, NU, true>(r, acc, u0, u1, xa, nullptr);
    if (u0 + NU < u1) acc = more_rounds<FMT, NU, true>(acc, st, u0 + NU, u1, lane, xa, nullptr);
  } else {
    const uint16_t* xg = (m < c.na && m >= nr) ? xsrc + (long)m * a.I + q * F::kCK : nullptr;
    consume_round<FMT, NU, false>(r, acc, u0, u1, xa, xg);
    if (u0 + NU < u1) acc = more_rounds<FMT, NU, false>(acc, st, u0 + NU, u1, lane, xa, xg);
  }
  float gsv = 1.0f;
  if constexpr (FMT == kNVFP4) gsv = a.gs ? a.gs[c.ws] : 1.0f;
  float* y = reinterpret_cast<float*>(a.out);
  if (ksplit == 1) {   // uniform: this wave holds the whole panel
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int mm = 4 * q + i;
      if (mm < c.na) y[(long)yrow[mm] * a.H + 16 * panel + m] = acc[i] * gsv;
    }
    return;
  }
  red[w][lane] = acc;
  __syncthreads();
  for (int t = threadIdx.x; t < ppb * 256; t += blockDim.x) {
    const int pq = t / 256, mm = (t % 256) / 16, n = t % 16;
    if (mm < c.na) {
      const int l = (mm / 4) * 16 + n, i = mm % 4;
      float v = 0.f;
      for (int k = 0; k < ksplit; ++k) v += red[pq * ksplit + k][l][i];
      y[(long)yrow[mm] * a.H + 16 * (c.sub * ppb + pq) + n] = v * gsv;
    }
  }
}

// ---------------------------------------------------------------------------
// Down projection with the weighted combine fused (moe4_smallm_dn2's
// Y[t] += w * (act_e W2_e^T)[t], computed without atomics).  The MFMA's 16 A
// rows are the batch's tokens (T <= 16): for active expert j, row t is the act
// row of pair (t, j) or any staged row when t did not route to j, and the
// result row t is added to token t's accumulator with the pair's weight (no
// addition when the weight is 0 or t has no pair on j; a token listing j
// twice has the weights summed, its two act rows being the same).  Token t's
// sum runs over its experts in active-slot order, so it does not depend on
// the other tokens.
//
// Workgroup: PPB panels of 16 output columns x KS waves; wave (p, ks) owns
// the units [ks*NPER, (ks+1)*NPER) of panel p for every active expert, with
// the loads of D experts in flight (a ring of registers; the slots past the
// active count get zero-length buffers, so the loads stay unconditional and
// the waits exact without touching memory).  All active act rows are staged
// in LDS once per workgroup; the KS partial sums are added in a fixed order.
struct DownCombineArgs {
  const uint16_t* act;        // [rows][I] bf16, sorted pair rows
  const uint8_t* w;
  const uint8_t* s;
  const float* gs;
  const int32_t* sorted_tok;
  const float* sorted_wts;
  const int32_t* seg_start;
  const int32_t* active;
  const int32_t* n_active;
  const int32_t* slot_map;
  void* out;                  // [T][H] bf16 or fp32
  int out_bf16;
  int T, H, I;
  int trash;                  // bucket after the last expert: seg_start[trash] = live rows
  int max_active;             // table capacity (>= n_active)
  int row_cap;                // sorted rows staged (>= the rows of every staged bucket)
  long w_estride, s_estride;
  int ks, ppb;
  const uint16_t* act_sh;     // shared experts' act rows [n_shared][T][I] (or null)
  int n_shared;               // buckets trash - n_shared .. trash - 1 are shared
};

constexpr int kDcTok = 16;    // tokens = MFMA rows
constexpr int kDcSB = 12;     // act pieces per thread in flight while staging
constexpr int kDcSegW = 4;    // bucket starts per thread in the first batch
constexpr size_t kDcLds = 80 * 1024;   // two workgroups per CU

// Waves the fused down's grid aims at (K split grows until reached).
#ifndef XTU_DC_WAVES
#define XTU_DC_WAVES 1024
#endif

template <int FMT, int NPER>
struct ExpLoad {
  u32x4_t w[NPER][WFmt<FMT>::kSPU];
  uint32_t sc0, sc1;          // fp4: the scale bytes of units u0.. (low byte first)
  float bsv;                  // fp8: lane l holds the block scale of unit u0 + l
};

template <int FMT, int NPER>
__device__ __forceinline__ void issue_expert(ExpLoad<FMT, NPER>& r, const DownCombineArgs& a,
                                             int ws, bool live, int panel, int u0,
                                             uint32_t lane) {
  using F = WFmt<FMT>;
  const long nsb = a.I / F::kSB;
  const uint8_t* sx = a.s + (long)ws * a.s_estride;
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.w + (long)ws * a.w_estride + (long)panel * nsb * 1024), 0,
      live ? (int)(nsb * 1024) : 0, kRawBufferFlags);
  if constexpr (FMT == kMXFP4 || FMT == kNVFP4) {
    const long gbytes = scale_groups(a.I, F::kUG) * 1024;
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(sx + (long)panel * gbytes), 0, live ? (int)gbytes : 0, kRawBufferFlags);
    // the NPER units' bytes sit in one 8-byte-aligned word of the lane's group
    const int off = (u0 % F::kUG) * F::kSBY;
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(
        sr, (int)lane * 16 + (off & 8), (u0 / F::kUG) * 1024, kAuxNontemporal);
    const uint64_t q = ((uint64_t)v[1] << 32 | v[0]) >> (8 * (off & 7));
    r.sc0 = (uint32_t)q;
    r.sc1 = (uint32_t)(q >> 32);
  } else if constexpr (FMT == kFP8) {
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(sx + (long)(panel / 8) * (a.I / 128) * 4), 0, live ? (a.I / 128) * 4 : 0,
        kRawBufferFlags);
    r.bsv = __builtin_bit_cast(float,
                               __builtin_amdgcn_raw_buffer_load_b32(sr, (int)lane * 4, u0 * 4, 0));
  }
#pragma unroll
  for (int i = 0; i < NPER; ++i)
#pragma unroll
    for (int j = 0; j < F::kSPU; ++j)
      r.w[i][j] = __builtin_bit_cast(
          u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(wr, (int)lane * 16,
                                                         ((u0 + i) * F::kSPU + j) * 1024,
                                                         kAuxNontemporal));
}

template <int FMT, int NPER>
__device__ __forceinline__ f32x4_t consume_expert(const ExpLoad<FMT, NPER>& r, int u0,
                                                  const uint16_t* xa) {
  f32x4_t pe = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < NPER; ++i) {
    uint32_t sraw = 0u;
    float bs = 1.0f;
    if constexpr (FMT == kMXFP4) {
      sraw = (i < 4 ? r.sc0 : r.sc1) >> (8 * (i % 4));
    } else if constexpr (FMT == kNVFP4) {
      sraw = (i < 2 ? r.sc0 : r.sc1) >> (16 * (i % 2));
    } else if constexpr (FMT == kFP8) {
      bs = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, r.bsv), i));
    }
    mma_unit<FMT, true>(r.w[i], sraw, bs, pe, u0 + i, xa, nullptr);
  }
  return pe;
}

// Ring depth in experts: about NU/2 units of weights in flight per wave
// (at most 128 VGPRs, so two 8-wave workgroups fit a CU).
#ifndef XTU_DC_RING_DIV
#define XTU_DC_RING_DIV 2
#endif
template <int FMT, int NPER>
constexpr int dc_depth() {
  constexpr int d = round_units<FMT>() / XTU_DC_RING_DIV / NPER;
  return d > 2 ? d : 2;
}

template <int FMT, int NPER>
__global__ __launch_bounds__(512) void decode_down_combine_kernel(DownCombineArgs a) {
  using F = WFmt<FMT>;
  constexpr int D = dc_depth<FMT, NPER>();
  extern __shared__ __attribute__((aligned(16))) uint8_t dyn[];
  const int ldx = a.I + 8;                       // staged row stride (bf16), 16 B of padding
  const int nseg = a.trash + 2;                  // seg_start entries
  const int sh_rows = a.act_sh ? a.n_shared * a.T : 0;   // staged after the sorted rows
  uint16_t* xs = reinterpret_cast<uint16_t*>(dyn);
  int* rowof = reinterpret_cast<int*>(dyn + (size_t)(a.row_cap + sh_rows) * ldx * 2);   // [max_active][16]
  float* wof = reinterpret_cast<float*>(rowof + a.max_active * kDcTok);      // [max_active][16]
  int* eslot = reinterpret_cast<int*>(wof + a.max_active * kDcTok);          // [max_active]
  int* l_act = eslot + a.max_active;                                         // [max_active]
  int* l_seg = l_act + a.max_active;                                         // [nseg]
  int* rtok = l_seg + nseg;                                                  // [row_cap]
  float* rw = reinterpret_cast<float*>(rtok + a.row_cap);                    // [row_cap]
  const int tid = threadIdx.x, bd = blockDim.x;
  const int w = wave_id();
  const uint32_t lane = tid % kWave;
  const int q = lane / 16, m = lane % 16;
  const int pp = w / a.ks, ks = w - pp * a.ks;
  const int panel = blockIdx.x * a.ppb + pp;
  const int u0 = ks * NPER;

  // Prologue.  Issue order: the active count and the first D active buckets
  // (scalar), the first batch of act pieces and table words (one level deep,
  // into registers), the first D experts' weights, then the LDS stores --
  // which wait for the batch only, not for the weights.  Rows past the live
  // ones are staged too (never selected).  Remainders (large batches) go
  // after the weights.
  const int per_row = a.I / 8;
  const int pieces = (a.row_cap + sh_rows) * per_row;
  const int nreg = a.row_cap * per_row;   // pieces of the sorted rows; then the shared rows
  const int nact_g = a.n_active[0];
  int e_first[D];
#pragma unroll
  for (int d = 0; d < D; ++d) e_first[d] = a.active[min(d, a.max_active - 1)];
  u32x4_t v[kDcSB];
#pragma unroll
  for (int k = 0; k < kDcSB; ++k) {
    const int c = min(tid + k * bd, pieces - 1);
    v[k] = *reinterpret_cast<const u32x4_t*>(c < nreg ? a.act + (long)c * 8
                                                       : a.act_sh + (long)(c - nreg) * 8);
  }
  const int act_v = a.active[min(tid, a.max_active - 1)];
  int seg_v[kDcSegW];
#pragma unroll
  for (int k = 0; k < kDcSegW; ++k) seg_v[k] = a.seg_start[min(tid + k * bd, nseg - 1)];
  const int tok_v = a.sorted_tok[min(tid, a.row_cap - 1)];
  const float w_v = a.sorted_wts[min(tid, a.row_cap - 1)];
  __builtin_amdgcn_sched_barrier(0);
  const int nact = min(nact_g, a.max_active);
  ExpLoad<FMT, NPER> ring[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const int e = d < nact ? min(max(e_first[d], 0), a.trash - 1) : 0;
    const int ws = a.slot_map ? a.slot_map[e] : e;
    issue_expert<FMT, NPER>(ring[d], a, ws, d < nact, panel, u0, lane);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int k = 0; k < kDcSB; ++k) {
    const int c = tid + k * bd;
    if (c < pieces)
      *reinterpret_cast<u32x4_t*>(xs + (c / per_row) * ldx + (c % per_row) * 8) = v[k];
  }
  if (tid < a.max_active) l_act[tid] = act_v;
#pragma unroll
  for (int k = 0; k < kDcSegW; ++k)
    if (tid + k * bd < nseg) l_seg[tid + k * bd] = seg_v[k];
  if (tid < a.row_cap) {
    rtok[tid] = tok_v;
    rw[tid] = w_v;
  }
  for (int c0 = tid + kDcSB * bd; c0 < pieces; c0 += kDcSB * bd) {
    u32x4_t vr[kDcSB];
#pragma unroll
    for (int k = 0; k < kDcSB; ++k) {
      const int c = min(c0 + k * bd, pieces - 1);
      vr[k] = *reinterpret_cast<const u32x4_t*>(c < nreg ? a.act + (long)c * 8
                                                         : a.act_sh + (long)(c - nreg) * 8);
    }
#pragma unroll
    for (int k = 0; k < kDcSB; ++k) {
      const int c = c0 + k * bd;
      if (c < pieces)
        *reinterpret_cast<u32x4_t*>(xs + (c / per_row) * ldx + (c % per_row) * 8) = vr[k];
    }
  }
  for (int j = tid + bd; j < a.max_active; j += bd) l_act[j] = a.active[j];
  for (int e = tid + kDcSegW * bd; e < nseg; e += bd) l_seg[e] = a.seg_start[e];
  for (int r = tid + bd; r < a.row_cap; r += bd) {
    rtok[r] = a.sorted_tok[r];
    rw[r] = a.sorted_wts[r];
  }
  // token -> act row and summed weight per active expert
  for (int i = tid; i < nact * kDcTok; i += bd) {
    rowof[i] = 0;
    wof[i] = 0.f;
  }
  __syncthreads();
  const int e_sh = a.trash - a.n_shared;   // first shared bucket
  for (int j = tid; j < nact; j += bd) {
    const int e = l_act[j];
    eslot[j] = a.slot_map ? a.slot_map[e] : e;
    if (a.act_sh && e >= e_sh) {
      // a shared expert's rows come from act_sh: token t at row_cap + s*T + t,
      // weight 1 (its bucket holds every token once, weight 1, never dropped)
      for (int t = 0; t < a.T; ++t) {
        rowof[j * kDcTok + t] = a.row_cap + (e - e_sh) * a.T + t;
        wof[j * kDcTok + t] = 1.0f;
      }
      continue;
    }
    const int r1 = min(l_seg[e + 1], a.row_cap);
    for (int r = max(l_seg[e], 0); r < r1; ++r) {
      const int t = rtok[r];
      if (t >= 0 && t < kDcTok) {
        rowof[j * kDcTok + t] = r;
        wof[j * kDcTok + t] += rw[r];
      }
    }
  }
  __syncthreads();

  f32x4_t tacc = {0.f, 0.f, 0.f, 0.f};   // tokens 4q + i, column m of the panel
  const int nit = (nact + D - 1) / D;
  for (int it = 0; it < nit; ++it) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int j = it * D + d;
      const bool live = j < nact;
      const int jt = live ? j : 0;
      const uint16_t* xa = xs + rowof[jt * kDcTok + m] * ldx + q * F::kCK;
      f32x4_t pe = consume_expert<FMT, NPER>(ring[d], u0, xa);
      if constexpr (FMT == kNVFP4) {
        const float g = a.gs ? a.gs[eslot[jt]] : 1.0f;
        pe = pe * g;
      }
      const f32x4_t wv = live ? *reinterpret_cast<const f32x4_t*>(wof + jt * kDcTok + 4 * q)
                              : f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 4; ++i)
        tacc[i] = wv[i] != 0.f ? __builtin_fmaf(wv[i], pe[i], tacc[i]) : tacc[i];
      const int jn = j + D;
      const int wsn = __builtin_amdgcn_readfirstlane(eslot[jn < nact ? jn : 0]);
      issue_expert<FMT, NPER>(ring[d], a, wsn, jn < nact, panel, u0, lane);
    }
  }
  // the KS partial sums, through the stage's memory once every wave is done with it
  __syncthreads();
  f32x4_t(*red)[kWave] = reinterpret_cast<f32x4_t(*)[kWave]>(dyn);
  red[w][lane] = tacc;
  __syncthreads();
  for (int t = tid; t < a.ppb * 256; t += bd) {   // tokens x 16 columns per panel
    const int pq = t / 256, tok = (t % 256) / 16, n = t % 16;
    if (tok < a.T) {
      const int l = (tok / 4) * 16 + n, i = tok % 4;
      float v = 0.f;
      for (int k = 0; k < a.ks; ++k) v += red[pq * a.ks + k][l][i];
      const long o = (long)tok * a.H + 16 * (blockIdx.x * a.ppb + pq) + n;
      if (a.out_bf16) reinterpret_cast<uint16_t*>(a.out)[o] = f32_to_bf16(v);
      else reinterpret_cast<float*>(a.out)[o] = v;
    }
  }
}

// Smallest K split (1, 2, 4) that keeps every wave's share within one round.
int pick_ksplit(int nunits, int nu, int max_split) {
  int k = 1;
  while (k < max_split && (nunits + k - 1) / k > nu) k *= 2;
  return k;
}

// The gate/up fast path's shape (every token row staged, one round per wave,
// at most 8 row pieces per thread); ksplit and the row-piece count out.
template <int FMT>
bool gate_up_fast_shape(int T, int H, int& ksplit, int& xc) {
  constexpr int NU = round_units<FMT>();
  const int cap = kLdsBudget / (H * 2);
  ksplit = pick_ksplit(H / 128, NU, 4);
  const int bd = 128 * ksplit;
  const long pieces = (long)T * (H / 8);
  xc = pieces <= bd ? 1 : pieces <= 2L * bd ? 2 : pieces <= 4L * bd ? 4 : 8;
  return T >= 1 && T <= cap && H / 128 <= NU * ksplit && pieces <= 8L * bd;
}

// Compute units of the current device (queried once per device).
int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

bool shape_ok(int fmt, int H, int I) {
  if (H <= 0 || I <= 0 || H % 128 || I % 128 || H > 16384 || I > 16384) return false;
  if (fmt == kFP8 && ((2 * I) % 128 || H % 128)) return false;
  return fmt >= 0 && fmt <= 3;
}

}  // namespace
}  // namespace xtu
