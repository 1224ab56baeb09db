// Grouped expert GEMMs for prefill-sized batches, and the weighted combine.
//
// Work items are (M tile, N block) pairs.  seg_scan_kernel cuts each expert's
// contiguous segment of sorted pairs into M tiles of 128 rows; gate/up N
// blocks hold 128 gate rows and the matching 128 up rows of w13, down N blocks
// 256 rows of w2.  Items are numbered tile-major (N block fastest) and dealt
// to the eight XCDs in contiguous ranges (workgroup i runs on XCD i % 8), so
// the workgroups resident on one XCD at a time share the A rows of a tile
// and the weight panels of an expert through that XCD's L2.
//
// A workgroup of four waves runs the K loop in steps of one super-block
// (128 k for fp4, 64 for fp8, 32 for bf16):
//   A: the tile's rows (gathered through sorted_tok for gate/up, contiguous
//      act rows for down) are loaded as bf16 into registers one step ahead
//      and stored to a double-buffered LDS stage (one barrier per step);
//   B: each wave owns four 16-row weight panels (64 output columns).  In the
//      P16 layout one 16-byte load per lane is exactly the B operand of
//      v_mfma_f32_16x16x32_bf16 for a panel, so the weights go from HBM to
//      registers (one step ahead), are dequantised there and never touch LDS.
// Per step a wave issues 8 row tiles x 4 panels x (chunk k / 8) MFMAs; row
// tiles past the tile's rows are skipped.
//
// Dequantisation: MXFP4 (e2m1 x e8m0) and NVFP4 (e2m1 x e4m3) products are
// exact in bf16; NVFP4's per-expert global scale multiplies the fp32 result.
// FP8 weights taken by this kernel become bf16(e4m3 * block scale), rounded
// to nearest even -- the operand the reference's GPU FP8 kernels form
// (gpu_prefill_fp8.py:148-149, 195-196).  That rounding misses the layer
// tolerance at DeepSeek-V3 size, so the layer's FP8 prefill runs the exact
// activation-pair GEMM of fp8pair.hip instead; this branch stays reachable
// only through xtu_gemm_gate_up / xtu_gemm_down with the FP8 format code.
//
// gate/up: panels 0,1 of a wave are gate rows and panels 2,3 the up rows of
// the same output columns, so each lane holds (g, u) of the same element and
// the epilogue writes the clamped-SwiGLU activation as bf16.  down writes
// fp32 y rows; the combine kernel adds them per token in top-k order.
#include <type_traits>

#include "weight_format.hpp"

namespace xtu {
namespace {

constexpr int kBM = 128;            // rows per M tile
constexpr int kRT = kBM / 16;       // 16-row MFMA tiles per M tile
constexpr int kGemmThreads = 256;
constexpr int kBufFlags = 0x00020000;   // raw buffer resource, dword 3

// SPS super-blocks per K step (BF16 only: its 32-k super-blocks make short
// steps, one barrier each).
template <int FMT, int SPS = 1>
struct GemmShape {
  using F = WFmt<FMT>;
  static_assert(SPS == 1 || FMT == kBF16, "several super-blocks per step: BF16 only");
  static constexpr int kBK = F::kSB * SPS;                    // k per step
  static constexpr int kLD = kBK + 8;                         // LDS row pitch (bf16)
  static constexpr int kAL = kBM * kBK / 8 / kGemmThreads;    // 16-byte A pieces per thread
  static constexpr int kG = F::kCK / 8;                       // MFMA k groups per super-block
  static constexpr int kABuf = kBM * kLD;                     // bf16 per A stage buffer
};

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

// One wave's weights of one step: a 16-byte chunk per panel, the chunk's raw
// fp4 scale bits, and (fp8) the block scales of panels 0,1 and 2,3.
template <int FMT, int PW, int SPS = 1>
struct BStep {
  u32x4_t w[PW * SPS];        // panel p, super-block j of the step: w[p * SPS + j]
  uint32_t sc[PW];
  float bs0, bs1;
};

// bf16 operand of MFMA group g of a chunk (k = q*kCK + 8g .. +7 of the lane's row),
// super-block j of the step.
template <int FMT, int PW, int SPS>
__device__ __forceinline__ bf16x8_t dequant_group(const BStep<FMT, PW, SPS>& b, int p, int g,
                                                  int j) {
  uint32_t o[4];
  if constexpr (FMT == kMXFP4) {
    fp4x8_to_bf16(b.w[p][g], e8m0_to_f32(b.sc[p]), o);
  } else if constexpr (FMT == kNVFP4) {
    const uint32_t raw = b.sc[p] >> (g < 2 ? 0 : 8);
    fp4x8_to_bf16_mul(b.w[p][g], e4m3_to_f32(raw & 0xffu), o);
  } else if constexpr (FMT == kFP8) {
    const float bs = p < PW / 2 ? b.bs0 : b.bs1;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t d = b.w[p][2 * g + h];
      f32x2_t lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(d, 1.0f, false);
      f32x2_t hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(d, 1.0f, true);
      lo = lo * bs;
      hi = hi * bs;
      o[2 * h] = __builtin_bit_cast(uint32_t, __builtin_convertvector(lo, bf16x2_t));
      o[2 * h + 1] = __builtin_bit_cast(uint32_t, __builtin_convertvector(hi, bf16x2_t));
    }
  } else {
    return as_bf16x8(b.w[p * SPS + j]);
  }
  return as_bf16x8(o[0], o[1], o[2], o[3]);
}

// Kernel shape: PW weight panels per wave (a workgroup covers 64*PW output
// columns), weights prefetched PD steps ahead in registers, register budget
// sized for WPS waves per SIMD.
template <int FMT, bool GU, int PW, int PD, int WPS, int SPS = 1>
__global__ __launch_bounds__(kGemmThreads, WPS) void moe_gemm_kernel(GemmArgs a) {
  using F = WFmt<FMT>;
  using S = GemmShape<FMT, SPS>;
  __shared__ __attribute__((aligned(16))) uint16_t As[2 * S::kABuf];

  // ---- work item
  const int nbn = GU ? a.I / (32 * PW) : a.H / (64 * PW);
  const int lo = a.tile_lo[0];
  const int total = (a.tile_hi[0] - lo) * nbn;
  const int per = (total + 7) / 8;
  const int idx = blockIdx.x / 8;
  if (idx >= per) return;
  const int item = (blockIdx.x % 8) * per + idx;
  if (item >= total) return;
  const int tile = lo + item / nbn, nb = item % nbn;
  const int e = a.tile_expert[tile];
  const int ws = a.slot_map ? a.slot_map[e] : e;
  const int row0 = a.tile_row0[tile];
  const int rows = min(kBM, a.seg_start[e + 1] - row0);
  const int K = GU ? a.H : a.I;
  const int nsteps = K / S::kBK;
  const int nsb = K / F::kSB;   // super-blocks per panel row
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid / 64);
  const int lane = tid % 64;

  // ---- A pieces of this thread: source byte offset at k = 0, LDS offset
  constexpr int ppr = S::kBK / 8;   // 16-byte pieces per row per step
  uint32_t aoff[S::kAL];
  int alds[S::kAL];
#pragma unroll
  for (int i = 0; i < S::kAL; ++i) {
    const int c = i * kGemmThreads + tid, r = c / ppr, col = c % ppr;
    const int rr = min(r, rows - 1);
    const uint32_t src = GU ? (uint32_t)a.sorted_tok[row0 + rr] : (uint32_t)rr;
    aoff[i] = src * (uint32_t)K * 2u + (uint32_t)col * 16u;
    alds[i] = r * S::kLD + col * 8;
  }
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(GU ? a.a : a.a + (long)row0 * K), 0, -1, kBufFlags);

  // ---- B: this wave's panels
  // gate/up: panels [0, PW/2) are gate rows, [PW/2, PW) the up rows of the
  // same columns; down: PW consecutive panels
  int pan[PW];
#pragma unroll
  for (int p = 0; p < PW; ++p) {
    if (GU) pan[p] = (p < PW / 2 ? 0 : a.I / 16) + (nb * 4 + w) * (PW / 2) + p % (PW / 2);
    else pan[p] = (nb * 4 + w) * PW + p;
  }
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.w + (long)ws * a.w_estride), 0, (int)a.w_estride, kBufFlags);
  const uint8_t* sexp = a.s ? a.s + (long)ws * a.s_estride : a.w;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)sexp, 0, (int)a.s_estride, kBufFlags);
  const int sgroups = (int)scale_groups(K, F::kUG);
  // fp8 block-scale rows of panels [0, PW/2) and [PW/2, PW) (each run of
  // panels lies inside one 128-row block)
  const float* bsc = reinterpret_cast<const float*>(sexp);
  const int kb128 = K / 128;
  const int rb0 = pan[0] / 8;
  const int rb1 = pan[PW / 2] / 8;

  // piece i holds rows [i, i + 1) * (kGemmThreads / ppr); np_tag: the pieces
  // that hold the rows the MFMAs read (the rest are never staged)
  auto load_a = [&](int s, u32x4_t (&ar)[S::kAL], auto np_tag) {
#pragma unroll
    for (int i = 0; i < decltype(np_tag)::value; ++i)
      ar[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                              ra, aoff[i], s * S::kBK * 2, 0));
  };
  auto store_a = [&](uint16_t* buf, const u32x4_t (&ar)[S::kAL], auto np_tag) {
#pragma unroll
    for (int i = 0; i < decltype(np_tag)::value; ++i)
      *reinterpret_cast<u32x4_t*>(buf + alds[i]) = ar[i];
  };
  auto load_b = [&](int s, BStep<FMT, PW, SPS>& b) {
#pragma unroll
    for (int p = 0; p < PW; ++p)
#pragma unroll
      for (int j = 0; j < SPS; ++j)
        b.w[p * SPS + j] = __builtin_bit_cast(
            u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                         rw, lane * 16, (pan[p] * nsb + s * SPS + j) * 1024, 0));
    if constexpr (F::kSBY > 0) {
      const int g = s / F::kUG, ob = (s % F::kUG) * F::kSBY;
#pragma unroll
      for (int p = 0; p < PW; ++p) {
        const uint32_t v = __builtin_amdgcn_raw_buffer_load_b32(
            rs, lane * 16, (pan[p] * sgroups + g) * 1024 + (ob & ~3), 0);
        b.sc[p] = v >> (8 * (ob & 3));
      }
    } else if constexpr (FMT == kFP8) {
      const int kb = s * S::kBK / 128;
      b.bs0 = bsc[rb0 * kb128 + kb];
      b.bs1 = bsc[rb1 * kb128 + kb];
    }
  };

  // LDS element offset of this lane's A operand (row lane%16, k = q*kCK)
  const int afrag = (lane % 16) * S::kLD + (lane / 16) * F::kCK;

  // K loop and epilogue for NR 16-row tiles (the tile's rows rounded up), so
  // the inner loop carries no per-row-tile branches.
  auto run = [&](auto nr_tag) {
    constexpr int NR = decltype(nr_tag)::value;
    f32x4_t acc[NR][PW];
#pragma unroll
    for (int m = 0; m < NR; ++m)
#pragma unroll
      for (int p = 0; p < PW; ++p) acc[m][p] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](const BStep<FMT, PW, SPS>& b, const uint16_t* buf) {
#pragma unroll
      for (int j = 0; j < SPS; ++j)
#pragma unroll
      for (int g = 0; g < S::kG; ++g) {
        bf16x8_t bv[PW];
#pragma unroll
        for (int p = 0; p < PW; ++p) bv[p] = dequant_group<FMT, PW, SPS>(b, p, g, j);
#pragma unroll
        for (int m = 0; m < NR; ++m) {
          const bf16x8_t av = as_bf16x8(*reinterpret_cast<const u32x4_t*>(
              buf + afrag + m * 16 * S::kLD + j * F::kSB + 8 * g));
#pragma unroll
          for (int p = 0; p < PW; ++p)
            acc[m][p] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv[p], acc[m][p], 0, 0, 0);
        }
      }
    };

    // Step s: issue the A rows of step s+1 and the weights of step s+PD,
    // run the MFMAs of step s, store the A rows to the other LDS buffer,
    // barrier.  Weight buffers rotate through PD+1 register sets (the step
    // loop is unrolled PD+1 times so every set is statically indexed).
    // Scheduling barriers keep the loads ahead of the MFMAs; left alone, the
    // compiler sinks them next to their first use.
    constexpr int U = PD + 1;
    // small-batch BF16 items (several super-blocks per step) stage only the
    // pieces holding the NR*16 rows the MFMAs read (tiny Mixtral 62.0 -> 59.0
    // us); the other shapes measured slower that way (Qwen3-Next NVFP4 T=8192
    // +6%) and stage every piece
    constexpr int kRowsPerPiece = kGemmThreads / ppr;
    constexpr int kNeed = (NR * 16 + kRowsPerPiece - 1) / kRowsPerPiece;
    constexpr std::integral_constant<int, (SPS > 1 && kNeed < S::kAL ? kNeed : S::kAL)> NP{};
    u32x4_t ar[S::kAL];
    BStep<FMT, PW, SPS> bb[U];
    load_a(0, ar, NP);
#pragma unroll
    for (int j = 0; j < PD; ++j) load_b(min(j, nsteps - 1), bb[j]);
    store_a(As, ar, NP);
    __syncthreads();
    for (int s0 = 0; s0 < nsteps; s0 += U) {
#pragma unroll
      for (int j = 0; j < U; ++j) {
        const int s = s0 + j;
        if (j == 0 || s < nsteps) {
          load_a(min(s + 1, nsteps - 1), ar, NP);
          load_b(min(s + PD, nsteps - 1), bb[(j + PD) % U]);
          __builtin_amdgcn_sched_barrier(0);
          compute(bb[j], As + (s & 1) * S::kABuf);
          __builtin_amdgcn_sched_barrier(0);
          store_a(As + ((s + 1) & 1) * S::kABuf, ar, NP);
          __syncthreads();
        }
      }
    }

    // NVFP4 second-level scales: [slot][2] (gate, up) for gate/up, [slot] for down
    float gsv = 1.0f, gsu = 1.0f;
    if constexpr (FMT == kNVFP4) {
      if (a.gs) {
        gsv = GU ? a.gs[2 * ws] : a.gs[ws];
        gsu = GU ? a.gs[2 * ws + 1] : gsv;
      }
    }
    const int r16 = lane % 16, q = lane / 16;
    // The 16x16 result (column lane % 16, rows 4 (lane / 16) + i) of each
    // row tile goes through this wave's own LDS region (the A buffers are
    // free once every wave is past the K loop) and is read back as 16-byte
    // row pieces: wide stores of the wave's contiguous columns (its panels
    // are adjacent) instead of one store per lane and value.
    __syncthreads();
    if constexpr (GU) {
      constexpr int NC = PW / 2 * 16;   // act columns of the wave
      constexpr int kAP = NC + 8;       // staged row pitch (bf16)
      uint16_t* stage = As + w * (16 * kAP);
      uint16_t* act = reinterpret_cast<uint16_t*>(a.out);
      const long col0 = (long)pan[0] * 16;
#pragma unroll
      for (int m = 0; m < NR; ++m) {
        if (m * 16 >= rows) break;
#pragma unroll
        for (int p = 0; p < PW / 2; ++p)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float g = acc[m][p][i] * gsv, u = acc[m][p + PW / 2][i] * gsu;
            stage[(4 * q + i) * kAP + 16 * p + r16] =
                f32_to_bf16(silu_gate(g, u, a.limit, a.alpha, a.beta));
          }
        __builtin_amdgcn_wave_barrier();
        for (int j = lane; j < 16 * (NC / 8); j += 64) {   // 16 rows x NC/8 pieces
          const int rr = j / (NC / 8), c8 = j % (NC / 8);
          if (m * 16 + rr < rows)
            *reinterpret_cast<u32x4_t*>(act + (long)(row0 + m * 16 + rr) * a.I + col0 + 8 * c8) =
                *reinterpret_cast<const u32x4_t*>(stage + rr * kAP + 8 * c8);
        }
        __builtin_amdgcn_wave_barrier();
      }
    } else {
      constexpr int NC = PW * 16;   // y columns of the wave
      constexpr int kYP = NC + 4;   // staged row pitch (floats)
      float* stage = reinterpret_cast<float*>(As) + w * (16 * kYP);
      float* y = reinterpret_cast<float*>(a.out);
      const long col0 = (long)pan[0] * 16;
#pragma unroll
      for (int m = 0; m < NR; ++m) {
        if (m * 16 >= rows) break;
#pragma unroll
        for (int p = 0; p < PW; ++p)
#pragma unroll
          for (int i = 0; i < 4; ++i) stage[(4 * q + i) * kYP + 16 * p + r16] = acc[m][p][i] * gsv;
        __builtin_amdgcn_wave_barrier();
        for (int j = lane; j < 16 * (NC / 4); j += 64) {   // 16 rows x NC/4 pieces
          const int rr = j / (NC / 4), c4 = j % (NC / 4);
          if (m * 16 + rr < rows)
            *reinterpret_cast<f32x4_t*>(y + (long)(row0 + m * 16 + rr) * a.H + col0 + 4 * c4) =
                *reinterpret_cast<const f32x4_t*>(stage + rr * kYP + 4 * c4);
        }
        __builtin_amdgcn_wave_barrier();
      }
    }
  };
  if (rows > 64) run(std::integral_constant<int, kRT>{});
  else if (rows > 32) run(std::integral_constant<int, 4>{});
  else if (rows > 16) run(std::integral_constant<int, 2>{});
  else run(std::integral_constant<int, 1>{});
}

// out[t][h] = sum_k w[t,k] * y[inv[t*K+k]][h] over the pairs that were not
// sent to the trash bucket (sorted position < *trash_start) and have a
// non-zero weight, in k order, + sum_s y[inv[T*K + t*NS + s]][h].
// KC, NSC > 0: K and NS fixed at compile time -- every row position is
// loaded first, then every row at once (two load latencies per token
// instead of one per pair); 0: loops over the run-time K and NS.
template <int KC, int NSC>
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
  if constexpr (KC > 0) {
    K = KC;
    NS = NSC;
    int pos[KC + NSC];
    float w[KC];
#pragma unroll
    for (int j = 0; j < KC; ++j) {
      pos[j] = inv[t * KC + j];
      w[j] = wts[t * KC + j];
    }
#pragma unroll
    for (int s = 0; s < NSC; ++s) pos[KC + s] = inv[T * KC + t * NSC + s];
    // a skipped pair reads row 0 and is not added
    bool ok[KC];
    f32x4_t v[KC + NSC];
    // y rows are read exactly once: streaming (nontemporal) loads
#pragma unroll
    for (int j = 0; j < KC; ++j) {
      ok[j] = pos[j] < trash && w[j] != 0.f;
      v[j] = __builtin_nontemporal_load(
          reinterpret_cast<const f32x4_t*>(y + (long)(ok[j] ? pos[j] : 0) * H + h));
    }
#pragma unroll
    for (int s = 0; s < NSC; ++s)
      v[KC + s] = __builtin_nontemporal_load(
          reinterpret_cast<const f32x4_t*>(y + (long)pos[KC + s] * H + h));
#pragma unroll
    for (int j = 0; j < KC; ++j) acc = ok[j] ? acc + w[j] * v[j] : acc;
#pragma unroll
    for (int s = 0; s < NSC; ++s) acc += v[KC + s];
  } else {
    for (int k = 0; k < K; ++k) {
      const int pos = inv[t * K + k];
      const float w = wts[t * K + k];
      if (pos >= trash || w == 0.f) continue;
      const f32x4_t v =
          __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(y + (long)pos * H + h));
      acc += w * v;
    }
    for (int s = 0; s < NS; ++s) {
      const f32x4_t v = __builtin_nontemporal_load(
          reinterpret_cast<const f32x4_t*>(y + (long)inv[T * K + t * NS + s] * H + h));
      acc += v;
    }
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

template <int KC, int NSC>
bool launch_combine_kn(dim3 grid, hipStream_t stream, const float* y, const int32_t* inv,
                       const float* w, const int32_t* trash, int T, int H, void* out,
                       int out_bf16) {
  combine_kernel<KC, NSC><<<grid, 256, 0, stream>>>(y, inv, w, trash, T, KC, NSC, H, out,
                                                    out_bf16);
  return true;
}

// combine_kernel over y rows in flat pair order (pair t*K + k at row t*K + k,
// shared pair (t, s) at row T*K + t*NS + s): the row addresses do not depend
// on inv, so every load of a token is issued at once (one memory latency).
// The skip test, the order and the arithmetic are combine_kernel's; the rows
// of skipped pairs are never written and never added (a select, not a
// multiply by zero).
template <int KC, int NSC>
__global__ __launch_bounds__(256) void combine_pairs_kernel(const float* __restrict__ y,
                                                            const int32_t* __restrict__ inv,
                                                            const float* __restrict__ wts,
                                                            const int32_t* __restrict__ trash_start,
                                                            int T, int H, void* out,
                                                            int out_bf16) {
  const int t = blockIdx.y;
  const int h = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (h >= H) return;
  const int trash = trash_start[0];
  int pos[KC];
  float w[KC];
  f32x4_t v[KC + NSC];
#pragma unroll
  for (int j = 0; j < KC; ++j) {
    pos[j] = inv[t * KC + j];
    w[j] = wts[t * KC + j];
    v[j] = __builtin_nontemporal_load(
        reinterpret_cast<const f32x4_t*>(y + (long)(t * KC + j) * H + h));
  }
#pragma unroll
  for (int s = 0; s < NSC; ++s)
    v[KC + s] = __builtin_nontemporal_load(
        reinterpret_cast<const f32x4_t*>(y + (long)(T * KC + t * NSC + s) * H + h));
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < KC; ++j) {
    const bool ok = pos[j] < trash && w[j] != 0.f;
    acc = ok ? acc + w[j] * v[j] : acc;
  }
#pragma unroll
  for (int s = 0; s < NSC; ++s) acc += v[KC + s];
  if (out_bf16) {
    uint16_t* o = reinterpret_cast<uint16_t*>(out) + (long)t * H + h;
    const uint32_t lo = f32_to_bf16(acc[0]) | ((uint32_t)f32_to_bf16(acc[1]) << 16);
    const uint32_t hi = f32_to_bf16(acc[2]) | ((uint32_t)f32_to_bf16(acc[3]) << 16);
    *reinterpret_cast<uint2*>(o) = make_uint2(lo, hi);
  } else {
    *reinterpret_cast<f32x4_t*>(reinterpret_cast<float*>(out) + (long)t * H + h) = acc;
  }
}

template <int KC>
bool launch_combine_pairs_k(dim3 grid, hipStream_t stream, const float* y, const int32_t* inv,
                            const float* w, const int32_t* trash, int T, int NS, int H, void* out,
                            int out_bf16) {
  switch (NS) {
    case 0: combine_pairs_kernel<KC, 0><<<grid, 256, 0, stream>>>(y, inv, w, trash, T, H, out, out_bf16); return true;
    case 1: combine_pairs_kernel<KC, 1><<<grid, 256, 0, stream>>>(y, inv, w, trash, T, H, out, out_bf16); return true;
    case 2: combine_pairs_kernel<KC, 2><<<grid, 256, 0, stream>>>(y, inv, w, trash, T, H, out, out_bf16); return true;
  }
  return false;
}

template <int KC>
bool launch_combine_k(dim3 grid, hipStream_t stream, const float* y, const int32_t* inv,
                      const float* w, const int32_t* trash, int T, int NS, int H, void* out,
                      int out_bf16) {
  switch (NS) {
    case 0: return launch_combine_kn<KC, 0>(grid, stream, y, inv, w, trash, T, H, out, out_bf16);
    case 1: return launch_combine_kn<KC, 1>(grid, stream, y, inv, w, trash, T, H, out, out_bf16);
    case 2: return launch_combine_kn<KC, 2>(grid, stream, y, inv, w, trash, T, H, out, out_bf16);
  }
  return false;
}

// The compile-time shapes: the routers' top-k of the configurations here
// (1, 2, 4, 6, 8, 10) with up to two shared experts.
bool launch_combine_fixed(dim3 grid, hipStream_t stream, const float* y, const int32_t* inv,
                          const float* w, const int32_t* trash, int T, int K, int NS, int H,
                          void* out, int out_bf16) {
  switch (K) {
    case 1: return launch_combine_k<1>(grid, stream, y, inv, w, trash, T, NS, H, out, out_bf16);
    case 2: return launch_combine_k<2>(grid, stream, y, inv, w, trash, T, NS, H, out, out_bf16);
    case 4: return launch_combine_k<4>(grid, stream, y, inv, w, trash, T, NS, H, out, out_bf16);
    case 6: return launch_combine_k<6>(grid, stream, y, inv, w, trash, T, NS, H, out, out_bf16);
    case 8: return launch_combine_k<8>(grid, stream, y, inv, w, trash, T, NS, H, out, out_bf16);
    case 10: return launch_combine_k<10>(grid, stream, y, inv, w, trash, T, NS, H, out, out_bf16);
  }
  return false;
}

// Kernel shape.  Measured on the DeepSeek-V3 FP8 layer (T = 8192): four
// panels per wave, weights one step ahead and two waves per SIMD beat eight
// panels per wave with two or three steps of prefetch at one wave per SIMD
// (the second wave hides the first one's load and LDS waits).  XTU_GEMM_PW
// = 8 selects the larger tile where N divides 512.
#ifndef XTU_GEMM_PW
#define XTU_GEMM_PW 4
#endif
#ifndef XTU_GEMM_PD
#define XTU_GEMM_PD 1
#endif
#ifndef XTU_GEMM_WPS
#define XTU_GEMM_WPS 2
#endif
constexpr long kGemmSmallItems = 512;   // below this, half-width work items

template <int FMT, int PW, int PD, int WPS, int SPS = 1>
hipError_t launch_shape(bool gu, const GemmArgs& a, int max_tiles, hipStream_t stream) {
  const long items = (long)max_tiles * (gu ? a.I / (32 * PW) : a.H / (64 * PW));
  const long grid = (items + 7) / 8 * 8;
  if (grid >= (1L << 31)) return hipErrorInvalidValue;
  const dim3 g((unsigned)grid);
  if (gu) {
    if constexpr (PW % 2 == 0)   // gate/up: gate and up halves of the panels
      moe_gemm_kernel<FMT, true, PW, PD, WPS, SPS><<<g, kGemmThreads, 0, stream>>>(a);
    else
      return hipErrorInvalidValue;
  } else {
    moe_gemm_kernel<FMT, false, PW, PD, WPS, SPS><<<g, kGemmThreads, 0, stream>>>(a);
  }
  return hipPeekAtLastError();
}

template <int FMT>
hipError_t launch_gemm(bool gu, GemmArgs a, int max_tiles, hipStream_t stream) {
  using F = WFmt<FMT>;
  const long N = gu ? 2L * a.I : a.H, K = gu ? a.H : a.I;
  if (!a.w_estride) a.w_estride = F::w_bytes(N, K);
  if (!a.s_estride) a.s_estride = F::s_bytes(N, K);
  if (a.w_estride >= (1L << 31) || a.s_estride >= (1L << 31)) return hipErrorInvalidValue;
  constexpr int PW = XTU_GEMM_PW;
  if constexpr (PW > 4) {
    if ((gu ? a.I % (32 * PW) : a.H % (64 * PW)) == 0)
      return launch_shape<FMT, PW, XTU_GEMM_PD, XTU_GEMM_WPS>(gu, a, max_tiles, stream);
  }
  // NVFP4's exact scale multiply keeps fp32 products live: four panels per
  // wave need more than half of the register file (one wave per SIMD), two
  // fit at two waves per SIMD -- measured 32% faster (Qwen3-Next T = 8192
  // gate/up 999 -> 678 us).  The down pass (short K: 4 steps at I = 512)
  // takes its weights three steps ahead (580 -> 490 us; no gain for gate/up).
  // H % 128 == 0 and I % 64 == 0 always hold here.
  if constexpr (FMT == kNVFP4) {
    if (gu) return launch_shape<FMT, 2, 1, 2>(gu, a, max_tiles, stream);
    return launch_shape<FMT, 2, 3, 2>(gu, a, max_tiles, stream);
  } else {
    // few work items (small batches over few experts, e.g. 128 tokens on 8
    // experts: 32 down items for 256 CUs): half-width items, twice as many
    // weight streams in flight
    const long items4 = (long)max_tiles * (gu ? a.I / 128 : a.H / 256);
#ifndef XTU_SMALL_SPS
#define XTU_SMALL_SPS 4
#endif
    if (items4 < kGemmSmallItems && (gu ? a.I % 64 : a.H % 128) == 0) {
      if constexpr (FMT == kBF16) {
        // the down pass with one panel per wave: four times the items (tiny
        // Mixtral: 128 instead of 64 workgroups; 52.2 -> 48.0 us per layer)
        if (!gu) return launch_shape<FMT, 1, 1, 2, XTU_SMALL_SPS>(gu, a, max_tiles, stream);
      }
      return launch_shape<FMT, 2, 1, 2, FMT == kBF16 ? XTU_SMALL_SPS : 1>(gu, a, max_tiles,
                                                                          stream);
    }
    return launch_shape<FMT, 4, 1, 2>(gu, a, max_tiles, stream);
  }
}

}  // namespace
}  // namespace xtu

using namespace xtu;

extern "C" {

int xtu_gemm_tile_m(int fmt) { return fmt >= 0 && fmt <= 3 ? kBM : 0; }

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
    case kMXFP4: return launch_gemm<kMXFP4>(true, a, max_tiles, stream);
    case kNVFP4: return launch_gemm<kNVFP4>(true, a, max_tiles, stream);
    case kFP8: return launch_gemm<kFP8>(true, a, max_tiles, stream);
    case kBF16: return launch_gemm<kBF16>(true, a, max_tiles, stream);
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
    case kMXFP4: return launch_gemm<kMXFP4>(false, a, max_tiles, stream);
    case kNVFP4: return launch_gemm<kNVFP4>(false, a, max_tiles, stream);
    case kFP8: return launch_gemm<kFP8>(false, a, max_tiles, stream);
    case kBF16: return launch_gemm<kBF16>(false, a, max_tiles, stream);
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
  if (!launch_combine_fixed(grid, stream, y, inv, topk_weights, trash_start, T, K, n_shared, H,
                            out, out_bf16))
    combine_kernel<0, 0><<<grid, 256, 0, stream>>>(y, inv, topk_weights, trash_start, T, K,
                                                   n_shared, H, out, out_bf16);
  return hipPeekAtLastError();
}

hipError_t xtu_combine_by_pair(const float* y, const int32_t* inv, const float* topk_weights,
                               const int32_t* trash_start, int T, int K, int n_shared, int H,
                               void* out, int out_bf16, hipStream_t stream) {
  XTU_CHECK_ARG(T >= 0 && T <= 65535 && H > 0 && H % 4 == 0 && n_shared >= 0 && n_shared <= 2 &&
                (K == 1 || K == 2 || K == 4 || K == 6 || K == 8 || K == 10));
  XTU_CHECK_ARG(T == 0 || (y && inv && out && trash_start && topk_weights));
  if (T == 0) return hipSuccess;
  (void)hipGetLastError();
  const dim3 grid((H / 4 + 255) / 256, T);
  switch (K) {
    case 1: launch_combine_pairs_k<1>(grid, stream, y, inv, topk_weights, trash_start, T, n_shared, H, out, out_bf16); break;
    case 2: launch_combine_pairs_k<2>(grid, stream, y, inv, topk_weights, trash_start, T, n_shared, H, out, out_bf16); break;
    case 4: launch_combine_pairs_k<4>(grid, stream, y, inv, topk_weights, trash_start, T, n_shared, H, out, out_bf16); break;
    case 6: launch_combine_pairs_k<6>(grid, stream, y, inv, topk_weights, trash_start, T, n_shared, H, out, out_bf16); break;
    case 8: launch_combine_pairs_k<8>(grid, stream, y, inv, topk_weights, trash_start, T, n_shared, H, out, out_bf16); break;
    default: launch_combine_pairs_k<10>(grid, stream, y, inv, topk_weights, trash_start, T, n_shared, H, out, out_bf16); break;
  }
  return hipPeekAtLastError();
}

}  // extern "C"
