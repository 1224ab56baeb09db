// Exact FP8-weight grouped GEMMs on the scaled fp8 MFMA
// (v_mfma_scale_f32_16x16x128_f8f6f4, e4m3 x e4m3).
//
// Activations: each bf16 row is cut into blocks of 32 k and every block is
// written as two e4m3 vectors with e8m0 scales,
//   x = hi * 2^(sa-127) + lo * 2^(sa-4-127),
// sa putting the block maximum at <= 448 (the largest e4m3 normal), hi the
// round-to-nearest-even e4m3 of x / 2^(sa-127) and lo the e4m3 of 16x the
// remainder (|remainder| <= half an ulp of hi <= 16, so 16x stays <= 256).
// A bf16 value has 8 significant bits, hi keeps 4 and the remainder has at
// most 4, so the pair is exact for every value at least 2^-6 after scaling
// (at least 2^-13.8 of its block's maximum); below that hi is subnormal and
// the last bit may be rounded (an error under 2^-19 of the block maximum).
//
// Weights (FP8): the e4m3 codes go from the P16 layout straight into the MFMA B
// operand.  The MFMA's 128-k reduction is exactly one 128 x 128 block of the
// fp32 block scales, so each (16-row tile, panel) pair is
//   part = mfma(hi, w, 0; scale sa) + mfma(lo, w, part; scale sa - 4)
//   acc  = fma(block scale, part, acc)
// which is the dequantised-fp32 product up to fp32 summation order -- no
// operand is rounded.  Two fp8 MFMAs take the time of the four bf16 ones of
// the same 128 k, and there is no weight dequantisation.
//
// Weights (MXFP4): the e2m1 codes go from the P16 layout straight into the
// MFMA B operand as fp4 (an fp4 B lane 16q + r holds k = 32q..32q+31 of
// column r, one P16 chunk, low nibble = even k; checked on the device) and
// the chunk's e8m0 byte is the lane's B scale, so
//   acc = mfma(hi, w, acc; sa, sw) ; acc = mfma(lo, w, acc; sa - 4, sw)
// is the dequantised-fp32 product with no fold at all.
//
// MFMA operand layout (checked on the device): lane 16q + r holds row r;
// operand bytes 0..15 are k = 16q..16q+15 and bytes 16..31 are
// k = 64 + 16q..64 + 16q + 15 of the 128-k block -- exactly the lane's P16
// chunks of the block's two 64-k super-blocks -- and the e8m0 scale of the
// 32-k block b comes from lanes 16b..16b+15.
//
// Work items are dealt to the XCDs in contiguous ranges as in gemm.hip, but
// ordered (expert, N block, M tile) with the M tile fastest: the weights are
// the bytes that matter (an expert's weight slice is 7x its rows), and the
// workgroups streaming one slice run side by side.  The double-buffered LDS
// stage of the gathered rows and the epilogues follow gemm.hip; M tiles hold 64 rows (4 row tiles) so the two register sets of
// weights fit beside the accumulators at two waves per SIMD (96 rows spill).
#include <type_traits>

#include "pairgemm.hpp"

namespace xtu {
namespace {

typedef int i32x8_t __attribute__((ext_vector_type(8)));

constexpr int kBM8 = 64;              // rows per M tile
constexpr int kRT8 = kBM8 / 16;       // 16-row tiles per M tile
constexpr int kPW8 = 4;               // 16-row weight panels per wave
constexpr int kThreads8 = 256;
constexpr int kLD8 = 272;             // LDS bytes per row: hi 128, lo 128, scales 4 + 4, pad 8
constexpr int kBuf8 = kBM8 * kLD8;    // LDS bytes per stage buffer
constexpr int kAP8 = kBM8 * 16 / kThreads8;   // 16-byte row pieces per thread per step
constexpr int kFlags8 = 0x00020000;   // raw buffer resource, dword 3

// ---------------------------------------------------------------------------
// bf16 rows -> (hi, lo, scale) pairs
// ---------------------------------------------------------------------------

// One thread per (row, 32-k block).
__global__ __launch_bounds__(256) void fp8pair_quant_kernel(const uint16_t* __restrict__ x, int M,
                                                            int K, uint8_t* __restrict__ hi,
                                                            uint8_t* __restrict__ lo,
                                                            uint8_t* __restrict__ shi,
                                                            uint8_t* __restrict__ slo) {
  const long nb = (long)M * (K / 32);
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nb) return;
  const long row = i / (K / 32), blk = i % (K / 32);
  uint32_t hw[8], lw[8];
  const int sa = pair_split32(x + row * K + blk * 32, hw, lw);
  uint8_t* dh = hi + row * K + blk * 32;
  uint8_t* dl = lo + row * K + blk * 32;
  *reinterpret_cast<u32x4_t*>(dh) = u32x4_t{hw[0], hw[1], hw[2], hw[3]};
  *reinterpret_cast<u32x4_t*>(dh + 16) = u32x4_t{hw[4], hw[5], hw[6], hw[7]};
  *reinterpret_cast<u32x4_t*>(dl) = u32x4_t{lw[0], lw[1], lw[2], lw[3]};
  *reinterpret_cast<u32x4_t*>(dl + 16) = u32x4_t{lw[4], lw[5], lw[6], lw[7]};
  const int sl = sa >= 4 ? sa - 4 : 0;
  shi[i] = (uint8_t)sa;
  slo[i] = (uint8_t)sl;
}

// ---------------------------------------------------------------------------
// grouped GEMM
// ---------------------------------------------------------------------------
struct Gemm8Args {
  const uint8_t* hi;          // gate/up: x pairs [T][K]; down: act pairs [A][K]
  const uint8_t* lo;
  const uint8_t* shi;         // [rows][K/32]
  const uint8_t* slo;
  const int32_t* sorted_tok;  // gate/up row gather
  const uint8_t* w;           // e4m3 P16 panels, expert-major
  const float* s;             // fp32 [N/128][K/128] block scales, expert-major
  const int32_t* seg_start;
  const int32_t* tile_expert;
  const int32_t* tile_row0;
  const int32_t* expert_tile_start;   // first tile of each bucket
  const int32_t* tile_lo;
  const int32_t* tile_hi;
  const int32_t* slot_map;
  void* out;                  // gate/up: act bf16 [A][I]; down: y fp32 [A][H]
  int H, I;
  long w_estride, s_estride;
  float limit, alpha, beta;
};

struct B8Step {
  i32x8_t w[kPW8];
  float bs0, bs1;     // FP8: block scales of the two panel pairs
  int sc[kPW8];       // MXFP4: the lane's e8m0 byte per panel
};

template <bool GU, int WF>
__global__ __launch_bounds__(kThreads8, 2) void gemm8_kernel(Gemm8Args a) {
  static_assert(WF == kFP8 || WF == kMXFP4, "FP8 or MXFP4 weights");
  constexpr bool MX = WF == kMXFP4;
  __shared__ __attribute__((aligned(16))) uint8_t As[2 * kBuf8];

  // ---- work item: (M tile, N block), XCD-contiguous, N block fastest
  const int nbn = GU ? a.I / 128 : a.H / 256;
  const int tlo = a.tile_lo[0];
  const int total = (a.tile_hi[0] - tlo) * nbn;
  const int per = (total + 7) / 8;
  const int idx = blockIdx.x / 8;
  if (idx >= per) return;
  const int item = (blockIdx.x % 8) * per + idx;
  if (item >= total) return;
  // an expert's items are contiguous (its tiles x nbn); inside them the M
  // tile runs fastest, so the workgroups that stream one weight slice start
  // together and share it through L2
  const int j0 = tlo + item / nbn;
  const int e = a.tile_expert[j0];
  const int t0 = a.expert_tile_start[e];
  const int ntl = a.expert_tile_start[e + 1] - t0;
  const int local = tlo * nbn + item - t0 * nbn;
  const int nb = local / ntl, tile = t0 + local % ntl;
  const int ws = a.slot_map ? a.slot_map[e] : e;
  const int row0 = a.tile_row0[tile];
  const int rows = min(kBM8, a.seg_start[e + 1] - row0);
  const int K = GU ? a.H : a.I;
  const int nsteps = K / 128;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid / 64);
  const int lane = tid % 64;

  // ---- row pieces of this thread.  Waves 0-1 stage the hi plane, waves 2-3
  // the lo plane (so each wave's buffer descriptor is uniform: no per-lane
  // descriptor loop); piece i of thread t covers plane bytes 16 * (f % 8) of
  // row f / 8, f = i * 128 + t % 128.  Scale words: wave 0 the hi scales,
  // wave 1 the lo scales, row = lane.
  const int aplane = __builtin_amdgcn_readfirstlane(tid / 128);
  uint32_t aoff[kAP8];
  int alds[kAP8];
#pragma unroll
  for (int i = 0; i < kAP8; ++i) {
    const int f = i * 128 + tid % 128;
    const int r = f / 8;
    const int rr = min(r, rows - 1);
    const uint32_t src = GU ? (uint32_t)a.sorted_tok[row0 + rr] : (uint32_t)(row0 + rr);
    aoff[i] = src * (uint32_t)K + (uint32_t)(f % 8) * 16u;
    alds[i] = r * kLD8 + aplane * 128 + (f % 8) * 16;
  }
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(aplane ? a.lo : a.hi), 0, -1, kFlags8);
  const bool sthr = tid < 2 * kBM8;
  const int splane = __builtin_amdgcn_readfirstlane(tid / 64);   // wave 0 / 1
  const int srow = sthr ? tid % 64 : 0;
  const uint32_t ssrc = GU ? (uint32_t)a.sorted_tok[row0 + min(srow, rows - 1)]
                           : (uint32_t)(row0 + min(srow, rows - 1));
  const uint32_t soff = ssrc * (uint32_t)(K / 32);
  // waves 2-3 store their (unused) word into the row padding: the store stays
  // unconditional, so the step has no branch the MFMAs could be sunk past
  const int slds = sthr ? srow * kLD8 + 256 + 4 * (splane & 1) : (tid % 64) * kLD8 + 264;
  const __amdgpu_buffer_rsrc_t rsc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((splane & 1) ? a.slo : a.shi), 0, -1, kFlags8);

  // ---- weights: this wave's panels, block-scale rows
  int pan[kPW8];
#pragma unroll
  for (int p = 0; p < kPW8; ++p) {
    if (GU) pan[p] = (p < 2 ? 0 : a.I / 16) + (nb * 4 + w) * 2 + (p & 1);
    else pan[p] = (nb * 4 + w) * kPW8 + p;
  }
  const long nw = GU ? 2L * a.I : (long)a.H;   // weight rows
  const long w_es = a.w_estride ? a.w_estride : WFmt<WF>::w_bytes(nw, K);
  const long s_es = a.s_estride ? a.s_estride : WFmt<WF>::s_bytes(nw, K);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.w + (long)ws * w_es), 0, (int)w_es, kFlags8);
  const float* bsc = reinterpret_cast<const float*>(reinterpret_cast<const uint8_t*>(a.s) +
                                                    (long)ws * s_es);
  const int kb128 = K / 128;
  const int rb0 = pan[0] / 8, rb1 = pan[kPW8 / 2] / 8;
  const int nsb = K / WFmt<WF>::kSB;
  // MXFP4 scale groups of a panel: [groups][64 lanes][16 B], 16 super-blocks each
  const int sgb = scale_groups(K, WFmt<kMXFP4>::kUG) * 1024;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(reinterpret_cast<const uint8_t*>(a.s) + (long)ws * s_es), 0, (int)s_es, kFlags8);

  auto load_a = [&](int s, u32x4_t (&ar)[kAP8], uint32_t& sw) {
#pragma unroll
    for (int i = 0; i < kAP8; ++i)
      ar[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                              ra, aoff[i], s * 128, 0));
    sw = __builtin_amdgcn_raw_buffer_load_b32(rsc, soff, s * 4, 0);
  };
  auto store_a = [&](uint8_t* buf, const u32x4_t (&ar)[kAP8], uint32_t sw) {
#pragma unroll
    for (int i = 0; i < kAP8; ++i) *reinterpret_cast<u32x4_t*>(buf + alds[i]) = ar[i];
    *reinterpret_cast<uint32_t*>(buf + slds) = sw;
  };
  auto load_b = [&](int s, B8Step& b) {
    if constexpr (MX) {   // one fp4 chunk and its e8m0 byte per panel
#pragma unroll
      for (int p = 0; p < kPW8; ++p) {
        const u32x4_t v = __builtin_bit_cast(
            u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rw, lane * 16,
                                                           (pan[p] * nsb + s) * 1024, 0));
#pragma unroll
        for (int q = 0; q < 4; ++q) b.w[p][q] = (int)v[q];
#pragma unroll
        for (int q = 4; q < 8; ++q) b.w[p][q] = 0;
        b.sc[p] = (int)__builtin_amdgcn_raw_buffer_load_b8(
            rs, lane * 16 + (s % 16), pan[p] * sgb + (s / 16) * 1024, 0);
      }
    } else {
#pragma unroll
      for (int p = 0; p < kPW8; ++p) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const u32x4_t v = __builtin_bit_cast(
              u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                           rw, lane * 16, (pan[p] * nsb + 2 * s + h) * 1024, 0));
#pragma unroll
          for (int q = 0; q < 4; ++q) b.w[p][4 * h + q] = (int)v[q];
        }
      }
      b.bs0 = bsc[rb0 * kb128 + s];
      b.bs1 = bsc[rb1 * kb128 + s];
    }
  };

  // LDS byte offset of this lane's operand (row lane%16, k = 16q) and scale byte
  const int q = lane / 16, r16 = lane % 16;
  const int afrag = r16 * kLD8 + 16 * q;
  const int sfrag = r16 * kLD8 + 256 + q;

  auto run = [&](auto nr_tag) {
    constexpr int NR = decltype(nr_tag)::value;
    f32x4_t acc[NR][kPW8];
#pragma unroll
    for (int m = 0; m < NR; ++m)
#pragma unroll
      for (int p = 0; p < kPW8; ++p) acc[m][p] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](const B8Step& b, const uint8_t* buf) {
#pragma unroll
      for (int m = 0; m < NR; ++m) {
        const uint8_t* rowp = buf + afrag + m * 16 * kLD8;
        const u32x4_t h0 = *reinterpret_cast<const u32x4_t*>(rowp);
        const u32x4_t h1 = *reinterpret_cast<const u32x4_t*>(rowp + 64);
        const u32x4_t l0 = *reinterpret_cast<const u32x4_t*>(rowp + 128);
        const u32x4_t l1 = *reinterpret_cast<const u32x4_t*>(rowp + 192);
        const int sh = buf[sfrag + m * 16 * kLD8];
        const int sl = buf[sfrag + m * 16 * kLD8 + 4];
        const i32x8_t ah = {(int)h0[0], (int)h0[1], (int)h0[2], (int)h0[3],
                            (int)h1[0], (int)h1[1], (int)h1[2], (int)h1[3]};
        const i32x8_t al = {(int)l0[0], (int)l0[1], (int)l0[2], (int)l0[3],
                            (int)l1[0], (int)l1[1], (int)l1[2], (int)l1[3]};
        if constexpr (MX) {   // the weight scale is the MFMA's B scale: no fold
#pragma unroll
          for (int p0 = 0; p0 < kPW8; p0 += 2) {
#pragma unroll
            for (int j = 0; j < 2; ++j)
              acc[m][p0 + j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                  ah, b.w[p0 + j], acc[m][p0 + j], 0, 4, 0, sh, 0, b.sc[p0 + j]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
              acc[m][p0 + j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                  al, b.w[p0 + j], acc[m][p0 + j], 0, 4, 0, sl, 0, b.sc[p0 + j]);
          }
          continue;
        }
        // two panels at a time: the hi products of both, then the lo ones
        // (independent MFMA chains back to back), then the scaled fold
#pragma unroll
        for (int p0 = 0; p0 < kPW8; p0 += 2) {
          f32x4_t part[2];
#pragma unroll
          for (int j = 0; j < 2; ++j)
            part[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                ah, b.w[p0 + j], f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, sh, 0, 127);
#pragma unroll
          for (int j = 0; j < 2; ++j)
            part[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(al, b.w[p0 + j], part[j],
                                                                       0, 0, 0, sl, 0, 127);
          const float bs = p0 < kPW8 / 2 ? b.bs0 : b.bs1;
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              acc[m][p0 + j][i] = __builtin_fmaf(bs, part[j][i], acc[m][p0 + j][i]);
        }
      }
    };

    u32x4_t ar[kAP8];
    uint32_t sw = 0u;
    B8Step b0, b1;
    load_a(0, ar, sw);
    load_b(0, b0);
    store_a(As, ar, sw);
    __syncthreads();
    // two steps per trip with no branch inside, so the MFMAs stay between
    // the next step's loads and the LDS stores that wait for them; an odd
    // last step runs after the loop (the step past the end is a re-read)
    int s = 0;
    for (; s + 1 < nsteps; s += 2) {
      load_a(s + 1, ar, sw);
      load_b(s + 1, b1);
      __builtin_amdgcn_sched_barrier(0);
      compute(b0, As);
      __builtin_amdgcn_sched_barrier(0);
      store_a(As + kBuf8, ar, sw);
      __syncthreads();
      const int s2 = min(s + 2, nsteps - 1);
      load_a(s2, ar, sw);
      load_b(s2, b0);
      __builtin_amdgcn_sched_barrier(0);
      compute(b1, As + kBuf8);
      __builtin_amdgcn_sched_barrier(0);
      store_a(As, ar, sw);
      __syncthreads();
    }
    if (s < nsteps) compute(b0, As);

    if constexpr (GU) {
      uint16_t* act = reinterpret_cast<uint16_t*>(a.out);
#pragma unroll
      for (int m = 0; m < NR; ++m)
#pragma unroll
        for (int p = 0; p < kPW8 / 2; ++p) {
          const long col = (long)pan[p] * 16 + r16;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = m * 16 + 4 * q + i;
            if (r < rows)
              act[(long)(row0 + r) * a.I + col] = f32_to_bf16(
                  silu_gate(acc[m][p][i], acc[m][p + kPW8 / 2][i], a.limit, a.alpha, a.beta));
          }
        }
    } else {
      float* y = reinterpret_cast<float*>(a.out);
#pragma unroll
      for (int m = 0; m < NR; ++m)
#pragma unroll
        for (int p = 0; p < kPW8; ++p) {
          const long col = (long)pan[p] * 16 + r16;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = m * 16 + 4 * q + i;
            if (r < rows) y[(long)(row0 + r) * a.H + col] = acc[m][p][i];
          }
        }
    }
  };
  if (rows > 64) run(std::integral_constant<int, kRT8>{});
  else if (rows > 32) run(std::integral_constant<int, 4>{});
  else if (rows > 16) run(std::integral_constant<int, 2>{});
  else run(std::integral_constant<int, 1>{});
}

hipError_t launch_gemm8(int wf, bool gu, const Gemm8Args& a, int max_tiles,
                        hipStream_t stream) {
  const long items = (long)max_tiles * (gu ? a.I / 128 : a.H / 256);
  const long grid = (items + 7) / 8 * 8;
  if (grid >= (1L << 31)) return hipErrorInvalidValue;
  if (grid == 0) return hipSuccess;
  const dim3 g((unsigned)grid);
  if (wf == kMXFP4) {
    if (gu) gemm8_kernel<true, kMXFP4><<<g, kThreads8, 0, stream>>>(a);
    else gemm8_kernel<false, kMXFP4><<<g, kThreads8, 0, stream>>>(a);
  } else {
    if (gu) gemm8_kernel<true, kFP8><<<g, kThreads8, 0, stream>>>(a);
    else gemm8_kernel<false, kFP8><<<g, kThreads8, 0, stream>>>(a);
  }
  return hipPeekAtLastError();
}

}  // namespace
}  // namespace xtu

using namespace xtu;

extern "C" {

int xtu_gemm8_tile_m(void) { return kBM8; }

hipError_t xtu_fp8pair_quant(const void* x, int M, int K, uint8_t* hi, uint8_t* lo, uint8_t* shi,
                             uint8_t* slo, hipStream_t stream) {
  XTU_CHECK_ARG(M >= 0 && K > 0 && K % 128 == 0 && (long)M * K < (1L << 32));
  XTU_CHECK_ARG(M == 0 || (x && hi && lo && shi && slo));
  if (M == 0) return hipSuccess;
  (void)hipGetLastError();
  const long nb = (long)M * (K / 32);
  fp8pair_quant_kernel<<<(unsigned)((nb + 255) / 256), 256, 0, stream>>>(
      (const uint16_t*)x, M, K, hi, lo, shi, slo);
  return hipPeekAtLastError();
}

hipError_t xtu_gemm8_gate_up(const uint8_t* hi, const uint8_t* lo, const uint8_t* shi,
                             const uint8_t* slo, const int32_t* sorted_tok, int H, int I,
                             const void* w13, const float* s13, long w_estride, long s_estride,
                             const int32_t* slot_map, const int32_t* seg_start,
                             const int32_t* tile_expert, const int32_t* tile_row0,
                             const int32_t* expert_tile_start, const int32_t* tile_lo,
                             const int32_t* tile_hi, int max_tiles, void* act, float limit,
                             float alpha, float beta, hipStream_t stream) {
  XTU_CHECK_ARG(H > 0 && I > 0 && H % 256 == 0 && I % 128 == 0 && H <= 65536);
  XTU_CHECK_ARG(max_tiles >= 0 && max_tiles < (1 << 30) && w_estride >= 0 && s_estride >= 0);
  XTU_CHECK_ARG(w_estride < (1L << 31) && 2L * I * H < (1L << 31));
  XTU_CHECK_ARG(hi && lo && shi && slo && sorted_tok && w13 && s13 && seg_start && tile_expert &&
                tile_row0 && expert_tile_start && tile_lo && tile_hi && act);
  if (max_tiles == 0) return hipSuccess;
  (void)hipGetLastError();
  Gemm8Args a{hi, lo, shi, slo, sorted_tok, (const uint8_t*)w13, s13, seg_start, tile_expert,
              tile_row0, expert_tile_start, tile_lo, tile_hi, slot_map, act, H, I, w_estride,
              s_estride, limit, alpha, beta};
  return launch_gemm8(kFP8, true, a, max_tiles, stream);
}

hipError_t xtu_gemm8_down(const uint8_t* hi, const uint8_t* lo, const uint8_t* shi,
                          const uint8_t* slo, int H, int I, const void* w2, const float* s2,
                          long w_estride, long s_estride, const int32_t* slot_map,
                          const int32_t* seg_start, const int32_t* tile_expert,
                          const int32_t* tile_row0, const int32_t* expert_tile_start,
                          const int32_t* tile_lo, const int32_t* tile_hi, int max_tiles,
                          float* y, hipStream_t stream) {
  XTU_CHECK_ARG(H > 0 && I > 0 && H % 256 == 0 && I % 128 == 0 && I <= 65536);
  XTU_CHECK_ARG(max_tiles >= 0 && max_tiles < (1 << 30) && w_estride >= 0 && s_estride >= 0);
  XTU_CHECK_ARG(w_estride < (1L << 31) && (long)H * I < (1L << 31));
  XTU_CHECK_ARG(hi && lo && shi && slo && w2 && s2 && seg_start && tile_expert && tile_row0 &&
                expert_tile_start && tile_lo && tile_hi && y);
  if (max_tiles == 0) return hipSuccess;
  (void)hipGetLastError();
  Gemm8Args a{hi, lo, shi, slo, nullptr, (const uint8_t*)w2, s2, seg_start, tile_expert,
              tile_row0, expert_tile_start, tile_lo, tile_hi, slot_map, y, H, I, w_estride,
              s_estride, 0.f, 1.f, 0.f};
  return launch_gemm8(kFP8, false, a, max_tiles, stream);
}

// Exact-pair grouped GEMMs for FP8 (fp32 block scales) or MXFP4 (packed e8m0
// scale groups) weights: xtu_gemm8_* with the weight format as an argument.
hipError_t xtu_gemm_pair_gate_up(int fmt, const uint8_t* hi, const uint8_t* lo,
                                 const uint8_t* shi, const uint8_t* slo,
                                 const int32_t* sorted_tok, int H, int I, const void* w13,
                                 const void* s13, long w_estride, long s_estride,
                                 const int32_t* slot_map, const int32_t* seg_start,
                                 const int32_t* tile_expert, const int32_t* tile_row0,
                                 const int32_t* expert_tile_start, const int32_t* tile_lo,
                                 const int32_t* tile_hi, int max_tiles, void* act, float limit,
                                 float alpha, float beta, hipStream_t stream) {
  XTU_CHECK_ARG(fmt == kFP8 || fmt == kMXFP4);
  XTU_CHECK_ARG(H > 0 && I > 0 && H % 256 == 0 && I % 128 == 0 && H <= 65536);
  XTU_CHECK_ARG(max_tiles >= 0 && max_tiles < (1 << 30) && w_estride >= 0 && s_estride >= 0);
  XTU_CHECK_ARG(w_estride < (1L << 31) && 2L * I * H < (1L << 31));
  XTU_CHECK_ARG(hi && lo && shi && slo && sorted_tok && w13 && s13 && seg_start && tile_expert &&
                tile_row0 && expert_tile_start && tile_lo && tile_hi && act);
  if (max_tiles == 0) return hipSuccess;
  (void)hipGetLastError();
  Gemm8Args a{hi, lo, shi, slo, sorted_tok, (const uint8_t*)w13, (const float*)s13, seg_start,
              tile_expert, tile_row0, expert_tile_start, tile_lo, tile_hi, slot_map, act, H, I,
              w_estride, s_estride, limit, alpha, beta};
  return launch_gemm8(fmt, true, a, max_tiles, stream);
}

hipError_t xtu_gemm_pair_down(int fmt, const uint8_t* hi, const uint8_t* lo, const uint8_t* shi,
                              const uint8_t* slo, int H, int I, const void* w2, const void* s2,
                              long w_estride, long s_estride, const int32_t* slot_map,
                              const int32_t* seg_start, const int32_t* tile_expert,
                              const int32_t* tile_row0, const int32_t* expert_tile_start,
                              const int32_t* tile_lo, const int32_t* tile_hi, int max_tiles,
                              float* y, hipStream_t stream) {
  XTU_CHECK_ARG(fmt == kFP8 || fmt == kMXFP4);
  XTU_CHECK_ARG(H > 0 && I > 0 && H % 256 == 0 && I % 128 == 0 && I <= 65536);
  XTU_CHECK_ARG(max_tiles >= 0 && max_tiles < (1 << 30) && w_estride >= 0 && s_estride >= 0);
  XTU_CHECK_ARG(w_estride < (1L << 31) && (long)H * I < (1L << 31));
  XTU_CHECK_ARG(hi && lo && shi && slo && w2 && s2 && seg_start && tile_expert && tile_row0 &&
                expert_tile_start && tile_lo && tile_hi && y);
  if (max_tiles == 0) return hipSuccess;
  (void)hipGetLastError();
  Gemm8Args a{hi, lo, shi, slo, nullptr, (const uint8_t*)w2, (const float*)s2, seg_start,
              tile_expert, tile_row0, expert_tile_start, tile_lo, tile_hi, slot_map, y, H, I,
              w_estride, s_estride, 0.f, 1.f, 0.f};
  return launch_gemm8(fmt, false, a, max_tiles, stream);
}

}  // extern "C"
