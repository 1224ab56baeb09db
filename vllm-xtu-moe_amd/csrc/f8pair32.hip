// Exact-pair grouped GEMMs for FP8 weights (e4m3 codes, fp32 128 x 128 block
// scales) on v_mfma_scale_f32_32x32x64_f8f6f4 (e4m3 x e4m3), both operands
// staged through LDS by direct-to-LDS loads, four stages deep (three where
// LDS does not hold four).
//
// Activations: the interleaved e4m3 pairs of xtu_pair_quant_il (row r is
// [K/64][hi 64 B | lo 64 B], e8m0 bytes [rows][K/32]), as for MXFP4.
// Weights: the e4m3 P16 panels; one 64-k step of a 16-row panel is one
// 1 KiB block [4 chunks][16 rows][16 B], copied to LDS as it is.
//
// Block scales.  A 128 x 128 block scale s(kb) multiplies the products of
// one 128-k block of one 128-row weight block.  The MFMAs accumulate into
// acc directly and, at each block boundary, acc is rescaled:
//   acc = acc * (s(kb-1) / s(kb)),   then the MFMAs of block kb,
// and the epilogue multiplies by s(last): acc = sum_kb s(kb) P(kb) up to one
// rounding of each ratio and each rescale (relative ~1e-7 per block).  This
// costs one multiply per accumulator per 128 k (4 per MFMA) and no
// partial-sum registers, so a wave holds 64 x 128 accumulators (128
// registers) and reads the MFMA results only in the epilogue.  Every block
// scale of the weights must be positive and finite (the host checks).
//
// Work item: 128 rows of one expert's sorted pairs (bm = 128) x 256 weight
// rows (gate/up: 128 gate rows and the matching 128 up rows; down: 256
// output columns), K in steps of 64.  Items expert-major, then N block, then
// m tile, dealt to the eight XCDs in contiguous ranges.  Four waves: wave w
// takes the 32-row blocks (w & 1) and (w & 1) + 2 of the tile and the 128
// weight rows of half w >> 1 (gate/up: 64 gate + the matching 64 up), four
// 32 x 32 blocks per row block.
//
// Operand layout of the 32x32x64 MFMA (checked on the device): lane l is row
// (column) l % 32, h = l / 32; an e4m3 operand lane holds k = 16h..16h+15
// and 32+16h..32+16h+15 of the 64-k block -- for a weight row, chunks h and
// 2 + h of its P16 super-block; the e8m0 scale of an A lane applies to its
// row and the 32-k block h.
//
// Pipeline: step s issues the loads of step s + STAGES - 1 between the first
// half of its MFMAs, waits for step s + 1 and meets the barrier, then reads
// the fragments of step s + 1 between the second half.  A step is 16 MFMAs
// per wave (half the MXFP4 kernel's), so the loads need the deeper lead.
#include <type_traits>

#include "pairgemm.hpp"

namespace xtu {
namespace {

typedef int i32x8_t __attribute__((ext_vector_type(8)));

constexpr int kQM = 128;            // rows per m tile
constexpr int kQN = 256;            // weight rows per work item
constexpr int kQThreads = 256;
constexpr int kQLA = kQM * 128;     // A codes [row][8 pieces of 16 B]
constexpr int kQLB = kQN * 64;      // B codes: 16 panels x 1 KiB
constexpr int kQStage = kQLA + kQLB;
constexpr int kQLdsMax = 160 * 1024;
constexpr int kQLoads = 8;          // loads per lane and step (A 4, B 4)

// stages | activation scales | source rows | ratios [2][K/128] + finals [2]
__host__ __device__ constexpr int q_lds_bytes(int stages, int K) {
  return stages * kQStage + asc_bytes(K, kQM) + 4 * kQM + 4 * (2 * (K / 128) + 2);
}

struct F8PairArgs {
  const uint8_t* hilo;        // gate/up: x pairs [T][2K]; down: act pairs [A][2K]
  const uint8_t* shi;         // [rows][K/32] e8m0 of hi
  const int32_t* sorted_tok;  // gate/up row gather
  const uint8_t* w;           // P16 e4m3 codes, expert-major
  const float* s;             // fp32 block scales [N/128][K/128] per expert
  const int32_t* seg_start;
  const int32_t* tile_expert;
  const int32_t* tile_row0;
  const int32_t* expert_tile_start;
  const int32_t* tile_lo;
  const int32_t* tile_hi;
  const int32_t* slot_map;
  void* out;                  // gate/up: act bf16 [A][I] (or its pairs [A][2I], qs set);
                              // down: y fp32 [A][H]
  int H, I;
  long w_estride, s_estride;
  float limit, alpha, beta;
  uint8_t* qs;                // gate/up: null, or the e8m0 bytes [A][I/32] of act written
                              // as exact pairs for the down pass
};

template <bool GU, int STAGES>
__global__ __launch_bounds__(kQThreads, 1) void f8_pair_gemm_kernel(F8PairArgs a) {
  constexpr int LEAD = STAGES - 1;   // steps of loads in flight ahead of the MFMAs
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

  // ---- work item
  const int nbn = GU ? a.I / 128 : a.H / 256;
  const int tlo = a.tile_lo[0];
  const int total = (a.tile_hi[0] - tlo) * nbn;
  const int per = (total + 7) / 8;
  const int idx = blockIdx.x / 8;
  if (idx >= per) return;
  const int item = (blockIdx.x % 8) * per + idx;
  if (item >= total) return;
  const int j0 = tlo + item / nbn;
  const int e = a.tile_expert[j0];
  const int t0 = a.expert_tile_start[e];
  const int ntl = a.expert_tile_start[e + 1] - t0;
  const int local = tlo * nbn + item - t0 * nbn;
  const int nb = local / ntl, tile = t0 + local % ntl;
  const int ws = a.slot_map ? a.slot_map[e] : e;
  const int row0 = a.tile_row0[tile];
  const int rows = min(kQM, a.seg_start[e + 1] - row0);
  const int K = GU ? a.H : a.I;
  const int nsteps = K / 64, nkb = K / 128;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid / 64);
  const int lane = tid % 64;
  const int wm = w & 1, wn = w >> 1;
  const int ascs = asc_stride(K);
  uint8_t* asc = lds + STAGES * kQStage;
  int32_t* srow = reinterpret_cast<int32_t*>(asc + asc_bytes(K, kQM));
  float* ratio = reinterpret_cast<float*>(srow + kQM);   // [2][nkb], then finals [2]

  const long nw = GU ? 2L * a.I : (long)a.H;
  const long w_es = a.w_estride ? a.w_estride : WFmt<kFP8>::w_bytes(nw, K);
  const long s_es = a.s_estride ? a.s_estride : WFmt<kFP8>::s_bytes(nw, K);
  const uint8_t* wexp = a.w + (long)ws * w_es;
  const float* bsc = reinterpret_cast<const float*>(reinterpret_cast<const uint8_t*>(a.s) +
                                                    (long)ws * s_es);
  // the item's two 128-row scale blocks: gate/up the gate block and the up
  // block of columns nb * 128 ..; down blocks 2 nb and 2 nb + 1
  const int rb[2] = {GU ? nb : 2 * nb, GU ? a.I / 128 + nb : 2 * nb + 1};

  // source row of every tile row (rows past the tile repeat its last row);
  // block-scale ratios s(kb - 1) / s(kb) of both blocks and their last scales
  if (tid < kQM) {
    const int rr = min(tid, rows - 1);
    srow[tid] = GU ? a.sorted_tok[row0 + rr] : row0 + rr;
  }
  for (int i = tid; i < 2 * nkb; i += kQThreads) {
    const int b = i / nkb, kb = i % nkb;
    const float* sr = bsc + (long)rb[b] * nkb;
    ratio[i] = kb == 0 ? 1.0f : sr[kb - 1] / sr[kb];
  }
  if (tid < 2) ratio[2 * nkb + tid] = bsc[(long)rb[tid] * nkb + nkb - 1];
  __syncthreads();

  // ---- A codes: instruction i of wave w covers tile rows 8 (4 w + i) ..
  // + 8: lane l holds row 8 (4 w + i) + l / 8, slot l % 8, i.e. piece
  // (l % 8) ^ (row & 7) of the row's 128-byte line
  uint32_t aoff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    aoff[i] = (uint32_t)srow[8 * (4 * w + i) + lane / 8] * (uint32_t)(2 * K) +
              (uint32_t)(((lane % 8) ^ (lane / 8)) * 16);

  // ---- weights: local panel p (16 rows) of the item -> global P16 panel
  auto gpanel = [&](int p) -> long {
    if (GU) return p < 8 ? nb * 8 + p : a.I / 16 + nb * 8 + (p - 8);
    return nb * 16 + p;
  };
  const long wpanel = (long)(K / 64) * 1024;   // bytes of one panel

  auto issue_one = [&](int s, int st, int d) {
    const uint8_t* sb = lds + st * kQStage;
    if (d < 4) {
      dma16(a.hilo + s * 128, aoff[d], sb + (4 * w + d) * 1024);
    } else {
      const int p = 4 * w + (d - 4);
      dma16(wexp + gpanel(p) * wpanel + s * 1024, 16 * lane, sb + kQLA + p * 1024);
    }
  };

  // ---- activation scales of the tile's rows, all of K (row r at r * ascs)
  {
    const int ascw = ascs / 4, nch = asc_bytes(K, kQM) / 256;
    for (int c = w; c < nch; c += 4) {
      const int d = 64 * c + lane;
      const int r = min(d / ascw, kQM - 1), q = d % ascw;
      dma4(a.shi, (uint32_t)srow[r] * (uint32_t)(K / 32) + 4 * (q < K / 128 ? q : 0), asc + 256 * c);
    }
  }

  // ---- fragments of this lane: A row blocks wm, wm + 2; B blocks cb of the
  // wave's 128 weight rows (gate/up: cb 0, 1 gate, 2, 3 the matching up)
  const int r32 = lane % 32, h = lane / 32;
  int arow[2];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) arow[mb] = 32 * (2 * mb + wm) + r32;
  const bool two_blocks = 32 * (2 + wm) < rows;
  int bofs[4];   // LDS offset of the column's chunk h inside a stage's B area
#pragma unroll
  for (int cb = 0; cb < 4; ++cb) {
    const int C = GU ? (cb < 2 ? 0 : 128) + 64 * wn + 32 * (cb % 2) + r32 : 128 * wn + 32 * cb + r32;
    bofs[cb] = (C / 16) * 1024 + h * 256 + (C % 16) * 16;
  }
  // scale block of B block cb: gate/up 0 for gate, 1 for up; down wn
  auto blk_of = [&](int cb) { return GU ? (cb < 2 ? 0 : 1) : wn; };

  f32x16_t acc[2][4];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[mb][cb][i] = 0.f;

  struct Frags {
    i32x8_t a[2][2];   // [mb][plane]
    int sa[2];         // e8m0 of hi; lo's is max(sa - 4, 0)
    i32x8_t b[4];
  };
  // fragment read k of step s: 0-3 B block k, 4-7 A row block (k - 4) / 2
  // plane (k - 4) % 2, 8-9 the A scale of row block k - 8
  constexpr int kReads = 10;
  auto read_one = [&](const uint8_t* buf, int s, Frags& f, int k) {
    if (k < 4) {
      const uint8_t* bp = buf + kQLA + bofs[k];
      const u32x4_t x0 = *reinterpret_cast<const u32x4_t*>(bp);
      const u32x4_t x1 = *reinterpret_cast<const u32x4_t*>(bp + 512);
      f.b[k] = i32x8_t{(int)x0[0], (int)x0[1], (int)x0[2], (int)x0[3],
                       (int)x1[0], (int)x1[1], (int)x1[2], (int)x1[3]};
    } else if (k < 8) {
      const int mb = (k - 4) / 2, p = (k - 4) % 2, R = arow[mb];
      const uint8_t* base = buf + R * 128;
      const u32x4_t x0 = *reinterpret_cast<const u32x4_t*>(base + 16 * ((4 * p + h) ^ (R & 7)));
      const u32x4_t x1 = *reinterpret_cast<const u32x4_t*>(base + 16 * ((4 * p + 2 + h) ^ (R & 7)));
      f.a[mb][p] = i32x8_t{(int)x0[0], (int)x0[1], (int)x0[2], (int)x0[3],
                           (int)x1[0], (int)x1[1], (int)x1[2], (int)x1[3]};
    } else {
      f.sa[k - 8] = asc[arow[k - 8] * ascs + 2 * s + h];
    }
  };
  // MFMA j (0..7) of row block mb: plane j / 4, B block j % 4
  auto mfma_one = [&](const Frags& f, int mb, int j) {
    const int p = j / 4, cb = j % 4;
    const int sa = p == 0 ? f.sa[mb] : (f.sa[mb] >= 4 ? f.sa[mb] - 4 : 0);
    acc[mb][cb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.a[mb][p], f.b[cb], acc[mb][cb],
                                                                  0, 0, 0, sa, 0, 127);
  };
  // rescale before block kb (the accumulators hold blocks up to kb - 1):
  // one 32 x 32 block, or (rescale_all) every live one
  auto ratio_of = [&](int cb, int kb) { return blk_of(cb) ? ratio[nkb + kb] : ratio[kb]; };
  auto rescale_one = [&](int mb, int cb, float r) {
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[mb][cb][i] *= r;
  };
  auto rescale_all = [&](int live, int kb) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      if (mb >= live) break;
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) rescale_one(mb, cb, ratio_of(cb, kb));
    }
  };

  // ---- pipeline: the loads of step s + LEAD are issued during step s
  // (nsteps = K / 64 is even and >= 2)
#pragma unroll
  for (int p = 0; p < LEAD; ++p) {
    if (p < nsteps) {
#pragma unroll
      for (int d = 0; d < kQLoads; ++d) issue_one(p, p, d);
    }
  }
  if (nsteps >= LEAD) __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0((LEAD - 1) * kQLoads));
  else __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(0));   // scales, step 0 landed
  __syncthreads();
  auto run = [&](auto live_c) {
    constexpr int LIVE = decltype(live_c)::value;
    constexpr int M = 8 * LIVE, H2 = M / 2;
    auto mfma_j = [&](const Frags& f, int j) { mfma_one(f, j / 8, j % 8); };
    // reads this variant needs: B 0-3, A row block 0 (4, 5), its scale (8),
    // and with two blocks A row block 1 (6, 7) and its scale (9)
    auto read_k = [&](int n) { return LIVE == 2 ? n : (n < 6 ? n : 8); };
    constexpr int kR = LIVE == 2 ? kReads : (LIVE == 1 ? 7 : 0);
    // Step s: the MFMAs of step s (fragments in cur); ISSUE: the loads of
    // step s + LEAD between the first half; NEXT: wait for step s + 1, the
    // barrier, and its fragments (into nxt) between the second half.
    // Rescaling with two row blocks: a 32 x 32 block's multiplies follow an
    // MFMA of the other row block (they issue while it runs): row block 0's
    // at the second half of an odd step before a block start (after its last
    // MFMA of block kb - 1), row block 1's at the first half of the even step
    // (before its first MFMA of block kb; step 0 multiplies by ratio 1).  One
    // row block: all of it at the even step's start.
    auto step = [&](auto odd_c, auto issue_c, auto next_c, int s, Frags& cur, Frags& nxt) {
      constexpr bool ODD = decltype(odd_c)::value;
      constexpr bool ISSUE = decltype(issue_c)::value;
      constexpr bool NEXT = decltype(next_c)::value;
      constexpr bool RS0 = LIVE == 2 && ODD && NEXT;   // row block 0, ratio (s + 1) / 2
      constexpr bool RS1 = LIVE == 2 && !ODD;          // row block 1, ratio s / 2
      float rr[4];
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (LIVE == 1 && !ODD) {
        if (s > 0) rescale_all(1, s / 2);
      }
      if constexpr (RS0 || RS1) {
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) rr[cb] = ratio_of(cb, ODD ? (s + 1) / 2 : s / 2);
      }
      __builtin_amdgcn_sched_barrier(0);
      const int sn = s + LEAD, stn = sn % STAGES;
      int d = 0;
#pragma unroll
      for (int j = 0; j < H2; ++j) {
        mfma_j(cur, j);
        if constexpr (RS1) {
          if (j < 4) rescale_one(1, j, rr[j]);
        }
        if constexpr (ISSUE) {
          if (d < kQLoads) issue_one(sn, stn, d++);
          if (LIVE == 1 && d < kQLoads) issue_one(sn, stn, d++);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (ISSUE) {
#pragma unroll
        for (; d < kQLoads; ++d) issue_one(sn, stn, d);
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (NEXT) {
        // step s + 1 landed: with ISSUE the later LEAD - 1 steps may still
        // be in flight; in the last steps wait for everything
        if constexpr (ISSUE) __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0((LEAD - 1) * kQLoads));
        else __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(0));
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t* buf = lds + ((s + 1) % STAGES) * kQStage;
        int n = 0;
#pragma unroll
        for (int j = H2; j < M; ++j) {
          if (n < kR) read_one(buf, s + 1, nxt, read_k(n++));
          if (n < kR) read_one(buf, s + 1, nxt, read_k(n++));
          mfma_j(cur, j);
          if constexpr (RS0) {
            if (j - H2 < 4) rescale_one(0, j - H2, rr[j - H2]);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (; n < kR; ++n) read_one(buf, s + 1, nxt, read_k(n));
      } else {
#pragma unroll
        for (int j = H2; j < M; ++j) mfma_j(cur, j);
      }
    };
    using T_ = std::true_type;
    using F_ = std::false_type;
    Frags f0, f1;
#pragma unroll
    for (int n = 0; n < kR; ++n) read_one(lds, 0, f0, read_k(n));
    int s = 0;
    for (; s + 1 + LEAD < nsteps; s += 2) {   // both steps issue
      step(F_{}, T_{}, T_{}, s, f0, f1);
      step(T_{}, T_{}, T_{}, s + 1, f1, f0);
    }
    // the rest: four steps (LEAD 3, nsteps >= 4), the first of them issuing
    // the last loads, or two
    if (LEAD == 3 && nsteps - s == 4) {
      step(F_{}, T_{}, T_{}, s, f0, f1);
      step(T_{}, F_{}, T_{}, s + 1, f1, f0);
      s += 2;
    }
    step(F_{}, F_{}, T_{}, s, f0, f1);
    step(T_{}, F_{}, F_{}, s + 1, f1, f0);
  };
  // a wave whose blocks both lie past the tile (tiles of at most 32 rows,
  // wm = 1) keeps its part of the loads and barriers and computes nothing
  if (two_blocks) run(std::integral_constant<int, 2>{});
  else if (32 * wm < rows) run(std::integral_constant<int, 1>{});
  else run(std::integral_constant<int, 0>{});

  // ---- epilogue: the last block's scale, then the 32x32 result layout
  // (column l % 32, rows 8 (i / 4) + 4 (l / 32) + i % 4).  Each wave's
  // results go through its own LDS region (the stages are free once every
  // wave is past the K loop) and are read back as 16-byte row pieces: wide
  // stores of whole row segments instead of one store per lane and value.
  const float sl0 = ratio[2 * nkb], sl1 = ratio[2 * nkb + 1];
  __syncthreads();
  if constexpr (GU) {
    constexpr int kAP = 72;   // staged row pitch in bf16 (64 + 8)
    uint16_t* stage = reinterpret_cast<uint16_t*>(lds) + w * (32 * kAP);
    uint16_t* act = reinterpret_cast<uint16_t*>(a.out);
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const int rb = 32 * (2 * mb + wm);
      if (rb >= rows) continue;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = 8 * (i / 4) + 4 * h + (i % 4);
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
          stage[r * kAP + 32 * cb + r32] = f32_to_bf16(silu_gate(
              acc[mb][cb][i] * sl0, acc[mb][cb + 2][i] * sl1, a.limit, a.alpha, a.beta));
      }
      __builtin_amdgcn_wave_barrier();
      if (a.qs) {
        // the down pass's pairs straight from the staged bf16 rows (the
        // values the act quantiser would read back): 32 rows x 2 blocks of
        // 32 k, one per lane
        const int rr = lane / 2, cb = lane % 2;
        if (rb + rr < rows) {
          const long row = row0 + rb + rr;
          const int blk = nb * 4 + wn * 2 + cb;
          uint32_t hw[8], lw[8];
          const int sa = pair_split32(stage + rr * kAP + 32 * cb, hw, lw);
          uint8_t* d = reinterpret_cast<uint8_t*>(a.out) + row * 2L * a.I + (blk / 2) * 128 +
                       (blk % 2) * 32;
          *reinterpret_cast<u32x4_t*>(d) = u32x4_t{hw[0], hw[1], hw[2], hw[3]};
          *reinterpret_cast<u32x4_t*>(d + 16) = u32x4_t{hw[4], hw[5], hw[6], hw[7]};
          *reinterpret_cast<u32x4_t*>(d + 64) = u32x4_t{lw[0], lw[1], lw[2], lw[3]};
          *reinterpret_cast<u32x4_t*>(d + 80) = u32x4_t{lw[4], lw[5], lw[6], lw[7]};
          a.qs[row * (a.I / 32) + blk] = (uint8_t)sa;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {   // 32 rows x 8 pieces of 8 bf16
          const int q = 64 * j + lane, rr = q / 8, c8 = q % 8;
          if (rb + rr < rows)
            *reinterpret_cast<u32x4_t*>(act + (long)(row0 + rb + rr) * a.I + (long)nb * 128 +
                                        64 * wn + 8 * c8) =
                *reinterpret_cast<const u32x4_t*>(stage + rr * kAP + 8 * c8);
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
  } else {
    constexpr int kYP = 136;   // staged row pitch in floats (128 + 8)
    float* stage = reinterpret_cast<float*>(lds) + w * (32 * kYP);
    float* y = reinterpret_cast<float*>(a.out);
    const float sl = wn ? sl1 : sl0;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const int rb = 32 * (2 * mb + wm);
      if (rb >= rows) continue;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = 8 * (i / 4) + 4 * h + (i % 4);
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) stage[r * kYP + 32 * cb + r32] = acc[mb][cb][i] * sl;
      }
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int j = 0; j < 16; ++j) {   // 32 rows x 32 pieces of 4 floats
        const int q = 64 * j + lane, rr = q / 32, c4 = q % 32;
        if (rb + rr < rows)
          *reinterpret_cast<f32x4_t*>(y + (long)(row0 + rb + rr) * a.H + (long)nb * 256 +
                                      128 * wn + 4 * c4) =
              *reinterpret_cast<const f32x4_t*>(stage + rr * kYP + 4 * c4);
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
}

// Shapes the kernel takes: gate/up N blocks of 128 gate rows, down of 256
// columns, K = H and K = I multiples of 128 (whole block scales, an even
// number of 64-k steps, at least 4), LDS for the activation scales of 128
// rows.
bool f8_fits(int H, int I) {
  return H > 0 && I > 0 && I % 128 == 0 && H % 256 == 0 && q_lds_bytes(3, H) <= kQLdsMax &&
         q_lds_bytes(3, I) <= kQLdsMax;
}

hipError_t f8_launch(bool gu, const F8PairArgs& a, int max_tiles, hipStream_t stream) {
  const long items = (long)max_tiles * (gu ? a.I / 128 : a.H / 256);
  const long grid = (items + 7) / 8 * 8;
  if (grid >= (1L << 31)) return hipErrorInvalidValue;
  if (grid == 0) return hipSuccess;
  const dim3 g((unsigned)grid);
  // four stages (three steps of loads ahead) where LDS holds them
  const int K = gu ? a.H : a.I;
  const bool deep = q_lds_bytes(4, K) <= kQLdsMax;
  const size_t lds = q_lds_bytes(deep ? 4 : 3, K);
  if (gu && deep) f8_pair_gemm_kernel<true, 4><<<g, kQThreads, lds, stream>>>(a);
  else if (gu) f8_pair_gemm_kernel<true, 3><<<g, kQThreads, lds, stream>>>(a);
  else if (deep) f8_pair_gemm_kernel<false, 4><<<g, kQThreads, lds, stream>>>(a);
  else f8_pair_gemm_kernel<false, 3><<<g, kQThreads, lds, stream>>>(a);
  return hipPeekAtLastError();
}

}  // namespace
}  // namespace xtu

using namespace xtu;

extern "C" {

int xtu_f8_pair_fits(int H, int I) { return f8_fits(H, I) ? 1 : 0; }

int xtu_f8_pair_tile_m(void) { return kQM; }

hipError_t xtu_f8_pair_gate_up(const uint8_t* hilo, const uint8_t* shi, const int32_t* sorted_tok,
                               int H, int I, const void* w13, const float* s13, long w_estride,
                               long s_estride, const int32_t* slot_map, const int32_t* seg_start,
                               const int32_t* tile_expert, const int32_t* tile_row0,
                               const int32_t* expert_tile_start, const int32_t* tile_lo,
                               const int32_t* tile_hi, int max_tiles, void* act, float limit,
                               float alpha, float beta, hipStream_t stream) {
  XTU_CHECK_ARG(f8_fits(H, I));
  XTU_CHECK_ARG(max_tiles >= 0 && max_tiles < (1 << 30) && w_estride >= 0 && s_estride >= 0);
  XTU_CHECK_ARG(2L * I * H < (1L << 32));
  XTU_CHECK_ARG(hilo && shi && sorted_tok && w13 && s13 && seg_start && tile_expert &&
                tile_row0 && expert_tile_start && tile_lo && tile_hi && act);
  if (max_tiles == 0) return hipSuccess;
  (void)hipGetLastError();
  F8PairArgs a{hilo, shi, sorted_tok, (const uint8_t*)w13, s13, seg_start, tile_expert, tile_row0,
               expert_tile_start, tile_lo, tile_hi, slot_map, act, H, I, w_estride, s_estride,
               limit, alpha, beta, nullptr};
  return f8_launch(true, a, max_tiles, stream);
}

hipError_t xtu_f8_pair_gate_up_q(const uint8_t* hilo, const uint8_t* shi,
                                 const int32_t* sorted_tok, int H, int I, const void* w13,
                                 const float* s13, long w_estride, long s_estride,
                                 const int32_t* slot_map, const int32_t* seg_start,
                                 const int32_t* tile_expert, const int32_t* tile_row0,
                                 const int32_t* expert_tile_start, const int32_t* tile_lo,
                                 const int32_t* tile_hi, int max_tiles, uint8_t* act_hilo,
                                 uint8_t* act_shi, float limit, float alpha, float beta,
                                 hipStream_t stream) {
  XTU_CHECK_ARG(f8_fits(H, I));
  XTU_CHECK_ARG(max_tiles >= 0 && max_tiles < (1 << 30) && w_estride >= 0 && s_estride >= 0);
  XTU_CHECK_ARG(2L * I * H < (1L << 32));
  XTU_CHECK_ARG(hilo && shi && sorted_tok && w13 && s13 && seg_start && tile_expert &&
                tile_row0 && expert_tile_start && tile_lo && tile_hi && act_hilo && act_shi);
  if (max_tiles == 0) return hipSuccess;
  (void)hipGetLastError();
  F8PairArgs a{hilo, shi, sorted_tok, (const uint8_t*)w13, s13, seg_start, tile_expert, tile_row0,
               expert_tile_start, tile_lo, tile_hi, slot_map, act_hilo, H, I, w_estride,
               s_estride, limit, alpha, beta, act_shi};
  return f8_launch(true, a, max_tiles, stream);
}

hipError_t xtu_f8_pair_down(const uint8_t* hilo, const uint8_t* shi, int H, int I, const void* w2,
                            const float* s2, long w_estride, long s_estride,
                            const int32_t* slot_map, const int32_t* seg_start,
                            const int32_t* tile_expert, const int32_t* tile_row0,
                            const int32_t* expert_tile_start, const int32_t* tile_lo,
                            const int32_t* tile_hi, int max_tiles, void* y, hipStream_t stream) {
  XTU_CHECK_ARG(f8_fits(H, I));
  XTU_CHECK_ARG(max_tiles >= 0 && max_tiles < (1 << 30) && w_estride >= 0 && s_estride >= 0);
  XTU_CHECK_ARG((long)H * I < (1L << 32));
  XTU_CHECK_ARG(hilo && shi && w2 && s2 && seg_start && tile_expert && tile_row0 &&
                expert_tile_start && tile_lo && tile_hi && y);
  if (max_tiles == 0) return hipSuccess;
  (void)hipGetLastError();
  F8PairArgs a{hilo, shi, nullptr, (const uint8_t*)w2, s2, seg_start, tile_expert, tile_row0,
               expert_tile_start, tile_lo, tile_hi, slot_map, y, H, I, w_estride, s_estride,
               0.f, 1.f, 0.f, nullptr};
  return f8_launch(false, a, max_tiles, stream);
}

}  // extern "C"
