// Exact-pair grouped GEMMs for MXFP4 weights on
// v_mfma_scale_f32_32x32x64_f8f6f4 (e4m3 activations x e2m1 weights), with
// the two operand layouts this kernel reads made for it:
//
// * activation pairs interleaved (xtu_pair_quant_il): row r of the plane is
//   [K/64 chunks][hi 64 B | lo 64 B], so the codes one 64-k step needs of a
//   row are one 128-byte line; the e8m0 bytes stay [rows][K/32].
// * weight scales step-major (xtu_mx_pair_scales, a re-layout of the packed
//   MXFP4 scale groups): [expert][K/64][N/16 panels][16 rows][2] bytes (the
//   two 32-k blocks of the step), so the scales of the work item's 512
//   weight rows for one step are one or two contiguous runs.
//
// Per 64-k step and 32 x 32 block:
//   acc = mfma(hi, w, acc; sa, sw) ; acc = mfma(lo, w, acc; sl, sw)
// with sl = max(sa - 4, 0) -- the weight's e8m0 byte is the MFMA's B scale,
// so every product is the dequantised-fp32 one and only the fp32 summation
// order differs.
//
// Work item: 128 rows of one expert's sorted pairs (an m tile of the
// segmentation, bm = 128) x 512 weight rows (gate/up: 256 gate rows and the
// matching 256 up rows; down: 512 output columns), K in steps of 64.  Items
// are expert-major, then N block, then m tile, dealt to the eight XCDs in
// contiguous ranges.  Four waves, each 64 rows x 256 weight rows (2 x 8
// blocks of 32 x 32, 256 accumulator registers).
//
// Operand layout of the 32x32x64 MFMA (checked on the device): lane l is row
// (column) l % 32, h = l / 32; an e4m3 operand lane holds k = 16h..16h+15
// (bytes 0-15) and 32+16h..32+16h+15 (bytes 16-31) of the 64-k block; an
// e2m1 operand lane holds k = 32h..32h+31 (16 bytes, low nibble first) --
// one P16 fp4 chunk; the e8m0 scale byte of a lane applies to its row
// (column) and the 32-k block h.
//
// LDS: the activation scales of the item's 128 rows for all of K, loaded
// once (with the rows' source indices); three stages of [A 128 rows x 128 B
// | B 512 x 32 B | B scales 1 KB]
// filled straight from memory by global_load_lds_dwordx4 / _dword (lane l's
// bytes land at the instruction's LDS base + 16 l / 4 l, so each lane loads
// the piece that belongs at its slot).  A row's eight 16-byte pieces (hi
// 0-3, lo 4-7) sit at slot piece ^ (row & 7), B's two at slot
// piece ^ ((col >> 3) & 1): the b128 fragment reads of consecutive rows hit
// distinct banks.
//
// Step s (one barrier): issue the loads of step s + 2 into the stage last
// read for step s - 1 (before the barrier of step s - 1); the MFMAs of row
// block 0 on the fragments of step s (read during step s - 1); wait until
// this wave's loads of step s + 1 have landed (the loads of step s + 2 may
// still be in flight) and its LDS reads are done; barrier; read the
// fragments of step s + 1; the MFMAs of row block 1.
#include <type_traits>

#include "pairgemm.hpp"

namespace xtu {
namespace {

typedef int i32x8_t __attribute__((ext_vector_type(8)));

constexpr int kPM = 128;            // rows per m tile
constexpr int kPN = 512;            // weight rows per work item
constexpr int kPThreads = 256;

constexpr int kLA = kPM * 128;      // A codes [row][8 pieces of 16 B]
constexpr int kLB = kPN * 32;       // B codes [col][2 pieces of 16 B]
constexpr int kLBS = kPN * 2;       // B scales [col][2]
constexpr int kStage = kLA + kLB + kLBS;
constexpr int kLdsMax = 160 * 1024;

// stages, the activation-scale area of 128 rows, then the tile's 128 source
// rows
__host__ __device__ constexpr int lds_bytes(int stages, int K) {
  return stages * kStage + asc_bytes(K, kPM) + 4 * kPM;
}

constexpr int kLoadsPerStep = 9;    // loads per lane and step (A 4, B 4, B scales 1)

struct MxPairArgs {
  const uint8_t* hilo;        // gate/up: x pairs [T][2K]; down: act pairs [A][2K]
  const uint8_t* shi;         // [rows][K/32] e8m0 of hi
  const int32_t* sorted_tok;  // gate/up row gather
  const uint8_t* w;           // P16 e2m1 codes, expert-major
  const uint8_t* s;           // step-major e8m0 [K/64][N/16][16][2] per expert
  const int32_t* seg_start;
  const int32_t* tile_expert;
  const int32_t* tile_row0;
  const int32_t* expert_tile_start;
  const int32_t* tile_lo;
  const int32_t* tile_hi;
  const int32_t* slot_map;
  void* out;                  // gate/up: act bf16 [A][I] (or its pairs / triples [A][2I],
                              // qs set); down: y fp32 [A][H]
  int H, I;
  long w_estride, s_estride;
  float limit, alpha, beta;
  uint8_t* qs;                // gate/up: null, or the e8m0 bytes [A][I/32] of act written
                              // quantised for the down pass (pairs in kPair, else triples)
};

// ---------------------------------------------------------------------------
// bf16 rows -> interleaved pairs; one thread per (row, 32-k block)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void mx_pair_quant_kernel(const uint16_t* __restrict__ x, int M,
                                                            int K, uint8_t* __restrict__ hilo,
                                                            uint8_t* __restrict__ shi) {
  const long nb = (long)M * (K / 32);
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nb) return;
  const long row = i / (K / 32), blk = i % (K / 32);
  uint32_t hw[8], lw[8];
  const int sa = pair_split32(x + row * K + blk * 32, hw, lw);
  uint8_t* d = hilo + row * 2L * K + (blk / 2) * 128 + (blk % 2) * 32;
  *reinterpret_cast<u32x4_t*>(d) = u32x4_t{hw[0], hw[1], hw[2], hw[3]};
  *reinterpret_cast<u32x4_t*>(d + 16) = u32x4_t{hw[4], hw[5], hw[6], hw[7]};
  *reinterpret_cast<u32x4_t*>(d + 64) = u32x4_t{lw[0], lw[1], lw[2], lw[3]};
  *reinterpret_cast<u32x4_t*>(d + 80) = u32x4_t{lw[4], lw[5], lw[6], lw[7]};
  shi[i] = (uint8_t)sa;
}

// bf16 rows -> interleaved triples; one thread per (row, 32-k block): the
// block's 64 bytes [p1 24 B | p2 24 B | p3 16 B] at byte 64 (blk % 2) of
// the row's 128-byte line of step blk / 2
__global__ __launch_bounds__(256) void mx_tri_quant_kernel(const uint16_t* __restrict__ x, int M,
                                                           int K, uint8_t* __restrict__ q,
                                                           uint8_t* __restrict__ sq) {
  const long nb = (long)M * (K / 32);
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nb) return;
  const long row = i / (K / 32), blk = i % (K / 32);
  uint32_t p1[6], p2[6], p3[4];
  const int s = tri_split32(x + row * K + blk * 32, p1, p2, p3);
  uint8_t* d = q + row * 2L * K + (blk / 2) * 128 + (blk % 2) * 64;
  *reinterpret_cast<u32x4_t*>(d) = u32x4_t{p1[0], p1[1], p1[2], p1[3]};
  *reinterpret_cast<u32x4_t*>(d + 16) = u32x4_t{p1[4], p1[5], p2[0], p2[1]};
  *reinterpret_cast<u32x4_t*>(d + 32) = u32x4_t{p2[2], p2[3], p2[4], p2[5]};
  *reinterpret_cast<u32x4_t*>(d + 48) = u32x4_t{p3[0], p3[1], p3[2], p3[3]};
  sq[i] = (uint8_t)s;
}

// ---------------------------------------------------------------------------
// packed MXFP4 scale groups -> step-major; one thread per output byte
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void mx_pair_scales_kernel(const uint8_t* __restrict__ s, int E,
                                                             int N, int K, long s_estride,
                                                             uint8_t* __restrict__ out) {
  const long per = (long)N * (K / 32);
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)E * per) return;
  const long e = i / per, o = i % per;
  // o = ((step * N/16 + p) * 16 + r) * 2 + c: row 16 p + r, 32-k block 2 step + c
  const int c = (int)(o % 2), r = (int)((o / 2) % 16);
  const long p = (o / 32) % (N / 16), step = o / 32 / (N / 16);
  const long j = 2 * step + c, sb = j / 4, q = j % 4;
  const long sgb = scale_groups(K, WFmt<kMXFP4>::kUG) * 1024;
  out[i] = s[e * s_estride + p * sgb + (sb / 16) * 1024 + (16 * q + r) * 16 + sb % 16];
}

// ---------------------------------------------------------------------------
// grouped GEMM
// ---------------------------------------------------------------------------
// Activation modes.  kTri: triples (fp6, fp6, fp4 pieces,
// mx_tri_quant_kernel) on the double-rate fp6 / fp4 x fp4 MFMA, three MFMAs
// per 32 x 32 block and step; kDuo: the same rows' first two pieces only
// (x ~ 2^e (p1 + p2 / 16), |error| <= 2^(e-6)), two double-rate MFMAs;
// kPair: exact e4m3 pairs, two MFMAs at the fp8 rate.
enum { kPair = 0, kTri = 1, kDuo = 2 };

template <bool GU, int MODE, int STAGES>
__global__ __launch_bounds__(kPThreads, 1) void mx_pair_gemm_kernel(MxPairArgs a) {
  constexpr bool TRI = MODE != kPair;   // the triple row layout (kTri, kDuo)
  constexpr int LEAD = STAGES - 1;   // steps of loads in flight ahead of the MFMAs
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

  // ---- work item
  const int nbn = GU ? a.I / 256 : a.H / 512;
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
  const int rows = min(kPM, a.seg_start[e + 1] - row0);
  const int K = GU ? a.H : a.I;
  const int nsteps = K / 64;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid / 64);
  const int lane = tid % 64;
  const int wm = w & 1, wn = w >> 1;
  const int ascs = asc_stride(K);
  uint8_t* asc = lds + STAGES * kStage;
  int32_t* srow = reinterpret_cast<int32_t*>(asc + asc_bytes(K, kPM));

  // source row of every tile row (rows past the tile repeat its last row)
  if (tid < kPM) {
    const int rr = min(tid, rows - 1);
    srow[tid] = GU ? a.sorted_tok[row0 + rr] : row0 + rr;
  }
  __syncthreads();

  // Every load address is a wave-uniform base (scalar registers) plus a
  // 32-bit per-lane offset: activation offsets are below rows * 2K < 2^32
  // (the quantiser's bound), weight offsets below two panels.
  //
  // ---- A codes: instruction i of wave w covers tile rows 8 (4 w + i) ..
  // + 8: lane l holds row 8 (4 w + i) + l / 8, slot l % 8, i.e. piece
  // (l % 8) ^ (row & 7) = (l % 8) ^ (l / 8) of the row's 128-byte line
  uint32_t aoff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    aoff[i] = (uint32_t)srow[8 * (4 * w + i) + lane / 8] * (uint32_t)(2 * K) +
              (uint32_t)(((lane % 8) ^ (lane / 8)) * 16);

  // ---- weights.  Local weight row c in [0, 512): gate/up rows 0..255 are
  // gate rows nb * 256 + c, rows 256..511 the up rows I + nb * 256 + c - 256;
  // down rows nb * 512 + c.  Global P16 panel of local panel p (16 rows):
  auto gpanel = [&](int p) -> long {
    if (GU) return p < 16 ? nb * 16 + p : a.I / 16 + nb * 16 + (p - 16);
    return nb * 32 + p;
  };
  const long nw = GU ? 2L * a.I : (long)a.H;
  const long w_es = a.w_estride ? a.w_estride : WFmt<kMXFP4>::w_bytes(nw, K);
  const long s_es = a.s_estride ? a.s_estride : nw * (K / 32);
  const uint8_t* wexp = a.w + (long)ws * w_es;
  const uint8_t* sexp = a.s + (long)ws * s_es;
  // chunk c = 4 w + i (i < 4) holds panels 2c, 2c + 1 (adjacent in memory
  // too): lane l -> column 32 c + l / 2 (panel 2c + l / 32, row (l / 2) % 16),
  // slot l % 2 = piece (l % 2) ^ ((col >> 3) & 1) = (l % 2) ^ ((l / 16) & 1)
  // of the step's two P16 chunks 2 (s % 2) + piece of super-block s / 2
  const long wpanel = (long)(K / 128) * 1024;
  const uint32_t boff = (uint32_t)((lane / 32) * wpanel +
                                   ((((lane % 2) ^ ((lane / 16) & 1)) * 16 + (lane / 2) % 16) * 16));
  // weight scales of step s: 32 bytes per panel, nw / 16 panels per step;
  // wave w loads local bytes 256 w .. + 256 (gate/up: waves 0, 1 the gate
  // run, 2, 3 the up run; down: one run of 1 KB)
  const long srun = GU ? (w < 2 ? (long)nb * 512 + 256 * w : (long)(a.I / 16 + nb * 16) * 32 + 256 * (w - 2))
                       : (long)nb * 1024 + 256 * w;
  const long sstep = (nw / 16) * 32;

  // load d (0..kLoadsPerStep-1) of the batch of step s into stage st:
  // 0-3 A codes, 4-7 B codes, 8 B scales
  auto issue_one = [&](int s, int st, int d) {
    const uint8_t* sb = lds + st * kStage;
    if (d < 4) {
      dma16(a.hilo + s * 128, aoff[d], sb + (4 * w + d) * 1024);
    } else if (d < 8) {
      const int i = d - 4;
      const uint8_t* wb = wexp + gpanel(2 * (4 * w + i)) * wpanel + (s / 2) * 1024 + (s % 2) * 512;
      dma16(wb, boff, sb + kLA + (4 * w + i) * 1024);
    } else {
      dma4(sexp + s * sstep + srun, 4 * lane, sb + kLA + kLB + 256 * w);
    }
  };
  auto issue = [&](int s, int st) {
#pragma unroll
    for (int d = 0; d < kLoadsPerStep; ++d) issue_one(s, st, d);
  };

  // ---- activation scales of the tile's rows, all of K (row r at r * ascs):
  // 256-byte chunks c = w, w + 4, ..., lane l -> dword 64 c + l of the area
  // (pad dwords load the row's first dword).  Issued before the first batch
  // of codes, so the wait for that batch covers them.
  {
    const int ascw = ascs / 4, nch = asc_bytes(K, kPM) / 256;
    for (int c = w; c < nch; c += 4) {
      const int d = 64 * c + lane;
      const int r = min(d / ascw, kPM - 1), q = d % ascw;
      dma4(a.shi, (uint32_t)srow[r] * (uint32_t)(K / 32) + 4 * (q < K / 128 ? q : 0), asc + 256 * c);
    }
  }

  // ---- fragments of this lane.  Wave w takes the 32-row blocks wm and
  // wm + 2 of the tile, so a tile of at most 64 rows leaves every wave at
  // most one live block (the waves then run the one-block loop below)
  const int r32 = lane % 32, h = lane / 32;
  int arow[2];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) arow[mb] = 32 * (2 * mb + wm) + r32;
  const bool two_blocks = 32 * (2 + wm) < rows;
  int bcol[8];
#pragma unroll
  for (int cb = 0; cb < 8; ++cb)
    bcol[cb] = GU ? (cb < 4 ? 0 : 256) + 128 * wn + 32 * (cb % 4) + r32 : 256 * wn + 32 * cb + r32;

  f32x16_t acc[2][8];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int cb = 0; cb < 8; ++cb)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[mb][cb][i] = 0.f;

  // A pieces per row block: the lane's four 16-byte LDS pieces.  Pairs:
  // plane p = pieces 2p, 2p + 1 (k 16h.. and 32 + 16h.. of the row's hi or
  // lo 64 bytes); triples: the lane's 64 bytes of its k-half h, p1 = dwords
  // 0-5, p2 = 6-11, p3 = 12-15.
  constexpr int kPieces = MODE == kTri ? 3 : 2;   // MFMAs per 32 x 32 block and step
  constexpr int kBlockMfma = 8 * kPieces;   // per row block and step
  struct Frags {
    u32x4_t a[2][4];   // [mb][piece]
    int sa[2];         // e8m0 byte of the row block's first piece
    u32x4_t b[8];
    int sb[8];
  };
  // fragment read k of step s from the stage at buf: 0-7 B block k (codes
  // and scale), 8-11 A row block (k - 8) / 2 plane (k - 8) % 2, 12-13 the A
  // scale of row block k - 12
  constexpr int kReads = 14;
  auto read_one = [&](const uint8_t* buf, int s, Frags& f, int k) {
    if (k < 8) {
      const int C = bcol[k];
      f.b[k] = *reinterpret_cast<const u32x4_t*>(buf + kLA + C * 32 + 16 * (h ^ ((C >> 3) & 1)));
      f.sb[k] = buf[kLA + kLB + C * 2 + h];
    } else if (k < 12) {
      // half p of row block mb: pairs plane p (pieces 4p + h, 4p + 2 + h);
      // triples pieces 4h + 2p, 4h + 2p + 1
      const int mb = (k - 8) / 2, p = (k - 8) % 2, R = arow[mb];
      const uint8_t* base = buf + R * 128;
      const int q0 = TRI ? 4 * h + 2 * p : 4 * p + h, q1 = TRI ? q0 + 1 : q0 + 2;
      f.a[mb][2 * p] = *reinterpret_cast<const u32x4_t*>(base + 16 * (q0 ^ (R & 7)));
      f.a[mb][2 * p + 1] = *reinterpret_cast<const u32x4_t*>(base + 16 * (q1 ^ (R & 7)));
    } else {
      f.sa[k - 12] = asc[arow[k - 12] * ascs + 2 * s + h];
    }
  };
  // MFMA j (0 .. kBlockMfma-1) of row block mb: piece j / 8, B block j % 8;
  // piece p's scale byte is sa - 4p (clamped at 0, where the quantiser
  // leaves the piece zero)
  auto mfma_one = [&](const Frags& f, int mb, int j) {
    const int p = j / 8, cb = j % 8;
    const int sa = p == 0 ? f.sa[mb] : (f.sa[mb] >= 4 * p ? f.sa[mb] - 4 * p : 0);
    const u32x4_t x = f.b[cb];
    const i32x8_t b = i32x8_t{(int)x[0], (int)x[1], (int)x[2], (int)x[3], 0, 0, 0, 0};
    const u32x4_t* A = f.a[mb];
    if constexpr (TRI) {
      if (p == 0) {
        const i32x8_t av{(int)A[0][0], (int)A[0][1], (int)A[0][2], (int)A[0][3],
                         (int)A[1][0], (int)A[1][1], 0, 0};
        acc[mb][cb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, b, acc[mb][cb], 2, 4,
                                                                      0, sa, 0, f.sb[cb]);
      } else if (p == 1) {
        const i32x8_t av{(int)A[1][2], (int)A[1][3], (int)A[2][0], (int)A[2][1],
                         (int)A[2][2], (int)A[2][3], 0, 0};
        acc[mb][cb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, b, acc[mb][cb], 2, 4,
                                                                      0, sa, 0, f.sb[cb]);
      } else {
        const i32x8_t av{(int)A[3][0], (int)A[3][1], (int)A[3][2], (int)A[3][3], 0, 0, 0, 0};
        acc[mb][cb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, b, acc[mb][cb], 4, 4,
                                                                      0, sa, 0, f.sb[cb]);
      }
    } else {
      const u32x4_t x0 = A[2 * p], x1 = A[2 * p + 1];
      const i32x8_t av{(int)x0[0], (int)x0[1], (int)x0[2], (int)x0[3],
                       (int)x1[0], (int)x1[1], (int)x1[2], (int)x1[3]};
      acc[mb][cb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, b, acc[mb][cb], 0, 4,
                                                                    0, sa, 0, f.sb[cb]);
    }
  };
  // ---- pipeline (nsteps = K / 64 is even and >= 4): the loads of the
  // first LEAD steps, then step 0's fragments
#pragma unroll
  for (int p = 0; p < LEAD; ++p) issue(p, p);
  __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0((LEAD - 1) * kLoadsPerStep));   // scales, step 0 landed
  __syncthreads();
  // Step s (LIVE row blocks, kBlockMfma LIVE MFMAs): the first half of its
  // MFMAs with the loads of step s + LEAD issued between them (ISSUE), the
  // wait and barrier, then the second half with the fragment reads of step
  // s + 1 between them (NEXT; the order is pinned: no instruction moves
  // across a sched_barrier).  The flags are compile-time, so the
  // steady-state loop has no branch between its MFMAs.  MFMA j: row block
  // j / kBlockMfma, piece (j / 8) % kPieces, B block j % 8.
  auto run = [&](auto live_c) {
    constexpr int LIVE = decltype(live_c)::value;
    constexpr int M = kBlockMfma * LIVE, H2 = M / 2;
    auto mfma_j = [&](const Frags& f, int j) { mfma_one(f, j / kBlockMfma, j % kBlockMfma); };
    // reads this variant needs: B 0-7, A row block 0 (8, 9), its scale (12),
    // and with two blocks A row block 1 (10, 11) and its scale (13)
    auto read_k = [&](int n) { return LIVE == 2 ? n : (n < 10 ? n : 12); };
    constexpr int kR = LIVE == 2 ? kReads : (LIVE == 1 ? 11 : 0);
    auto step = [&](auto issue_c, auto next_c, int s, Frags& cur, Frags& nxt) {
      constexpr bool ISSUE = decltype(issue_c)::value;
      constexpr bool NEXT = decltype(next_c)::value;
      const int sn = s + LEAD, stn = sn % STAGES;
      __builtin_amdgcn_sched_barrier(0);
      int d = 0;
#pragma unroll
      for (int j = 0; j < H2; ++j) {
        mfma_j(cur, j);
        if constexpr (ISSUE) {
          if ((LIVE == 1 || j % 2 == 1) && d < kLoadsPerStep) issue_one(sn, stn, d++);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (ISSUE) {
#pragma unroll
        for (; d < kLoadsPerStep; ++d) issue_one(sn, stn, d);
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (NEXT) {
        // step s + 1 landed: with ISSUE the later LEAD - 1 steps may still
        // be in flight; in the last steps wait for everything
        if constexpr (ISSUE) __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0((LEAD - 1) * kLoadsPerStep));
        else __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(0));
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t* buf = lds + ((s + 1) % STAGES) * kStage;
        int n = 0;
#pragma unroll
        for (int j = H2; j < M; ++j) {
          if (n < kR) read_one(buf, s + 1, nxt, read_k(n++));
          if (LIVE == 1 && n < kR) read_one(buf, s + 1, nxt, read_k(n++));
          mfma_j(cur, j);
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
      step(T_{}, T_{}, s, f0, f1);
      step(T_{}, T_{}, s + 1, f1, f0);
    }
    // the rest (nsteps - s is even): with LEAD 3 and four steps left, the
    // first of them issues the last loads
    if (LEAD == 3 && nsteps - s == 4) {
      step(T_{}, T_{}, s, f0, f1);
      step(F_{}, T_{}, s + 1, f1, f0);
      s += 2;
    }
    step(F_{}, T_{}, s, f0, f1);
    step(F_{}, F_{}, s + 1, f1, f0);
  };
  // a wave whose blocks both lie past the tile (tiles of at most 32 rows,
  // wm = 1) keeps its part of the loads and barriers and computes nothing
  if (two_blocks) run(std::integral_constant<int, 2>{});
  else if (32 * wm < rows) run(std::integral_constant<int, 1>{});
  else run(std::integral_constant<int, 0>{});

  // ---- epilogue.  32x32 result lane layout: column l % 32, rows
  // 8 (i / 4) + 4 (l / 32) + i % 4.
  if constexpr (GU) {
    // Each wave's SwiGLU rows go through its own LDS region (the stages are
    // free once every wave is past the K loop), one value per lane as the
    // MFMA result lies, and are read back as 16-byte row pieces: wide stores
    // of whole row segments instead of one 2-byte store per lane and value.
    __syncthreads();
    constexpr int kAP = 136;   // staged row pitch in bf16 (128 + 8)
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
        for (int cb = 0; cb < 4; ++cb)
          stage[r * kAP + 32 * cb + r32] = f32_to_bf16(
              silu_gate(acc[mb][cb][i], acc[mb][cb + 4][i], a.limit, a.alpha, a.beta));
      }
      __builtin_amdgcn_wave_barrier();
      if (a.qs) {
        // the down pass's operand straight from the staged bf16 rows (the
        // values the act quantiser would read back): 32 rows x 4 blocks of
        // 32 k, two per lane, in the pair / triple row layout
        uint8_t* qo = reinterpret_cast<uint8_t*>(a.out);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int u = 64 * j + lane, rr = u / 4, cb = u % 4;
          if (rb + rr < rows) {
            const long row = row0 + rb + rr;
            const int blk = nb * 8 + wn * 4 + cb;
            const uint16_t* src = stage + rr * kAP + 32 * cb;
            if constexpr (MODE == kPair) {
              uint32_t hw[8], lw[8];
              const int sa = pair_split32(src, hw, lw);
              uint8_t* d = qo + row * 2L * a.I + (blk / 2) * 128 + (blk % 2) * 32;
              *reinterpret_cast<u32x4_t*>(d) = u32x4_t{hw[0], hw[1], hw[2], hw[3]};
              *reinterpret_cast<u32x4_t*>(d + 16) = u32x4_t{hw[4], hw[5], hw[6], hw[7]};
              *reinterpret_cast<u32x4_t*>(d + 64) = u32x4_t{lw[0], lw[1], lw[2], lw[3]};
              *reinterpret_cast<u32x4_t*>(d + 80) = u32x4_t{lw[4], lw[5], lw[6], lw[7]};
              a.qs[row * (a.I / 32) + blk] = (uint8_t)sa;
            } else {
              uint32_t p1[6], p2[6], p3[4];
              const int sc = tri_split32(src, p1, p2, p3);
              uint8_t* d = qo + row * 2L * a.I + (blk / 2) * 128 + (blk % 2) * 64;
              *reinterpret_cast<u32x4_t*>(d) = u32x4_t{p1[0], p1[1], p1[2], p1[3]};
              *reinterpret_cast<u32x4_t*>(d + 16) = u32x4_t{p1[4], p1[5], p2[0], p2[1]};
              *reinterpret_cast<u32x4_t*>(d + 32) = u32x4_t{p2[2], p2[3], p2[4], p2[5]};
              *reinterpret_cast<u32x4_t*>(d + 48) = u32x4_t{p3[0], p3[1], p3[2], p3[3]};
              a.qs[row * (a.I / 32) + blk] = (uint8_t)sc;
            }
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {   // 32 rows x 16 pieces of 8 bf16
          const int q = 64 * j + lane, rr = q / 16, c8 = q % 16;
          if (rb + rr < rows)
            *reinterpret_cast<u32x4_t*>(act + (long)(row0 + rb + rr) * a.I + (long)nb * 256 +
                                        128 * wn + 8 * c8) =
                *reinterpret_cast<const u32x4_t*>(stage + rr * kAP + 8 * c8);
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
  } else {
    // fp32 y: 32 lanes store 128 contiguous bytes of a row per value, and
    // staging these through LDS measured slower (DeepSeek-V3 down, T = 8192)
    float* y = reinterpret_cast<float*>(a.out);
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = 32 * (2 * mb + wm) + 8 * (i / 4) + 4 * h + (i % 4);
        if (r >= rows) continue;
        const long prow = row0 + r;
#pragma unroll
        for (int cb = 0; cb < 8; ++cb)
          y[prow * a.H + (long)nb * 512 + 256 * wn + 32 * cb + r32] = acc[mb][cb][i];
      }
    }
  }
}

// Shapes the kernel takes: gate/up N blocks of 256, down of 512 (so K = H
// and K = I are multiples of 256: an even number of 64-k steps, at least 4),
// LDS for three stages and the activation scales of 128 rows.
bool mx_fits(int H, int I) {
  return H > 0 && I > 0 && I % 256 == 0 && H % 512 == 0 && lds_bytes(3, H) <= kLdsMax &&
         lds_bytes(3, I) <= kLdsMax;
}

// three stages (loads two steps ahead); a fourth stage for the down pass
// (K = 2048 leaves LDS for it) measured no faster at DeepSeek-V3 T = 8192
constexpr int kStages = 3;

template <bool GU, int MODE>
hipError_t launch_k(dim3 g, int K, const MxPairArgs& a, hipStream_t stream) {
  mx_pair_gemm_kernel<GU, MODE, kStages><<<g, kPThreads, lds_bytes(kStages, K), stream>>>(a);
  return hipPeekAtLastError();
}

hipError_t launch(bool gu, int mode, const MxPairArgs& a, int max_tiles, hipStream_t stream) {
  const long items = (long)max_tiles * (gu ? a.I / 256 : a.H / 512);
  const long grid = (items + 7) / 8 * 8;
  if (grid >= (1L << 31)) return hipErrorInvalidValue;
  if (grid == 0) return hipSuccess;
  const dim3 g((unsigned)grid);
  const int K = gu ? a.H : a.I;
  if (gu) {
    if (mode == kTri) return launch_k<true, kTri>(g, K, a, stream);
    if (mode == kDuo) return launch_k<true, kDuo>(g, K, a, stream);
    return launch_k<true, kPair>(g, K, a, stream);
  }
  if (mode == kTri) return launch_k<false, kTri>(g, K, a, stream);
  if (mode == kDuo) return launch_k<false, kDuo>(g, K, a, stream);
  return launch_k<false, kPair>(g, K, a, stream);
}

}  // namespace
}  // namespace xtu

using namespace xtu;

extern "C" {

int xtu_mx_pair_fits(int H, int I) { return mx_fits(H, I) ? 1 : 0; }

int xtu_mx_pair_tile_m(void) { return kPM; }

hipError_t xtu_pair_quant_il(const void* x, int M, int K, uint8_t* hilo, uint8_t* shi,
                             hipStream_t stream) {
  XTU_CHECK_ARG(M >= 0 && K > 0 && K % 128 == 0 && 2L * M * K < (1L << 32));
  XTU_CHECK_ARG(M == 0 || (x && hilo && shi));
  if (M == 0) return hipSuccess;
  (void)hipGetLastError();
  const long n = (long)M * (K / 32);
  mx_pair_quant_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(
      (const uint16_t*)x, M, K, hilo, shi);
  return hipPeekAtLastError();
}

hipError_t xtu_mx_pair_scales(const uint8_t* s, int E, int N, int K, long s_estride, uint8_t* out,
                              hipStream_t stream) {
  XTU_CHECK_ARG(E >= 0 && N > 0 && N % 16 == 0 && K > 0 && K % 128 == 0);
  XTU_CHECK_ARG(s_estride >= WFmt<kMXFP4>::s_bytes(N, K) && (long)E * N * (K / 32) < (1L << 40));
  XTU_CHECK_ARG(E == 0 || (s && out));
  if (E == 0) return hipSuccess;
  (void)hipGetLastError();
  const long n = (long)E * N * (K / 32);
  mx_pair_scales_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(s, E, N, K, s_estride,
                                                                          out);
  return hipPeekAtLastError();
}

static hipError_t gate_up(int mode, const uint8_t* hilo, const uint8_t* shi,
                          const int32_t* sorted_tok, int H, int I, const void* w13,
                          const uint8_t* s13p, long w_estride, long s_estride,
                          const int32_t* slot_map, const int32_t* seg_start,
                          const int32_t* tile_expert, const int32_t* tile_row0,
                          const int32_t* expert_tile_start, const int32_t* tile_lo,
                          const int32_t* tile_hi, int max_tiles, void* act, float limit,
                          float alpha, float beta, hipStream_t stream,
                          uint8_t* act_scales = nullptr) {
  XTU_CHECK_ARG(mx_fits(H, I));
  XTU_CHECK_ARG(max_tiles >= 0 && max_tiles < (1 << 30) && w_estride >= 0 && s_estride >= 0);
  XTU_CHECK_ARG(w_estride < (1L << 31) && 2L * I * H < (1L << 32));
  XTU_CHECK_ARG(hilo && shi && sorted_tok && w13 && s13p && seg_start && tile_expert &&
                tile_row0 && expert_tile_start && tile_lo && tile_hi && act);
  if (max_tiles == 0) return hipSuccess;
  (void)hipGetLastError();
  const MxPairArgs a{hilo, shi, sorted_tok, (const uint8_t*)w13, s13p, seg_start, tile_expert,
                     tile_row0, expert_tile_start, tile_lo, tile_hi, slot_map, act, H, I,
                     w_estride, s_estride, limit, alpha, beta, act_scales};
  return launch(true, mode, a, max_tiles, stream);
}

static hipError_t down(int mode, const uint8_t* hilo, const uint8_t* shi, int H, int I,
                       const void* w2, const uint8_t* s2p, long w_estride, long s_estride,
                       const int32_t* slot_map, const int32_t* seg_start,
                       const int32_t* tile_expert, const int32_t* tile_row0,
                       const int32_t* expert_tile_start, const int32_t* tile_lo,
                       const int32_t* tile_hi, int max_tiles, float* y, hipStream_t stream) {
  XTU_CHECK_ARG(mx_fits(H, I));
  XTU_CHECK_ARG(max_tiles >= 0 && max_tiles < (1 << 30) && w_estride >= 0 && s_estride >= 0);
  XTU_CHECK_ARG(w_estride < (1L << 31) && (long)H * I < (1L << 31));
  XTU_CHECK_ARG(hilo && shi && w2 && s2p && seg_start && tile_expert && tile_row0 &&
                expert_tile_start && tile_lo && tile_hi && y);
  if (max_tiles == 0) return hipSuccess;
  (void)hipGetLastError();
  const MxPairArgs a{hilo, shi, nullptr, (const uint8_t*)w2, s2p, seg_start, tile_expert,
                     tile_row0, expert_tile_start, tile_lo, tile_hi, slot_map, y, H, I,
                     w_estride, s_estride, 0.f, 1.f, 0.f, nullptr};
  return launch(false, mode, a, max_tiles, stream);
}

hipError_t xtu_mx_pair_gate_up(const uint8_t* hilo, const uint8_t* shi, const int32_t* sorted_tok,
                               int H, int I, const void* w13, const uint8_t* s13p,
                               long w_estride, long s_estride, const int32_t* slot_map,
                               const int32_t* seg_start, const int32_t* tile_expert,
                               const int32_t* tile_row0, const int32_t* expert_tile_start,
                               const int32_t* tile_lo, const int32_t* tile_hi, int max_tiles,
                               void* act, float limit, float alpha, float beta,
                               hipStream_t stream) {
  return gate_up(kPair, hilo, shi, sorted_tok, H, I, w13, s13p, w_estride, s_estride, slot_map,
                 seg_start, tile_expert, tile_row0, expert_tile_start, tile_lo, tile_hi,
                 max_tiles, act, limit, alpha, beta, stream);
}

hipError_t xtu_mx_pair_down(const uint8_t* hilo, const uint8_t* shi, int H, int I, const void* w2,
                            const uint8_t* s2p, long w_estride, long s_estride,
                            const int32_t* slot_map, const int32_t* seg_start,
                            const int32_t* tile_expert, const int32_t* tile_row0,
                            const int32_t* expert_tile_start, const int32_t* tile_lo,
                            const int32_t* tile_hi, int max_tiles, float* y, hipStream_t stream) {
  return down(kPair, hilo, shi, H, I, w2, s2p, w_estride, s_estride, slot_map, seg_start,
              tile_expert, tile_row0, expert_tile_start, tile_lo, tile_hi, max_tiles, y, stream);
}

hipError_t xtu_tri_quant_il(const void* x, int M, int K, uint8_t* q, uint8_t* sq,
                            hipStream_t stream) {
  XTU_CHECK_ARG(M >= 0 && K > 0 && K % 128 == 0 && 2L * M * K < (1L << 32));
  XTU_CHECK_ARG(M == 0 || (x && q && sq));
  if (M == 0) return hipSuccess;
  (void)hipGetLastError();
  const long n = (long)M * (K / 32);
  mx_tri_quant_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>((const uint16_t*)x, M, K,
                                                                        q, sq);
  return hipPeekAtLastError();
}

hipError_t xtu_mx_tri_gate_up(const uint8_t* q, const uint8_t* sq, const int32_t* sorted_tok,
                              int H, int I, const void* w13, const uint8_t* s13p, long w_estride,
                              long s_estride, const int32_t* slot_map, const int32_t* seg_start,
                              const int32_t* tile_expert, const int32_t* tile_row0,
                              const int32_t* expert_tile_start, const int32_t* tile_lo,
                              const int32_t* tile_hi, int max_tiles, void* act, float limit,
                              float alpha, float beta, hipStream_t stream) {
  return gate_up(kTri, q, sq, sorted_tok, H, I, w13, s13p, w_estride, s_estride, slot_map,
                 seg_start, tile_expert, tile_row0, expert_tile_start, tile_lo, tile_hi,
                 max_tiles, act, limit, alpha, beta, stream);
}

hipError_t xtu_mx_tri_down(const uint8_t* q, const uint8_t* sq, int H, int I, const void* w2,
                           const uint8_t* s2p, long w_estride, long s_estride,
                           const int32_t* slot_map, const int32_t* seg_start,
                           const int32_t* tile_expert, const int32_t* tile_row0,
                           const int32_t* expert_tile_start, const int32_t* tile_lo,
                           const int32_t* tile_hi, int max_tiles, float* y, hipStream_t stream) {
  return down(kTri, q, sq, H, I, w2, s2p, w_estride, s_estride, slot_map, seg_start, tile_expert,
              tile_row0, expert_tile_start, tile_lo, tile_hi, max_tiles, y, stream);
}

hipError_t xtu_mx_duo_gate_up(const uint8_t* q, const uint8_t* sq, const int32_t* sorted_tok,
                              int H, int I, const void* w13, const uint8_t* s13p, long w_estride,
                              long s_estride, const int32_t* slot_map, const int32_t* seg_start,
                              const int32_t* tile_expert, const int32_t* tile_row0,
                              const int32_t* expert_tile_start, const int32_t* tile_lo,
                              const int32_t* tile_hi, int max_tiles, void* act, float limit,
                              float alpha, float beta, hipStream_t stream) {
  return gate_up(kDuo, q, sq, sorted_tok, H, I, w13, s13p, w_estride, s_estride, slot_map,
                 seg_start, tile_expert, tile_row0, expert_tile_start, tile_lo, tile_hi,
                 max_tiles, act, limit, alpha, beta, stream);
}

hipError_t xtu_mx_gate_up_q(int mode, const uint8_t* q, const uint8_t* sq,
                            const int32_t* sorted_tok, int H, int I, const void* w13,
                            const uint8_t* s13p, long w_estride, long s_estride,
                            const int32_t* slot_map, const int32_t* seg_start,
                            const int32_t* tile_expert, const int32_t* tile_row0,
                            const int32_t* expert_tile_start, const int32_t* tile_lo,
                            const int32_t* tile_hi, int max_tiles, uint8_t* act_q,
                            uint8_t* act_sq, float limit, float alpha, float beta,
                            hipStream_t stream) {
  XTU_CHECK_ARG(mode == kPair || mode == kTri || mode == kDuo);
  XTU_CHECK_ARG(act_q && act_sq);
  return gate_up(mode, q, sq, sorted_tok, H, I, w13, s13p, w_estride, s_estride, slot_map,
                 seg_start, tile_expert, tile_row0, expert_tile_start, tile_lo, tile_hi,
                 max_tiles, act_q, limit, alpha, beta, stream, act_sq);
}

hipError_t xtu_mx_duo_down(const uint8_t* q, const uint8_t* sq, int H, int I, const void* w2,
                           const uint8_t* s2p, long w_estride, long s_estride,
                           const int32_t* slot_map, const int32_t* seg_start,
                           const int32_t* tile_expert, const int32_t* tile_row0,
                           const int32_t* expert_tile_start, const int32_t* tile_lo,
                           const int32_t* tile_hi, int max_tiles, float* y, hipStream_t stream) {
  return down(kDuo, q, sq, H, I, w2, s2p, w_estride, s_estride, slot_map, seg_start, tile_expert,
              tile_row0, expert_tile_start, tile_lo, tile_hi, max_tiles, y, stream);
}

}  // extern "C"
