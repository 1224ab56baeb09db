// INT8-activation x FP4-code expert path (ALIGN rule), exact int32 accumulation.
//
//   activation row a (fp32 of bf16): m = max|a|, crow = ceil(log2(m/127)) from
//     the exponent field, a8 = clamp(rne(a * 2^-crow), +-127)
//   weight row n of MXFP4: w4 = 2*e2m1 in {0,+-1,+-2,+-3,+-4,+-6,+-8,+-12},
//     emin_n = min over the row's e8m0 bytes b, w8' = w4 << (b - emin_n)
//     (requires b - emin_n <= 3 so |w8'| <= 96 fits int8)
//   ACC = sum_k a8 * w8'  (int32, exact; |ACC| <= 127*96*K)
//   C   = float(ACC) * 2^(emin_n - 128 + crow)
//
// A weight row whose e8m0 spread exceeds 3 cannot take the integer path (the
// reference routes such tiles to its fp32 path, moe_v2_packed4_w4a8.inc:
// 1344-1366).  xtu_i8_prepare marks it (emin byte 0xFF, int8 weights 0); the
// integer GEMMs leave its output column unwritten -- for gate/up the column
// pair n of act when gate row n or up row n is marked -- and the fallback
// kernels compute exactly those columns in fp32 from the MXFP4 weights and
// the bf16 activations (the fp32 path's operands).
//
// The shifted int8 weights are expanded once per layer (xtu_i8_prepare) into
// the P16 panel layout with 16 int8 per chunk, next to a per-row emin; the
// GEMM then runs v_mfma_i32_32x32x32_i8 on LDS tiles with the same tile list
// and epilogues as the bf16 grouped GEMM.
#include <type_traits>

#include "weight_format.hpp"

namespace xtu {
namespace {

constexpr int kBK = 128;   // k per step (64 measured 6% slower: twice the barriers)
constexpr int kI8Marked = 0xFF;   // emin of a row that takes the fp32 fallback
constexpr int kBN = 256;
constexpr int kLDB = kBK + 16;   // LDS pitch in bytes

__device__ __forceinline__ int w4_of(uint32_t nib) {
  const int m = nib & 7;
  const int mag = m < 4 ? m : ((4 + (m & 1) * 2) << ((m >> 1) & 1));
  return (nib & 8) ? -mag : mag;
}

// per row n: emin = min over its K/32 e8m0 scale bytes (packed scale groups)
__global__ __launch_bounds__(256) void i8_emin_kernel(const uint8_t* __restrict__ s, int N, int K,
                                                      long s_estride, uint8_t* __restrict__ emin,
                                                      int32_t* __restrict__ dmax) {
  const int e = blockIdx.y;
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  const int p = n / 16, r = n % 16;
  const long nsbk = K / 128;
  const uint8_t* se = s + (long)e * s_estride;
  int mn = 255, mx = 0;
  for (long sb = 0; sb < nsbk; ++sb)
    for (int q = 0; q < 4; ++q) {
      const int b = se[scale_offset<kMXFP4>(p, sb, q * 16 + r, K)];
      mn = min(mn, b);
      mx = max(mx, b);
    }
  // a row the integer path cannot hold (spread > 3) is marked with 0xFF
  emin[(long)e * N + n] = (uint8_t)(mx - mn > 3 ? kI8Marked : mn);
  atomicMax(dmax, mx - mn);
}

// one thread per fp4 chunk: 32 codes -> 32 int8 w8' in two int8 chunks
__global__ __launch_bounds__(256) void i8_expand_kernel(const uint8_t* __restrict__ w,
                                                        const uint8_t* __restrict__ s, int N, int K,
                                                        long w_estride, long s_estride,
                                                        const uint8_t* __restrict__ emin,
                                                        uint8_t* __restrict__ w8, long w8_estride) {
  const int e = blockIdx.y;
  const long c = (long)blockIdx.x * 256 + threadIdx.x;   // chunk index inside the expert
  const long nchunks = (long)N * K / 32;
  if (c >= nchunks) return;
  const long nsb4 = K / 128, nsb8 = K / 64;
  // fp4 layout: [p][sb4][q4][r] chunks
  const long p = c / (nsb4 * 64);
  const long rem = c % (nsb4 * 64);
  const long sb4 = rem / 64;
  const int q4 = (int)(rem % 64) / 16, r = (int)(rem % 16);
  const int n = (int)(p * 16 + r);
  const u32x4_t raw = *reinterpret_cast<const u32x4_t*>(w + (long)e * w_estride + c * 16);
  const int b = s[(long)e * s_estride + scale_offset<kMXFP4>(p, sb4, q4 * 16 + r, K)];
  const int em = emin[(long)e * N + n];
  const int d = em == kI8Marked ? 0 : b - em;
  const bool zero = em == kI8Marked;   // marked row: int8 weights 0
  const int k0 = (int)(sb4 * 128 + q4 * 32);
  uint32_t outw[8];
#pragma unroll
  for (int dw = 0; dw < 4; ++dw) {
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int bb = 0; bb < 4; ++bb) {
      const uint32_t byte = (raw[dw] >> (8 * bb)) & 0xffu;
      const uint32_t v0 = zero ? 0u : (uint32_t)(w4_of(byte & 15u) * (1 << d)) & 0xffu;
      const uint32_t v1 = zero ? 0u : (uint32_t)(w4_of(byte >> 4) * (1 << d)) & 0xffu;
      const int j = bb * 2;   // k offset inside this dword's 8 values
      if (j < 4) lo |= (v0 << (8 * j)) | (v1 << (8 * (j + 1)));
      else hi |= (v0 << (8 * (j - 4))) | (v1 << (8 * (j - 3)));
    }
    outw[dw * 2] = lo;
    outw[dw * 2 + 1] = hi;
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int kk = k0 + 16 * h;
    const long sb8 = kk / 64;
    const int q8 = (kk % 64) / 16;
    uint8_t* dst = w8 + (long)e * w8_estride + ((p * nsb8 + sb8) * 1024) + (q8 * 16 + r) * 16;
    u32x4_t v = {outw[4 * h], outw[4 * h + 1], outw[4 * h + 2], outw[4 * h + 3]};
    *reinterpret_cast<u32x4_t*>(dst) = v;
  }
}

// one wave per row: crow and a8 of a bf16 row of length K (K % 512 == 0 not
// required; K % 8 == 0)
__global__ __launch_bounds__(256) void i8_quant_rows_kernel(const uint16_t* __restrict__ src,
                                                            int M, int K, int8_t* __restrict__ a8,
                                                            int32_t* __restrict__ crow) {
  const int row = blockIdx.x * 4 + threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  if (row >= M) return;
  const uint16_t* s = src + (long)row * K;
  float m = 0.f;
  for (int k = lane * 8; k < K; k += 512) {
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(s + k);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      m = fmaxf(m, fabsf(__uint_as_float(v[i] << 16)));
      m = fmaxf(m, fabsf(__uint_as_float(v[i] & 0xffff0000u)));
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  int c = 0;
  if (m > 0.f) {
    const uint32_t b = __float_as_uint(m);
    const int ef = (int)((b >> 23) & 0xffu);
    if (ef == 0xff) c = 120;
    else if (ef == 0) c = -120;
    else c = (ef - 127) - 6 + (((b & 0x7fffffu) > 8257536u) ? 1 : 0);
    c = max(-120, min(120, c));
  }
  const float inv = __uint_as_float((uint32_t)(127 - c) << 23);
  for (int k = lane * 8; k < K; k += 512) {
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(s + k);
    uint32_t packed[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float f0 = __uint_as_float(v[i] << 16), f1 = __uint_as_float(v[i] & 0xffff0000u);
      const int q0 = (int)fminf(fmaxf(__builtin_rintf(f0 * inv), -127.f), 127.f);
      const int q1 = (int)fminf(fmaxf(__builtin_rintf(f1 * inv), -127.f), 127.f);
      const uint32_t pr = ((uint32_t)q0 & 0xffu) | (((uint32_t)q1 & 0xffu) << 8);
      packed[i / 2] |= pr << (16 * (i % 2));
    }
    *reinterpret_cast<uint2*>(a8 + (long)row * K + k) = make_uint2(packed[0], packed[1]);
  }
  if (lane == 0) crow[row] = c;
}

struct I8GemmArgs {
  const int8_t* a;            // gate/up: a8 of hidden rows [T][K]; down: a8 of act rows [A][K]
  const int32_t* crow;        // per A row (token for gate/up, pair row for down)
  const int32_t* sorted_tok;
  const uint8_t* w8;          // expanded weights (P16, 16 int8 per chunk)
  const uint8_t* emin;        // [E][N]
  const int32_t* seg_start;
  const int32_t* tile_expert;
  const int32_t* tile_row0;
  const int32_t* tile_lo;     // m-tile range [*tile_lo, *tile_hi) of the tile list
  const int32_t* tile_hi;
  const int32_t* slot_map;    // expert -> weight slot (null: identity)
  void* out;
  int32_t* acc_out;           // optional raw int32 accumulators [A][N] (tests)
  int H, I;
  long w_estride;
  float limit, alpha, beta;
};

// Two waves per SIMD (at most 256 registers; 272 unbounded, one wave per
// SIMD): measured 32% faster on Qwen3-Next T = 8192 (gate/up 851 -> 577 us).
template <int BM, bool GU>
__global__ __launch_bounds__(256, 2) void i8_gemm_kernel(I8GemmArgs a) {
  constexpr int MT = BM / 32;
  constexpr int A_CH = BM * kBK / 16 / 256;   // 16-byte A chunks per thread
  constexpr int CPP = (kBK / 16) * 16;        // B chunks per panel per K step
  constexpr int B_CH = 16 * CPP / 256;
  __shared__ __attribute__((aligned(16))) int8_t As[BM * kLDB];
  __shared__ __attribute__((aligned(16))) int8_t Bs[kBN * kLDB];

  // work item (M tile, N block), N block fastest, dealt to the eight XCDs in
  // contiguous ranges (workgroup i runs on XCD i % 8): the workgroups
  // resident on one XCD share a tile's rows and an expert's weights in L2
  const int nbn = GU ? a.I / 128 : a.H / 256;
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
  const int rows = min(BM, a.seg_start[e + 1] - row0);
  const int K = GU ? a.H : a.I;
  const int N = GU ? 2 * a.I : a.H;
  const int tid = threadIdx.x, w = tid / 64, lane = tid % 64;
  const long nsbk = K / 64;
  const uint8_t* wexp = a.w8 + (long)ws * a.w_estride;

  const int8_t* asrc[A_CH];
#pragma unroll
  for (int i = 0; i < A_CH; ++i) {
    const int c = i * 256 + tid, r = c / (kBK / 16);
    if (r < rows) {
      const long src = GU ? (long)a.sorted_tok[row0 + r] : (long)(row0 + r);
      asrc[i] = a.a + src * K + (c % (kBK / 16)) * 16;
    } else {
      asrc[i] = nullptr;
    }
  }
  long bpanel[B_CH];
  int boff[B_CH];
#pragma unroll
  for (int i = 0; i < B_CH; ++i) {
    const int c = i * 256 + tid, pl = c / CPP;
    boff[i] = c % CPP;
    if (GU) bpanel[i] = pl < 8 ? (long)nb * 8 + pl : (long)(a.I / 16) + nb * 8 + (pl - 8);
    else bpanel[i] = (long)nb * 16 + pl;
  }
  u32x4_t areg[A_CH], breg[B_CH];
  auto gload = [&](int kk) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      u32x4_t v = {0u, 0u, 0u, 0u};
      if (asrc[i]) v = *reinterpret_cast<const u32x4_t*>(asrc[i] + kk);
      areg[i] = v;
    }
    const long sb = kk / 64;
#pragma unroll
    for (int i = 0; i < B_CH; ++i)
      breg[i] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4_t*>(wexp + (bpanel[i] * nsbk + sb) * 1024 + boff[i] * 16));
  };
  auto lstore = [&]() {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int c = i * 256 + tid;
      const int r = c / (kBK / 16), col = c % (kBK / 16);
      *reinterpret_cast<u32x4_t*>(&As[r * kLDB + col * 16]) = areg[i];
    }
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      const int c = i * 256 + tid, pl = c / CPP;
      const int r = boff[i] % 16, qr = boff[i] / 16;
      *reinterpret_cast<u32x4_t*>(&Bs[(pl * 16 + r) * kLDB + qr * 16]) = breg[i];
    }
  };
  const int jt0 = GU ? 32 * w : 64 * w;
  const int jt1 = GU ? 128 + 32 * w : 64 * w + 32;
  // K loop and epilogue for NT 32-row tiles (the tile's rows rounded up):
  // a partial tile does no MFMAs for rows it does not hold
  auto run = [&](auto nt_tag) {
    constexpr int NT = decltype(nt_tag)::value;
    i32x16_t acc[NT][2];
#pragma unroll
    for (int m = 0; m < NT; ++m)
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[m][n][i] = 0;

    // single LDS stage (a double-buffered one, one barrier per step, measured
    // 8% slower): the next step's loads are in flight during the MFMAs
    const int nk = K / kBK;
    gload(0);
    for (int kt = 0; kt < nk; ++kt) {
      __syncthreads();
      lstore();
      __syncthreads();
      if (kt + 1 < nk) gload((kt + 1) * kBK);
#pragma unroll
      for (int ks = 0; ks < kBK / 32; ++ks) {
        const int kofs = ks * 32 + (lane / 32) * 16;
        const i32x4_t b0 =
            *reinterpret_cast<const i32x4_t*>(&Bs[(jt0 + lane % 32) * kLDB + kofs]);
        const i32x4_t b1 =
            *reinterpret_cast<const i32x4_t*>(&Bs[(jt1 + lane % 32) * kLDB + kofs]);
#pragma unroll
        for (int m = 0; m < NT; ++m) {
          const i32x4_t av =
              *reinterpret_cast<const i32x4_t*>(&As[(m * 32 + lane % 32) * kLDB + kofs]);
          acc[m][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, b0, acc[m][0], 0, 0, 0);
          acc[m][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, b1, acc[m][1], 0, 0, 0);
        }
      }
    }
    const int ncol = lane % 32;
    long gcol0, gcol1;   // global weight rows of the two column tiles
    if (GU) {
      gcol0 = (long)nb * 128 + 32 * w + ncol;
      gcol1 = (long)a.I + nb * 128 + 32 * w + ncol;
    } else {
      gcol0 = (long)nb * 256 + jt0 + ncol;
      gcol1 = (long)nb * 256 + jt1 + ncol;
    }
    const int em0 = a.emin[(long)ws * N + gcol0];
    const int em1 = a.emin[(long)ws * N + gcol1];
    if constexpr (GU) {
      if (!a.acc_out) {
        // act rows through LDS as for y below: the wave's 32 act columns of
        // each row tile (bf16), read back as 16-byte pieces (8 columns), two
        // wide stores per lane and row tile instead of sixteen 2-byte ones.
        // A column pair with a marked row gets a value (from zero int8
        // weights); the fp32 fallback that follows overwrites it.
        constexpr int kAP = 40;   // LDS row pitch in bf16 (32 + 8)
        uint16_t* stage = reinterpret_cast<uint16_t*>(Bs) + w * (32 * kAP);
        __syncthreads();   // every wave is done with the K loop's LDS tiles
        uint16_t* act = reinterpret_cast<uint16_t*>(a.out);
#pragma unroll
        for (int m = 0; m < NT; ++m) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int r = (i / 4) * 8 + (lane / 32) * 4 + (i % 4);
            const int cr = m * 32 + r < rows ? a.crow[a.sorted_tok[row0 + m * 32 + r]] : 0;
            const float c0 = (float)acc[m][0][i] * ldexpf(1.0f, em0 - 128 + cr);
            const float c1 = (float)acc[m][1][i] * ldexpf(1.0f, em1 - 128 + cr);
            stage[r * kAP + ncol] = f32_to_bf16(silu_gate(c0, c1, a.limit, a.alpha, a.beta));
          }
          __builtin_amdgcn_wave_barrier();
          const int r = lane / 4, c8 = lane % 4;   // 16 rows x 4 pieces per pass
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int rr = r + 16 * j;
            if (m * 32 + rr < rows) {
              const u32x4_t v = *reinterpret_cast<const u32x4_t*>(&stage[rr * kAP + 8 * c8]);
              *reinterpret_cast<u32x4_t*>(
                  &act[(long)(row0 + m * 32 + rr) * a.I + (long)nb * 128 + 32 * w + 8 * c8]) = v;
            }
          }
          __builtin_amdgcn_wave_barrier();
        }
        return;
      }
    }
    if constexpr (!GU) {
      if (!a.acc_out) {
        // y rows through LDS: the wave's 32 x 64 block of each row tile is
        // written to its own LDS region (one fp32 per lane and value, as the
        // MFMA result lies), then read back as 16-byte row pieces, so each
        // lane issues 8 wide stores per row tile instead of 32 scalar ones.
        // A marked column's value (its int8 weights are zero) is written
        // too; the fp32 fallback that follows overwrites it.
        constexpr int kYP = 68;   // LDS row pitch in floats (64 + 4 against bank conflicts)
        float* stage = reinterpret_cast<float*>(Bs) + w * (32 * kYP);
        __syncthreads();   // every wave is done with the K loop's LDS tiles
        float* y = reinterpret_cast<float*>(a.out);
#pragma unroll
        for (int m = 0; m < NT; ++m) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int r = (i / 4) * 8 + (lane / 32) * 4 + (i % 4);
            const int cr = m * 32 + r < rows ? a.crow[row0 + m * 32 + r] : 0;
            stage[r * kYP + ncol] = (float)acc[m][0][i] * ldexpf(1.0f, em0 - 128 + cr);
            stage[r * kYP + 32 + ncol] = (float)acc[m][1][i] * ldexpf(1.0f, em1 - 128 + cr);
          }
          __builtin_amdgcn_wave_barrier();
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int q = j * 64 + lane, r = q / 16, c4 = q % 16;
            if (m * 32 + r < rows) {
              const f32x4_t v = *reinterpret_cast<const f32x4_t*>(&stage[r * kYP + 4 * c4]);
              *reinterpret_cast<f32x4_t*>(
                  &y[(long)(row0 + m * 32 + r) * a.H + (long)nb * 256 + 64 * w + 4 * c4]) = v;
            }
          }
          __builtin_amdgcn_wave_barrier();
        }
        return;
      }
    }
#pragma unroll
    for (int m = 0; m < NT; ++m)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = m * 32 + (i / 4) * 8 + (lane / 32) * 4 + (i % 4);
        if (r < rows) {
          const long prow = row0 + r;
          const int cr = a.crow[GU ? (long)a.sorted_tok[prow] : prow];
          const float sc0 = ldexpf(1.0f, em0 - 128 + cr);
          const float sc1 = ldexpf(1.0f, em1 - 128 + cr);
          const float c0 = (float)acc[m][0][i] * sc0;
          const float c1 = (float)acc[m][1][i] * sc1;
          if (a.acc_out) {
            a.acc_out[prow * N + gcol0] = acc[m][0][i];
            a.acc_out[prow * N + gcol1] = acc[m][1][i];
          }
          // marked rows' columns are the fallback kernels' to write
          if (GU) {
            uint16_t* act = reinterpret_cast<uint16_t*>(a.out);
            if (em0 != kI8Marked && em1 != kI8Marked)
              act[prow * a.I + gcol0] = f32_to_bf16(silu_gate(c0, c1, a.limit, a.alpha, a.beta));
          } else {
            float* y = reinterpret_cast<float*>(a.out);
            if (em0 != kI8Marked) y[prow * a.H + gcol0] = c0;
            if (em1 != kI8Marked) y[prow * a.H + gcol1] = c1;
          }
        }
      }
  };
  if (rows > 96) run(std::integral_constant<int, MT>{});
  else if (rows > 64) run(std::integral_constant<int, 3>{});
  else if (rows > 32) run(std::integral_constant<int, 2>{});
  else run(std::integral_constant<int, 1>{});
}

// fp32 value of MXFP4 weight (row n, k) of one expert matrix [N][K] (P16)
__device__ __forceinline__ float mxfp4_at(const uint8_t* w, const uint8_t* s, int n, int k,
                                          int K) {
  const long p = n / 16, r = n % 16, sb = k / 128, q = (k % 128) / 32, j = k % 32;
  const long nsb = K / 128;
  const uint8_t byte = w[(((p * nsb + sb) * 4 + q) * 16 + r) * 16 + j / 2];
  const int nib = (j & 1) ? (byte >> 4) : (byte & 15);
  const int b = s[scale_offset<kMXFP4>(p, sb, (int)(q * 16 + r), K)];
  return ldexpf(0.5f * (float)w4_of((uint32_t)nib), b - 127);   // e2m1 = w4 / 2, exact
}

struct I8FallbackArgs {
  const uint16_t* x;          // gate/up: hidden rows [T][H]; down: act rows [A][I] (bf16)
  const int32_t* sorted_tok;  // gate/up only
  const uint8_t* w;           // MXFP4 P16 codes (expert-major)
  const uint8_t* s;           // packed e8m0 scale groups
  const int32_t* seg_start;
  const int32_t* tile_expert;
  const int32_t* tile_row0;
  const int32_t* tile_lo;
  const int32_t* tile_hi;
  const int32_t* slot_map;
  const int32_t* col_start;   // [n_slots + 1] CSR of marked columns per weight slot
  const int32_t* cols;        // gate/up: column pair n in [0, I); down: column h
  void* out;                  // act bf16 [A][I] / y fp32 [A][H]
  int H, I, bm;
  float limit, alpha, beta;
};

// One workgroup per m tile of the tile list; for each marked column of the
// tile's weight slot, the marked weight row(s) are dequantised to fp32 in LDS
// and every row of the tile takes its dot product with them: one wave per
// row, lanes over k, reduced across the wave in a fixed order.
template <bool GU>
__global__ __launch_bounds__(256) void i8_fallback_kernel(I8FallbackArgs a) {
  constexpr int kChunk = 2048;   // k per LDS fill
  __shared__ float wl[2][kChunk];
  const int tile = a.tile_lo[0] + blockIdx.x;
  if (tile >= a.tile_hi[0]) return;
  const int e = a.tile_expert[tile];
  const int ws = a.slot_map ? a.slot_map[e] : e;
  const int c0 = a.col_start[ws], c1 = a.col_start[ws + 1];
  if (c0 == c1) return;
  const int row0 = a.tile_row0[tile];
  const int rows = min(a.bm, a.seg_start[e + 1] - row0);
  const int K = GU ? a.H : a.I;
  const int N = GU ? 2 * a.I : a.H;
  const long w_es = WFmt<kMXFP4>::w_bytes(N, K), s_es = WFmt<kMXFP4>::s_bytes(N, K);
  const uint8_t* we = a.w + (long)ws * w_es;
  const uint8_t* se = a.s + (long)ws * s_es;
  const int w = threadIdx.x / 64, lane = threadIdx.x % 64;
  for (int ci = c0; ci < c1; ++ci) {
    const int col = a.cols[ci];
    const int nr0 = col, nr1 = GU ? a.I + col : col;   // weight rows (gate, up) or (h)
    // each wave owns rows w, w+4, ...: at most bm/4 partial sums per lane pair
    float accg[32], accu[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) accg[i] = accu[i] = 0.f;
    for (int k0 = 0; k0 < K; k0 += kChunk) {
      const int kn = min(kChunk, K - k0);
      __syncthreads();
      for (int k = threadIdx.x; k < kn; k += 256) {
        wl[0][k] = mxfp4_at(we, se, nr0, k0 + k, K);
        if (GU) wl[1][k] = mxfp4_at(we, se, nr1, k0 + k, K);
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const int r = w + 4 * i;
        if (r < rows) {
          const long src = GU ? (long)a.sorted_tok[row0 + r] : (long)(row0 + r);
          const uint16_t* xr = a.x + src * K + k0;
          float g = 0.f, u = 0.f;
          for (int k = lane; k < kn; k += 64) {
            const float xv = __uint_as_float((uint32_t)xr[k] << 16);
            g = __builtin_fmaf(xv, wl[0][k], g);
            if (GU) u = __builtin_fmaf(xv, wl[1][k], u);
          }
          accg[i] += g;
          accu[i] += u;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const int r = w + 4 * i;
      float g = accg[i], u = accu[i];
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        g += __shfl_xor(g, off, 64);
        if (GU) u += __shfl_xor(u, off, 64);
      }
      if (lane == 0 && r < rows) {
        const long prow = row0 + r;
        if (GU)
          reinterpret_cast<uint16_t*>(a.out)[prow * a.I + col] =
              f32_to_bf16(silu_gate(g, u, a.limit, a.alpha, a.beta));
        else
          reinterpret_cast<float*>(a.out)[prow * a.H + col] = g;
      }
    }
  }
}

// per expert: the smallest e8m0 byte of its [N][K] matrix (every row and
// k group, the P16 scale groups' padding excluded), written to eminmin[e]
__global__ __launch_bounds__(256) void i8_emin_min_kernel(const uint8_t* __restrict__ s, int N,
                                                          int K, long s_estride,
                                                          int32_t* __restrict__ eminmin) {
  __shared__ int red[256];
  const int e = blockIdx.x;
  const uint8_t* se = s + (long)e * s_estride;
  const long nsbk = K / 128;
  const long units = (long)N * nsbk * 4;   // (row, super-block, chunk) scale bytes
  int mn = 255;
  for (long u = threadIdx.x; u < units; u += 256) {
    const int n = (int)(u / (nsbk * 4));
    const long rem = u % (nsbk * 4);
    const int q = (int)(rem % 4);
    const long sb = rem / 4;
    mn = min(mn, (int)se[scale_offset<kMXFP4>(n / 16, sb, q * 16 + n % 16, K)]);
  }
  red[threadIdx.x] = mn;
  __syncthreads();
  for (int off = 128; off >= 1; off >>= 1) {
    if (threadIdx.x < off) red[threadIdx.x] = min(red[threadIdx.x], red[threadIdx.x + off]);
    __syncthreads();
  }
  if (threadIdx.x == 0) eminmin[e] = red[0];
}

// The engine's offset guard (moe_v2_packed4_w4a8.inc:436, :1361-1364): an
// integer tile whose activation exponent plus weight exponent falls below
// 2^-24 (crow + emin - 128 < -24) is computed on the fp32 path.  Restated
// per row: a sorted row whose activation row exponent (crow of its token
// for gate/up, of its act row for down) plus its expert's smallest e8m0
// byte, minus 128, is below -24 is recomputed whole in fp32 here, after the
// integer GEMM wrote it: every output column of the row, from the bf16
// activations and the exactly dequantised MXFP4 weights (the operands of the
// engine's fp32 path).  One workgroup per m tile; the activation row is
// staged in LDS as fp32 in chunks; each thread owns output columns and sums
// over k in order (deterministic).
struct I8RowFallbackArgs {
  const uint16_t* x;          // gate/up: hidden rows [T][H]; down: act rows [A][I] (bf16)
  const int32_t* sorted_tok;  // gate/up only
  const int32_t* crow;        // gate/up: per token [T]; down: per sorted row [A]
  const int32_t* eminmin;     // per weight slot
  const uint8_t* w;
  const uint8_t* s;
  const int32_t* seg_start;
  const int32_t* tile_expert;
  const int32_t* tile_row0;
  const int32_t* tile_lo;
  const int32_t* tile_hi;
  const int32_t* slot_map;
  void* out;                  // act bf16 [A][I] / y fp32 [A][H]
  int H, I, bm;
  float limit, alpha, beta;
};

constexpr int kI8OffMin = -24;

template <bool GU>
__global__ __launch_bounds__(256) void i8_row_fallback_kernel(I8RowFallbackArgs a) {
  constexpr int kChunk = 2048;
  __shared__ float xl[kChunk];
  __shared__ int fail_rows[128];
  __shared__ int n_fail;
  const int tile = a.tile_lo[0] + blockIdx.x;
  if (tile >= a.tile_hi[0]) return;
  const int e = a.tile_expert[tile];
  const int ws = a.slot_map ? a.slot_map[e] : e;
  const int emn = a.eminmin[ws];
  const int row0 = a.tile_row0[tile];
  const int rows = min(a.bm, a.seg_start[e + 1] - row0);
  if (threadIdx.x == 0) n_fail = 0;
  __syncthreads();
  for (int r = threadIdx.x; r < rows; r += 256) {
    const long pos = row0 + r;
    const int cr = GU ? a.crow[a.sorted_tok[pos]] : a.crow[pos];
    if (cr + emn - 128 < kI8OffMin) fail_rows[atomicAdd(&n_fail, 1)] = r;
  }
  __syncthreads();
  const int nf = n_fail;
  if (nf == 0) return;
  const int K = GU ? a.H : a.I;
  const int N = GU ? 2 * a.I : a.H;
  const int ncol = GU ? a.I : a.H;   // output columns (gate/up: column pairs)
  const long w_es = WFmt<kMXFP4>::w_bytes(N, K), s_es = WFmt<kMXFP4>::s_bytes(N, K);
  const uint8_t* we = a.w + (long)ws * w_es;
  const uint8_t* se = a.s + (long)ws * s_es;
  for (int f = 0; f < nf; ++f) {
    const long pos = row0 + fail_rows[f];
    const long src = GU ? (long)a.sorted_tok[pos] : pos;
    const uint16_t* xr = a.x + src * K;
    for (int c0 = 0; c0 < ncol; c0 += 256) {
      const int col = c0 + threadIdx.x;
      float g = 0.f, u = 0.f;
      for (int k0 = 0; k0 < K; k0 += kChunk) {
        const int kn = min(kChunk, K - k0);
        __syncthreads();
        for (int k = threadIdx.x; k < kn; k += 256)
          xl[k] = __uint_as_float((uint32_t)xr[k0 + k] << 16);
        __syncthreads();
        if (col < ncol) {
          for (int k = 0; k < kn; ++k) {
            g = __builtin_fmaf(xl[k], mxfp4_at(we, se, col, k0 + k, K), g);
            if (GU) u = __builtin_fmaf(xl[k], mxfp4_at(we, se, a.I + col, k0 + k, K), u);
          }
        }
      }
      if (col < ncol) {
        if (GU)
          reinterpret_cast<uint16_t*>(a.out)[pos * a.I + col] =
              f32_to_bf16(silu_gate(g, u, a.limit, a.alpha, a.beta));
        else
          reinterpret_cast<float*>(a.out)[pos * a.H + col] = g;
      }
    }
  }
}

}  // namespace
}  // namespace xtu

using namespace xtu;

extern "C" {

size_t xtu_i8_weight_bytes(int N, int K) { return (size_t)N * (size_t)K; }

hipError_t xtu_i8_prepare(const void* w, const void* s, int E, int N, int K, void* w8,
                          void* emin, int32_t* dmax, hipStream_t stream) {
  // dmax must hold 0 on entry; it receives the largest b - emin over all rows
  XTU_CHECK_ARG(E > 0 && N > 0 && K > 0 && N % 16 == 0 && K % 128 == 0);
  XTU_CHECK_ARG(w && s && w8 && emin && dmax);
  (void)hipGetLastError();
  const long w_es = WFmt<kMXFP4>::w_bytes(N, K), s_es = WFmt<kMXFP4>::s_bytes(N, K),
             w8_es = (long)N * K;
  i8_emin_kernel<<<dim3((N + 255) / 256, E), 256, 0, stream>>>((const uint8_t*)s, N, K, s_es,
                                                               (uint8_t*)emin, dmax);
  const long nch = (long)N * K / 32;
  i8_expand_kernel<<<dim3((unsigned)((nch + 255) / 256), E), 256, 0, stream>>>(
      (const uint8_t*)w, (const uint8_t*)s, N, K, w_es, s_es, (const uint8_t*)emin,
      (uint8_t*)w8, w8_es);
  return hipPeekAtLastError();
}

hipError_t xtu_i8_quant_rows(const void* rows_bf16, int M, int K, int8_t* a8, int32_t* crow,
                             hipStream_t stream) {
  XTU_CHECK_ARG(M >= 0 && K > 0 && K % 8 == 0);
  if (M == 0) return hipSuccess;
  XTU_CHECK_ARG(rows_bf16 && a8 && crow);
  (void)hipGetLastError();
  i8_quant_rows_kernel<<<(M + 3) / 4, 256, 0, stream>>>((const uint16_t*)rows_bf16, M, K, a8, crow);
  return hipPeekAtLastError();
}

static hipError_t i8_gemm(bool gu, I8GemmArgs a, int max_tiles, hipStream_t stream) {
  const long items = (long)max_tiles * (gu ? a.I / 128 : a.H / 256);
  const long grid = (items + 7) / 8 * 8;
  if (grid >= (1L << 31)) return hipErrorInvalidValue;
  if (grid == 0) return hipSuccess;
  if (gu) {
    a.w_estride = 2L * a.I * a.H;
    i8_gemm_kernel<128, true><<<dim3((unsigned)grid), 256, 0, stream>>>(a);
  } else {
    a.w_estride = (long)a.H * a.I;
    i8_gemm_kernel<128, false><<<dim3((unsigned)grid), 256, 0, stream>>>(a);
  }
  return hipPeekAtLastError();
}

hipError_t xtu_i8_gemm_gate_up(const int8_t* a8, const int32_t* crow, const int32_t* sorted_tok,
                               int H, int I, const void* w8, const void* emin,
                               const int32_t* slot_map, const int32_t* seg_start,
                               const int32_t* tile_expert, const int32_t* tile_row0,
                               const int32_t* tile_lo, const int32_t* tile_hi, int max_tiles,
                               void* act, int32_t* acc_out, float limit, float alpha, float beta,
                               hipStream_t stream) {
  XTU_CHECK_ARG(H > 0 && I > 0 && H % 256 == 0 && I % 128 == 0 && max_tiles >= 0);
  XTU_CHECK_ARG(a8 && crow && sorted_tok && w8 && emin && seg_start && tile_expert && tile_row0 &&
                tile_lo && tile_hi && act);
  if (max_tiles == 0) return hipSuccess;
  (void)hipGetLastError();
  I8GemmArgs a{a8, crow, sorted_tok, (const uint8_t*)w8, (const uint8_t*)emin, seg_start,
               tile_expert, tile_row0, tile_lo, tile_hi, slot_map, act, acc_out, H, I, 0,
               limit, alpha, beta};
  return i8_gemm(true, a, max_tiles, stream);
}

hipError_t xtu_i8_gemm_down(const int8_t* a8, const int32_t* crow, int H, int I, const void* w8,
                            const void* emin, const int32_t* slot_map, const int32_t* seg_start,
                            const int32_t* tile_expert, const int32_t* tile_row0,
                            const int32_t* tile_lo, const int32_t* tile_hi, int max_tiles,
                            float* y, int32_t* acc_out, hipStream_t stream) {
  XTU_CHECK_ARG(H > 0 && I > 0 && H % 256 == 0 && I % 128 == 0 && max_tiles >= 0);
  XTU_CHECK_ARG(a8 && crow && w8 && emin && seg_start && tile_expert && tile_row0 && tile_lo &&
                tile_hi && y);
  if (max_tiles == 0) return hipSuccess;
  (void)hipGetLastError();
  I8GemmArgs a{a8, crow, nullptr, (const uint8_t*)w8, (const uint8_t*)emin, seg_start,
               tile_expert, tile_row0, tile_lo, tile_hi, slot_map, y, acc_out, H, I, 0, 0.f,
               1.f, 0.f};
  return i8_gemm(false, a, max_tiles, stream);
}

hipError_t xtu_i8_fallback(int gate_up, const void* x, const int32_t* sorted_tok, int H, int I,
                           const void* w, const void* s, const int32_t* slot_map,
                           const int32_t* seg_start, const int32_t* tile_expert,
                           const int32_t* tile_row0, const int32_t* tile_lo,
                           const int32_t* tile_hi, int max_tiles, int bm,
                           const int32_t* col_start, const int32_t* cols, void* out, float limit,
                           float alpha, float beta, hipStream_t stream) {
  XTU_CHECK_ARG(H > 0 && I > 0 && H % 256 == 0 && I % 128 == 0 && max_tiles >= 0);
  XTU_CHECK_ARG(bm > 0 && bm <= 128);
  XTU_CHECK_ARG(x && w && s && seg_start && tile_expert && tile_row0 && tile_lo && tile_hi &&
                col_start && cols && out && (!gate_up || sorted_tok));
  if (max_tiles == 0) return hipSuccess;
  (void)hipGetLastError();
  I8FallbackArgs a{(const uint16_t*)x, sorted_tok, (const uint8_t*)w, (const uint8_t*)s,
                   seg_start, tile_expert, tile_row0, tile_lo, tile_hi, slot_map, col_start,
                   cols, out, H, I, bm, limit, alpha, beta};
  if (gate_up) i8_fallback_kernel<true><<<max_tiles, 256, 0, stream>>>(a);
  else i8_fallback_kernel<false><<<max_tiles, 256, 0, stream>>>(a);
  return hipPeekAtLastError();
}

hipError_t xtu_i8_emin_min(const void* s, int E, int N, int K, int32_t* eminmin,
                           hipStream_t stream) {
  XTU_CHECK_ARG(E >= 0 && N > 0 && K > 0 && N % 16 == 0 && K % 128 == 0);
  if (E == 0) return hipSuccess;
  XTU_CHECK_ARG(s && eminmin);
  (void)hipGetLastError();
  i8_emin_min_kernel<<<E, 256, 0, stream>>>((const uint8_t*)s, N, K, WFmt<kMXFP4>::s_bytes(N, K),
                                             eminmin);
  return hipPeekAtLastError();
}

hipError_t xtu_i8_row_fallback(int gate_up, const void* x, const int32_t* sorted_tok,
                               const int32_t* crow, const int32_t* eminmin, int H, int I,
                               const void* w, const void* s, const int32_t* slot_map,
                               const int32_t* seg_start, const int32_t* tile_expert,
                               const int32_t* tile_row0, const int32_t* tile_lo,
                               const int32_t* tile_hi, int max_tiles, int bm, void* out,
                               float limit, float alpha, float beta, hipStream_t stream) {
  XTU_CHECK_ARG(H > 0 && I > 0 && H % 256 == 0 && I % 128 == 0 && max_tiles >= 0);
  XTU_CHECK_ARG(bm > 0 && bm <= 128);
  XTU_CHECK_ARG(x && crow && eminmin && w && s && seg_start && tile_expert && tile_row0 &&
                tile_lo && tile_hi && out && (!gate_up || sorted_tok));
  if (max_tiles == 0) return hipSuccess;
  (void)hipGetLastError();
  I8RowFallbackArgs a{(const uint16_t*)x, sorted_tok, crow, eminmin, (const uint8_t*)w,
                      (const uint8_t*)s, seg_start, tile_expert, tile_row0, tile_lo, tile_hi,
                      slot_map, out, H, I, bm, limit, alpha, beta};
  if (gate_up) i8_row_fallback_kernel<true><<<max_tiles, 256, 0, stream>>>(a);
  else i8_row_fallback_kernel<false><<<max_tiles, 256, 0, stream>>>(a);
  return hipPeekAtLastError();
}

}  // extern "C"
