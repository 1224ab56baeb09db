// Routing (a1) and token permutation / segmentation (a2) for the MoE expert path.
//
// Routing: one wave64 per token.  Each lane owns experts lane, lane+64, ...;
// top-k is K rounds of a wave argmax under the total order (score desc,
// index asc), so the result is unique and identical to a sequential scan.
// Weights are formed by lane 0 in a fixed fp32 sequence (see xtu_expf).
//
// Segmentation: a stable counting sort of the flat (token, expert) pairs by
// bucket, in three launches (per-block histogram in LDS, one-workgroup scan,
// per-block stable scatter).  Ranks inside a block are exact: a wave finds
// the lanes sharing its bucket with ballots, waves are ordered through LDS
// counters, and blocks through the scanned histogram.
#include "xtu_common.hpp"

namespace xtu {
namespace {

constexpr int kWave = 64;
constexpr int kMaxPerLane = 16;  // E <= 1024

__device__ __forceinline__ bool better(float sa, int ia, float sb, int ib) {
  return (sa > sb) || (sa == sb && ia < ib);
}

// One DPP step of the wave argmax: combine with the lane selected by `ctrl`
// (lanes whose source is masked keep their own value).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ void dpp_argmax_step(float& s, int& i) {
  const float os = __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(s), __float_as_int(s), CTRL, ROW_MASK, 0xF, false));
  const int oi = __builtin_amdgcn_update_dpp(i, i, CTRL, ROW_MASK, 0xF, false);
  if (better(os, oi, s, i)) {
    s = os;
    i = oi;
  }
}

// wave argmax of (s, i) pairs under `better`; every lane gets the winner.
// quad xor 1, quad xor 2, half-row mirror, row mirror, row_bcast15, row_bcast31
// leave the maximum in lane 63, which is then read back as a uniform value.
__device__ __forceinline__ void wave_argmax(float& s, int& i) {
  dpp_argmax_step<0xB1, 0xF>(s, i);   // quad_perm [1,0,3,2]
  dpp_argmax_step<0x4E, 0xF>(s, i);   // quad_perm [2,3,0,1]
  dpp_argmax_step<0x141, 0xF>(s, i);  // row_half_mirror
  dpp_argmax_step<0x140, 0xF>(s, i);  // row_mirror
  dpp_argmax_step<0x142, 0xA>(s, i);  // row_bcast15 into rows 1, 3
  dpp_argmax_step<0x143, 0xC>(s, i);  // row_bcast31 into rows 2, 3
  s = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 63));
  i = __builtin_amdgcn_readlane(i, 63);
}

__device__ __forceinline__ float lane_read(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Route one token with one wave.  MODE 0: softmax top-k, MODE 1: grouped
// sigmoid.  NPER = experts per lane (E <= 64 * NPER); sb is this wave's LDS
// scratch of E floats.  On return lanes k < K hold the k-th choice in
// (id, weight); the fp32 weight sequence is the one the host oracle restates.
template <int MODE, int NPER>
__device__ __forceinline__ void route_one_token(const float* __restrict__ l,
                                                const float* __restrict__ bias, int E, int K,
                                                int n_group, int topk_group, float scale,
                                                int renorm, float* sb, int lane, int& my_id,
                                                float& my_w) {
#pragma clang fp contract(off)
  const float NEG = -__builtin_inff();
  float sel[NPER], wsc[NPER];
#pragma unroll
  for (int j = 0; j < NPER; ++j) {
    const int e = lane + kWave * j;
    float v = NEG, w = 0.f;
    if (e < E) {
      const float x = l[e];
      if (MODE == 0) {
        v = x;
      } else {
        w = xtu_sigmoid(x);
        v = w + (bias ? bias[e] : 0.0f);
      }
    }
    sel[j] = v;
    wsc[j] = w;
  }
  uint64_t gmask = ~0ull;
  int gsz = E;
  if (MODE == 1) {
#pragma unroll
    for (int j = 0; j < NPER; ++j) {
      const int e = lane + kWave * j;
      if (e < E) sb[e] = sel[j];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    gsz = E / n_group;
    float g = NEG;
    if (lane < n_group) {
      // two best (score desc, index asc) of the group, kept in registers
      float v1 = NEG, v2 = NEG;
      int i1 = -1, i2 = -1;
      for (int q = 0; q < gsz; ++q) {
        const int e = lane * gsz + q;
        const float v = sb[e];
        if (i1 < 0 || better(v, e, v1, i1)) {
          v2 = v1; i2 = i1;
          v1 = v; i1 = e;
        } else if (i2 < 0 || better(v, e, v2, i2)) {
          v2 = v; i2 = e;
        }
      }
      g = (gsz >= 2) ? (v1 + v2) : v1;
    }
    gmask = 0;
    bool taken = false;
    for (int k = 0; k < topk_group; ++k) {
      float s = (lane < n_group && !taken) ? g : NEG;
      int i = (lane < n_group && !taken) ? lane : 0x7fffffff;
      wave_argmax(s, i);
      if (lane == i) taken = true;
      gmask |= 1ull << i;
    }
  }
  uint32_t used = 0;
  my_id = -1;
  float my_s = 0.f, my_wsc = 0.f;
  for (int k = 0; k < K; ++k) {
    float s = NEG;
    int i = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < NPER; ++j) {
      const int e = lane + kWave * j;
      if (e < E && !((used >> j) & 1u) && ((gmask >> (e / gsz)) & 1ull)) {
        if (better(sel[j], e, s, i)) {
          s = sel[j];
          i = e;
        }
      }
    }
    wave_argmax(s, i);
    const int owner = i % kWave, jw = i / kWave;
    float w = 0.f;
#pragma unroll
    for (int j = 0; j < NPER; ++j)
      if (j == jw) w = wsc[j];
    if (lane == owner) used |= 1u << jw;
    w = lane_read(w, owner);
    if (lane == k) {
      my_id = i;
      my_s = s;
      my_wsc = w;
    }
  }
  if (MODE == 0) {
    const float lmax = lane_read(my_s, 0);
    const float ev = (lane < K) ? xtu_expf(my_s - lmax) : 0.f;
    float sum = 0.0f;
    if (renorm) {
      for (int k = 0; k < K; ++k) sum = sum + lane_read(ev, k);
    } else {
#pragma unroll
      for (int j = 0; j < NPER; ++j) {
        const int e = lane + kWave * j;
        const float x = (e < E) ? xtu_expf(l[e] - lmax) : 0.f;
        for (int q = 0; q < kWave; ++q)
          if (q + kWave * j < E) sum = sum + lane_read(x, q);
      }
    }
    my_w = __fdiv_rn(ev, sum);
  } else {
    float sum = 0.0f;
    for (int k = 0; k < K; ++k) sum = sum + lane_read(my_wsc, k);
    my_w = renorm ? __fdiv_rn(my_wsc, sum) * scale : my_wsc * scale;
  }
}

template <int MODE, int NPER>
__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits,
                                                    const float* __restrict__ bias, int T, int E,
                                                    int K, int n_group, int topk_group,
                                                    float scale, int renorm,
                                                    int32_t* __restrict__ ids,
                                                    float* __restrict__ wts) {
  __shared__ float sb[4][64 * NPER];
  const int wv = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int t = blockIdx.x * 4 + wv;
  if (t >= T) return;   // no block-wide barrier below
  int id;
  float w;
  route_one_token<MODE, NPER>(logits + (size_t)t * E, bias, E, K, n_group, topk_group, scale,
                              renorm, sb[wv], lane, id, w);
  if (lane < K) {
    ids[(size_t)t * K + lane] = id;
    wts[(size_t)t * K + lane] = w;
  }
}

// ----------------------------------------------------------------------------
// segmentation
// ----------------------------------------------------------------------------
constexpr int kSegThreads = 256;
constexpr int kSegRounds = 16;
constexpr int kSegChunk = kSegThreads * kSegRounds;   // pairs per block

struct SegArgs {
  const int32_t* ids;
  const float* wts;
  const int32_t* id_map;   // optional id translation applied before bucketing
  int T, K, E, NS, drop_zero, A, NB;
};

__device__ __forceinline__ int bucket_of(const SegArgs& a, int p, float* w_out, int* tok_out) {
  const int TK = a.T * a.K;
  if (p < TK) {
    int e = a.ids[p];
    if (a.id_map && e >= 0 && e < a.E) e = a.id_map[e];
    const float w = a.wts[p];
    *w_out = w;
    *tok_out = p / a.K;
    int b = (e < 0 || e >= a.E) ? (a.E + a.NS) : e;
    if (a.drop_zero && w == 0.0f) b = a.E + a.NS;
    return b;
  }
  const int q = p - TK;
  *w_out = 1.0f;
  *tok_out = q / a.NS;
  return a.E + q % a.NS;
}

__global__ __launch_bounds__(kSegThreads) void seg_hist_kernel(SegArgs a,
                                                               int32_t* __restrict__ bcnt) {
  extern __shared__ int cnt[];
  for (int e = threadIdx.x; e < a.NB; e += kSegThreads) cnt[e] = 0;
  __syncthreads();
  const int base = blockIdx.x * kSegChunk;
  for (int r = 0; r < kSegRounds; ++r) {
    const int p = base + r * kSegThreads + threadIdx.x;
    if (p < a.A) {
      float w;
      int tok;
      atomicAdd(&cnt[bucket_of(a, p, &w, &tok)], 1);
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < a.NB; e += kSegThreads)
    bcnt[(size_t)blockIdx.x * a.NB + e] = cnt[e];
}

// One workgroup: per-bucket exclusive prefix over blocks (in place), bucket
// totals, seg_start, the list of non-empty expert buckets and the GEMM tile
// list (tiles of bm rows inside each non-trash bucket).
__global__ __launch_bounds__(1024) void seg_scan_kernel(int NB, int nblocks, int bm,
                                                        int32_t* __restrict__ bcnt,
                                                        int32_t* __restrict__ seg_start,
                                                        int32_t* __restrict__ active,
                                                        int32_t* __restrict__ n_active,
                                                        int32_t* __restrict__ tile_expert,
                                                        int32_t* __restrict__ tile_row0,
                                                        int32_t* __restrict__ n_tiles,
                                                        int32_t* __restrict__ expert_tile_start) {
  __shared__ int s_tot[2048];
  __shared__ int s_act[2048];
  __shared__ int s_til[2048];
  __shared__ int s_part[3][32];
  const int tid = threadIdx.x;
  // per-bucket running sum over blocks
  for (int e = tid; e < NB; e += 1024) {
    int run = 0;
    int b = 0;
    for (; b + 4 <= nblocks; b += 4) {
      const int c0 = bcnt[(size_t)(b + 0) * NB + e];
      const int c1 = bcnt[(size_t)(b + 1) * NB + e];
      const int c2 = bcnt[(size_t)(b + 2) * NB + e];
      const int c3 = bcnt[(size_t)(b + 3) * NB + e];
      bcnt[(size_t)(b + 0) * NB + e] = run;
      bcnt[(size_t)(b + 1) * NB + e] = run + c0;
      bcnt[(size_t)(b + 2) * NB + e] = run + c0 + c1;
      bcnt[(size_t)(b + 3) * NB + e] = run + c0 + c1 + c2;
      run += c0 + c1 + c2 + c3;
    }
    for (; b < nblocks; ++b) {
      const int c = bcnt[(size_t)b * NB + e];
      bcnt[(size_t)b * NB + e] = run;
      run += c;
    }
    s_tot[e] = run;
    const bool expert = e < NB - 1;   // last bucket is the trash bucket
    s_act[e] = (expert && run > 0) ? 1 : 0;
    s_til[e] = expert ? (run + bm - 1) / bm : 0;
  }
  __syncthreads();
  // exclusive scans of s_tot, s_act, s_til over NB <= 2048 entries: each
  // thread owns two consecutive entries; wave scans, then a scan of wave sums.
  int v[3][2];
  const int i0 = 2 * tid, i1 = 2 * tid + 1;
  int* arr[3] = {s_tot, s_act, s_til};
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    v[q][0] = i0 < NB ? arr[q][i0] : 0;
    v[q][1] = i1 < NB ? arr[q][i1] : 0;
  }
  int incl[3];
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    int s = v[q][0] + v[q][1];
    const int lane = tid % 64;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int o = __shfl_up(s, off, 64);
      if (lane >= off) s += o;
    }
    incl[q] = s;
    if (lane == 63) s_part[q][tid / 64] = s;
  }
  __syncthreads();
  if (tid < 32) {
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      int s = tid < 16 ? s_part[q][tid] : 0;
      for (int off = 1; off < 32; off <<= 1) {
        const int o = __shfl_up(s, off, 32);
        if (tid >= off) s += o;
      }
      s_part[q][tid] = s;   // inclusive over waves
    }
  }
  __syncthreads();
  int ex[3][2];
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    const int w = tid / 64;
    const int wave_base = w > 0 ? s_part[q][w - 1] : 0;
    const int excl = wave_base + incl[q] - (v[q][0] + v[q][1]);
    ex[q][0] = excl;
    ex[q][1] = excl + v[q][0];
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int e = 2 * tid + h;
    if (e < NB) {
      seg_start[e] = ex[0][h];
      if (e == NB - 1) seg_start[NB] = ex[0][h] + v[0][h];
      if (v[1][h]) active[ex[1][h]] = e;
      expert_tile_start[e] = ex[2][h];
      if (e == NB - 1) expert_tile_start[NB] = ex[2][h] + v[2][h];
      const int nt = v[2][h];
      for (int j = 0; j < nt; ++j) {
        tile_expert[ex[2][h] + j] = e;
        tile_row0[ex[2][h] + j] = ex[0][h] + j * bm;
      }
    }
  }
  if (tid == 1023) {
    n_active[0] = s_part[1][15];
    n_tiles[0] = s_part[2][15];
  }
}

__global__ __launch_bounds__(kSegThreads) void seg_scatter_kernel(
    SegArgs a, const int32_t* __restrict__ bexcl, const int32_t* __restrict__ seg_start,
    int32_t* __restrict__ sorted_pair, int32_t* __restrict__ sorted_tok,
    float* __restrict__ sorted_wts, int32_t* __restrict__ inv) {
  extern __shared__ int lds[];
  int* run = lds;                       // [NB] running count of this block
  int* wcnt = lds + a.NB;               // [4][NB] per-wave counts of the round
  const int wv = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  for (int e = threadIdx.x; e < a.NB; e += kSegThreads) {
    run[e] = seg_start[e] + bexcl[(size_t)blockIdx.x * a.NB + e];
    wcnt[e] = wcnt[a.NB + e] = wcnt[2 * a.NB + e] = wcnt[3 * a.NB + e] = 0;
  }
  __syncthreads();
  const int base = blockIdx.x * kSegChunk;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int r = 0; r < kSegRounds; ++r) {
    const int p = base + r * kSegThreads + threadIdx.x;
    const bool valid = p < a.A;
    float w = 0.f;
    int tok = 0;
    const int bk = valid ? bucket_of(a, p, &w, &tok) : -1;
    // lanes of this wave that share my bucket
    uint64_t remaining = __ballot(valid);
    int rank = 0, wcount = 0;
    bool leader = false;
    while (remaining) {
      const int ld = __builtin_ctzll(remaining);
      const int lb = __shfl(bk, ld, kWave);
      const uint64_t m = __ballot(valid && bk == lb);
      if (valid && bk == lb) {
        rank = __builtin_popcountll(m & lt_mask);
        wcount = __builtin_popcountll(m);
        leader = (lane == ld);
      }
      remaining &= ~m;
    }
    if (leader) wcnt[wv * a.NB + bk] = wcount;
    __syncthreads();
    if (valid) {
      int before = 0;
      for (int q = 0; q < wv; ++q) before += wcnt[q * a.NB + bk];
      const int pos = run[bk] + before + rank;
      sorted_pair[pos] = p;
      sorted_tok[pos] = tok;
      sorted_wts[pos] = w;
      inv[p] = pos;
    }
    __syncthreads();
    // advance the running counters and clear the round's wave counts
    if (leader) {
      // the last wave holding this bucket adds the whole round's count
      int total = 0;
      bool last = true;
      for (int q = 0; q < 4; ++q) {
        const int c = wcnt[q * a.NB + bk];
        total += c;
        if (q > wv && c > 0) last = false;
      }
      if (last) run[bk] += total;
    }
    __syncthreads();
    if (leader) wcnt[wv * a.NB + bk] = 0;
    __syncthreads();
  }
}

// ----------------------------------------------------------------------------
// Small batches (decode): routing and the whole segmentation in one
// workgroup.  A = T*K + T*NS <= 1024 pairs, NB <= 2048 buckets.  Same
// outputs, same order and same fp32 sequence as the multi-launch path.
// ----------------------------------------------------------------------------
constexpr int kSmallMaxA = 1024;
constexpr int kSmallMaxNB = 2048;

// In-place exclusive scan of a[0, n) (n <= 2048) by 256 threads; returns the total.
__device__ int block_excl_scan_256(int* a, int n, int* wsum) {
  const int tid = threadIdx.x, lane = tid % kWave, wv = tid / kWave;
  const int per = (n + 255) / 256;
  int loc[8];
  int s = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int idx = tid * per + i;
    const int v = (i < per && idx < n) ? a[idx] : 0;
    loc[i] = s;
    s += v;
  }
  int incl = s;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int o = __shfl_up(incl, off, kWave);
    if (lane >= off) incl += o;
  }
  if (lane == kWave - 1) wsum[wv] = incl;
  __syncthreads();
  int base = 0;
  for (int q = 0; q < wv; ++q) base += wsum[q];
  const int total = wsum[0] + wsum[1] + wsum[2] + wsum[3];
  const int ex = base + incl - s;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int idx = tid * per + i;
    if (i < per && idx < n) a[idx] = ex + loc[i];
  }
  __syncthreads();
  return total;
}

struct SmallArgs {
  const float* logits;
  const float* bias;
  int32_t* ids;
  float* wts;
  const int32_t* id_map;
  int T, K, E, n_group, topk_group, renorm, NS, drop_zero, bm;
  float scale;
  int32_t *sorted_pair, *sorted_tok, *inv, *seg_start, *active, *n_active;
  float* sorted_wts;
  int32_t *tile_expert, *tile_row0, *n_tiles, *expert_tile_start;
};

// MODE 0: softmax routing, 1: grouped sigmoid routing, 2: ids/wts given.
template <int MODE, int NPER>
__global__ __launch_bounds__(256) void route_seg_small_kernel(SmallArgs a) {
  __shared__ float sb[4][64 * NPER];
  __shared__ int s_ids[kSmallMaxA];
  __shared__ float s_w[kSmallMaxA];
  __shared__ int s_bk[kSmallMaxA];
  __shared__ int s_cnt[kSmallMaxNB];
  __shared__ int s_act[kSmallMaxNB];
  __shared__ int s_til[kSmallMaxNB];
  __shared__ int s_wsum[4];
  const int tid = threadIdx.x, wv = tid / kWave, lane = tid % kWave;
  const int T = a.T, K = a.K, E = a.E, NS = a.NS;
  const int TK = T * K, A = TK + T * NS, NB = E + NS + 1;
  if (MODE < 2) {
    for (int t = wv; t < T; t += 4) {
      int id;
      float w;
      route_one_token<MODE < 2 ? MODE : 0, NPER>(a.logits + (size_t)t * E, a.bias, E, K,
                                                  a.n_group, a.topk_group, a.scale, a.renorm,
                                                  sb[wv], lane, id, w);
      if (lane < K) {
        a.ids[t * K + lane] = id;
        a.wts[t * K + lane] = w;
        s_ids[t * K + lane] = id;
        s_w[t * K + lane] = w;
      }
    }
  } else {
    for (int p = tid; p < TK; p += 256) {
      s_ids[p] = a.ids[p];
      s_w[p] = a.wts[p];
    }
  }
  for (int e = tid; e < NB; e += 256) s_cnt[e] = 0;
  __syncthreads();
  for (int p = tid; p < A; p += 256) {
    int b;
    if (p < TK) {
      int e = s_ids[p];
      if (a.id_map && e >= 0 && e < E) e = a.id_map[e];
      b = (e < 0 || e >= E) ? (E + NS) : e;
      if (a.drop_zero && s_w[p] == 0.0f) b = E + NS;
    } else {
      b = E + (p - TK) % NS;
    }
    s_bk[p] = b;
    atomicAdd(&s_cnt[b], 1);
  }
  __syncthreads();
  for (int e = tid; e < NB; e += 256) {
    const int c = s_cnt[e];
    const bool expert = e < NB - 1;
    s_act[e] = (expert && c > 0) ? 1 : 0;
    s_til[e] = expert ? (c + a.bm - 1) / a.bm : 0;
  }
  __syncthreads();
  block_excl_scan_256(s_cnt, NB, s_wsum);
  const int n_act = block_excl_scan_256(s_act, NB, s_wsum);
  const int n_til = block_excl_scan_256(s_til, NB, s_wsum);
  for (int e = tid; e < NB; e += 256) {
    const int st = s_cnt[e];
    const int en = (e + 1 < NB) ? s_cnt[e + 1] : A;
    const int c = en - st;
    a.seg_start[e] = st;
    a.expert_tile_start[e] = s_til[e];
    if (e == NB - 1) {
      a.seg_start[NB] = A;
      a.expert_tile_start[NB] = n_til;
    }
    if (e < NB - 1 && c > 0) {
      a.active[s_act[e]] = e;
      const int nt = (c + a.bm - 1) / a.bm;
      for (int j = 0; j < nt; ++j) {
        a.tile_expert[s_til[e] + j] = e;
        a.tile_row0[s_til[e] + j] = st + j * a.bm;
      }
    }
  }
  if (tid == 0) {
    a.n_active[0] = n_act;
    a.n_tiles[0] = n_til;
  }
  for (int p = tid; p < A; p += 256) {
    const int b = s_bk[p];
    int r = 0;
    for (int q = 0; q < p; ++q) r += (s_bk[q] == b) ? 1 : 0;
    const int pos = s_cnt[b] + r;
    a.sorted_pair[pos] = p;
    a.inv[p] = pos;
    if (p < TK) {
      a.sorted_tok[pos] = p / K;
      a.sorted_wts[pos] = s_w[p];
    } else {
      a.sorted_tok[pos] = (p - TK) / NS;
      a.sorted_wts[pos] = 1.0f;
    }
  }
}

template <int MODE>
void launch_small(const SmallArgs& a, hipStream_t stream) {
  if (a.E <= 64) route_seg_small_kernel<MODE, 1><<<1, 256, 0, stream>>>(a);
  else if (a.E <= 256) route_seg_small_kernel<MODE, 4><<<1, 256, 0, stream>>>(a);
  else if (a.E <= 512) route_seg_small_kernel<MODE, 8><<<1, 256, 0, stream>>>(a);
  else route_seg_small_kernel<MODE, 16><<<1, 256, 0, stream>>>(a);
}

template <int MODE>
void launch_route(const float* logits, const float* bias, int T, int E, int K, int n_group,
                  int topk_group, float scale, int renorm, int32_t* ids, float* wts,
                  hipStream_t stream) {
  const dim3 grid((T + 3) / 4);
  if (E <= 64)
    route_kernel<MODE, 1><<<grid, 256, 0, stream>>>(logits, bias, T, E, K, n_group, topk_group,
                                                    scale, renorm, ids, wts);
  else if (E <= 256)
    route_kernel<MODE, 4><<<grid, 256, 0, stream>>>(logits, bias, T, E, K, n_group, topk_group,
                                                    scale, renorm, ids, wts);
  else if (E <= 512)
    route_kernel<MODE, 8><<<grid, 256, 0, stream>>>(logits, bias, T, E, K, n_group, topk_group,
                                                    scale, renorm, ids, wts);
  else
    route_kernel<MODE, 16><<<grid, 256, 0, stream>>>(logits, bias, T, E, K, n_group, topk_group,
                                                     scale, renorm, ids, wts);
}

}  // namespace
}  // namespace xtu

using namespace xtu;

extern "C" {

hipError_t xtu_route_softmax_topk(const float* logits, int T, int E, int K, int renormalize,
                                  int32_t* topk_ids, float* topk_weights, hipStream_t stream) {
  XTU_CHECK_ARG(T >= 0 && E > 0 && E <= 1024 && K > 0 && K <= 16 && K <= E);
  XTU_CHECK_ARG(T == 0 || (logits && topk_ids && topk_weights));
  if (T == 0) return hipSuccess;
  (void)hipGetLastError();
  launch_route<0>(logits, nullptr, T, E, K, 1, 1, 1.0f, renormalize, topk_ids, topk_weights,
                  stream);
  return hipPeekAtLastError();
}

hipError_t xtu_route_grouped_sigmoid(const float* logits, const float* bias, int T, int E,
                                     int n_group, int topk_group, int K, float routed_scaling,
                                     int renormalize, int32_t* topk_ids, float* topk_weights,
                                     hipStream_t stream) {
  XTU_CHECK_ARG(T >= 0 && E > 0 && E <= 1024 && K > 0 && K <= 16);
  XTU_CHECK_ARG(n_group > 0 && n_group <= 64 && E % n_group == 0);
  XTU_CHECK_ARG(topk_group > 0 && topk_group <= n_group && K <= topk_group * (E / n_group));
  XTU_CHECK_ARG(T == 0 || (logits && topk_ids && topk_weights));
  if (T == 0) return hipSuccess;
  (void)hipGetLastError();
  launch_route<1>(logits, bias, T, E, K, n_group, topk_group, routed_scaling, renormalize,
                  topk_ids, topk_weights, stream);
  return hipPeekAtLastError();
}

size_t xtu_segment_workspace_bytes(int T, int K, int E, int n_shared) {
  const long A = (long)T * K + (long)T * n_shared;
  const long NB = E + n_shared + 1;
  const long nblocks = (A + kSegChunk - 1) / kSegChunk;
  return (size_t)((nblocks > 0 ? nblocks : 1) * NB * sizeof(int32_t));
}

int xtu_segment_max_tiles(int T, int K, int E, int n_shared, int bm) {
  const long A = (long)T * K + (long)T * n_shared;
  const long nb = E + n_shared;
  return (int)(A / bm + (A < nb ? A : nb) + 1);
}

hipError_t xtu_segment(const int32_t* topk_ids, const float* topk_weights,
                       const int32_t* id_map, int T, int K, int E, int n_shared, int drop_zero,
                       int bm, void* workspace, int32_t* sorted_pair, int32_t* sorted_tok,
                       float* sorted_wts, int32_t* inv, int32_t* seg_start, int32_t* active,
                       int32_t* n_active, int32_t* tile_expert, int32_t* tile_row0,
                       int32_t* n_tiles, int32_t* expert_tile_start, hipStream_t stream) {
  XTU_CHECK_ARG(T >= 0 && K >= 0 && E > 0 && n_shared >= 0 && bm > 0);
  const int NB = E + n_shared + 1;
  XTU_CHECK_ARG(NB <= 2048);
  const long A = (long)T * K + (long)T * n_shared;
  XTU_CHECK_ARG(A < (1l << 30));
  XTU_CHECK_ARG(workspace && seg_start && active && n_active && tile_expert && tile_row0 &&
                n_tiles && expert_tile_start);
  XTU_CHECK_ARG(A == 0 || (sorted_pair && sorted_tok && sorted_wts && inv));
  XTU_CHECK_ARG(T * K == 0 || (topk_ids && topk_weights));
  const int nblocks = (int)((A + kSegChunk - 1) / kSegChunk);
  SegArgs a{topk_ids, topk_weights, id_map, T, K, E, n_shared, drop_zero, (int)A, NB};
  int32_t* bcnt = (int32_t*)workspace;
  (void)hipGetLastError();
  if (nblocks > 0) {
    seg_hist_kernel<<<nblocks, kSegThreads, NB * sizeof(int), stream>>>(a, bcnt);
  }
  seg_scan_kernel<<<1, 1024, 0, stream>>>(NB, nblocks, bm, bcnt, seg_start, active, n_active,
                                          tile_expert, tile_row0, n_tiles, expert_tile_start);
  if (nblocks > 0) {
    seg_scatter_kernel<<<nblocks, kSegThreads, 5 * NB * sizeof(int), stream>>>(
        a, bcnt, seg_start, sorted_pair, sorted_tok, sorted_wts, inv);
  }
  return hipPeekAtLastError();
}

int xtu_route_segment_small_max_pairs(void) { return kSmallMaxA; }

hipError_t xtu_route_segment_small(int mode, const float* logits, const float* bias,
                                   int32_t* topk_ids, float* topk_weights, int T, int E, int K,
                                   int n_group, int topk_group, float routed_scaling,
                                   int renormalize, const int32_t* id_map, int n_shared,
                                   int drop_zero, int bm, int32_t* sorted_pair,
                                   int32_t* sorted_tok, float* sorted_wts, int32_t* inv,
                                   int32_t* seg_start, int32_t* active, int32_t* n_active,
                                   int32_t* tile_expert, int32_t* tile_row0, int32_t* n_tiles,
                                   int32_t* expert_tile_start, hipStream_t stream) {
  XTU_CHECK_ARG(mode >= 0 && mode <= 2 && T >= 0 && E > 0 && E <= 1024 && K > 0 && K <= 16 &&
                K <= E && n_shared >= 0 && bm > 0);
  XTU_CHECK_ARG((long)T * K + (long)T * n_shared <= kSmallMaxA && E + n_shared + 1 <= kSmallMaxNB);
  if (mode == 1)
    XTU_CHECK_ARG(n_group > 0 && n_group <= 64 && E % n_group == 0 && topk_group > 0 &&
                  topk_group <= n_group && K <= topk_group * (E / n_group));
  XTU_CHECK_ARG(topk_ids && topk_weights && (mode == 2 || T == 0 || logits));
  XTU_CHECK_ARG(sorted_pair && sorted_tok && sorted_wts && inv && seg_start && active &&
                n_active && tile_expert && tile_row0 && n_tiles && expert_tile_start);
  SmallArgs a{logits, bias, topk_ids, topk_weights, id_map, T, K, E, n_group, topk_group,
              renormalize, n_shared, drop_zero, bm, routed_scaling, sorted_pair, sorted_tok, inv,
              seg_start, active, n_active, sorted_wts, tile_expert, tile_row0, n_tiles,
              expert_tile_start};
  (void)hipGetLastError();
  if (mode == 0) launch_small<0>(a, stream);
  else if (mode == 1) launch_small<1>(a, stream);
  else launch_small<2>(a, stream);
  return hipPeekAtLastError();
}

}  // extern "C"
