// Routing (a1) and token permutation / segmentation (a2) for the MoE expert path.
//
// Routing: one 256-thread workgroup per token, selection by ranks under the
// total order (score desc, index asc), so the choice and its order equal a
// sequential scan's and take a fixed number of barriers: each expert's rank
// inside its group (grouped routing) or 32-expert chunk (softmax) prunes the
// candidates to K per group, group scores and group ranks pick the groups,
// and a candidate's rank among the survivors is its output slot.  Weights
// are formed by one thread in a fixed fp32 sequence (see xtu_expf).
//
// Segmentation: a stable counting sort of the flat (token, expert) pairs by
// bucket, in three launches (per-block histogram in LDS, one-workgroup scan,
// per-block stable scatter).  Ranks inside a block are exact: a wave finds
// the lanes sharing its bucket with ballots, waves are ordered through LDS
// counters, and blocks through the scanned histogram.
#include <mutex>
#include <stdio.h>

#include "route_tiny.hpp"
#include "xtu_common.hpp"

// Segmentation workspace of xtu_segment_noalloc: one statically allocated
// array per GPU (each device holds its own copy until the process ends).
// Host code must not use this name as an address: it is a host-side stand-in.
// The device address comes from hipGetSymbolAddress, once per device.
static constexpr size_t kNoAllocScratchBytes = 4u << 20;
static __device__ __align__(256) int32_t scratch[kNoAllocScratchBytes / sizeof(int32_t)];

namespace xtu {
namespace {

using tiny::SmallArgs;

constexpr int kWave = 64;

__device__ __forceinline__ bool better(float sa, int ia, float sb, int ib) {
  return (sa > sb) || (sa == sb && ia < ib);
}

constexpr int kMaxE = 1024;
constexpr int kMaxK = 16;
constexpr int kMaxGroups = 64;

// Routing scratch of one team in LDS, laid out from a base for E experts and
// nc = groups * K candidate slots (words): sc, ws [E]; csc, ce [ncp];
// g1, g2, gs, gsel [64]; sel_e, sel_ws, sel_sc [16]; sum.
__host__ __device__ constexpr int route_team_words(int E, int nc) {
  return 2 * E + 2 * ((nc + 3) & ~3) + 4 * kMaxGroups + 3 * kMaxK + 4;
}

struct RouteScratch {
  float *sc, *ws, *csc, *g1, *g2, *gs, *sel_ws, *sel_sc;
  int *ce, *gsel, *sel_e;
  __device__ RouteScratch(float* base, int E, int nc) {
    const int ncp = (nc + 3) & ~3;
    sc = base;
    ws = sc + E;
    csc = ws + E;
    ce = reinterpret_cast<int*>(csc + ncp);
    g1 = reinterpret_cast<float*>(ce + ncp);
    g2 = g1 + kMaxGroups;
    gs = g2 + kMaxGroups;
    gsel = reinterpret_cast<int*>(gs + kMaxGroups);
    sel_e = gsel + kMaxGroups;
    sel_ws = reinterpret_cast<float*>(sel_e + kMaxK);
    sel_sc = sel_ws + kMaxK;
  }
};

// Make this wave's LDS writes visible to its other lanes.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// A team of TEAM threads routes one token: TEAM = 64 is one wave (synced as
// a wave), TEAM = 256 is a quarter of a 1024-thread workgroup whose four
// teams run in lockstep through workgroup barriers.
template <int TEAM>
__device__ __forceinline__ void team_sync() {
  if constexpr (TEAM == kWave) wave_sync();
  else __syncthreads();
}

// Number of (score, index) pairs in [j0, j1) that beat (v, e): 4-wide LDS
// reads, independent of each other, so the latencies overlap.
__device__ __forceinline__ int count_better(const float* sc, const int* idx, int j0, int j1,
                                            float v, int e) {
  int r = 0;
  int j = j0;
  if ((j0 & 3) == 0) {
#pragma unroll 4
    for (; j + 4 <= j1; j += 4) {
      const f32x4_t s4 = *reinterpret_cast<const f32x4_t*>(sc + j);
      if (idx) {
        const i32x4_t i4 = *reinterpret_cast<const i32x4_t*>(idx + j);
#pragma unroll
        for (int q = 0; q < 4; ++q) r += better(s4[q], i4[q], v, e) ? 1 : 0;
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) r += better(s4[q], j + q, v, e) ? 1 : 0;
      }
    }
  }
  for (; j < j1; ++j) r += better(sc[j], idx ? idx[j] : j, v, e) ? 1 : 0;
  return r;
}

// Route one token with a team (thread `tid` of TEAM; `valid` false: no token,
// the team only keeps step with the barriers).  MODE 0: softmax top-k over
// the logits; MODE 1: DeepSeek-V3 grouped sigmoid.  Threads k < K write the
// k-th choice to ids_out[k] / wts_out[k] (and to the LDS copies if given).
template <int MODE, int TEAM>
__device__ void route_token(const float* __restrict__ l, const float* __restrict__ bias, int E,
                            int K, int n_group, int topk_group, float scale, int renorm,
                            const RouteScratch& s, int tid, bool valid, int32_t* ids_out,
                            float* wts_out, int* ids_lds = nullptr, float* wts_lds = nullptr) {
#pragma clang fp contract(off)
  const float NEG = -__builtin_inff();
  const int gsz = MODE == 1 ? E / n_group : 32;   // group, or pruning chunk
  const int ng = MODE == 1 ? n_group : (E + 31) / 32;
  const int nc = ng * K;
  const int ncp = (nc + 3) & ~3;
  if (valid) {
    for (int e = tid; e < E; e += TEAM) {
      const float x = l[e];
      if (MODE == 0) {
        s.sc[e] = x;
        s.ws[e] = x;
      } else {
        const float w = xtu_sigmoid(x);
        s.sc[e] = w + (bias ? bias[e] : 0.0f);
        s.ws[e] = w;
      }
    }
  }
  for (int c = tid; c < ncp; c += TEAM) {
    s.csc[c] = NEG;
    s.ce[c] = 0x7fffffff;
  }
  team_sync<TEAM>();
  // rank inside the group / chunk; the K best of each become candidates
  if (valid) {
    for (int e = tid; e < E; e += TEAM) {
      const int g = e / gsz, j0 = g * gsz;
      const float v = s.sc[e];
      const int r = count_better(s.sc, nullptr, j0, min(j0 + gsz, E), v, e);
      if (r < K) {
        s.csc[g * K + r] = v;
        s.ce[g * K + r] = e;
      }
      if (MODE == 1) {
        if (r == 0) s.g1[g] = v;
        if (r == 1) s.g2[g] = v;
      }
    }
  }
  team_sync<TEAM>();
  if (MODE == 1) {
    // group score = best + second best; keep the topk_group best groups
    if (tid < ng) s.gs[tid] = gsz >= 2 ? s.g1[tid] + s.g2[tid] : s.g1[tid];
    team_sync<TEAM>();
    if (tid < ng) s.gsel[tid] = count_better(s.gs, nullptr, 0, ng, s.gs[tid], tid) < topk_group;
    team_sync<TEAM>();
    for (int c = tid; c < nc; c += TEAM)   // drop the candidates of the other groups
      if (!s.gsel[c / K]) {
        s.csc[c] = NEG;
        s.ce[c] = 0x7fffffff;
      }
    team_sync<TEAM>();
  }
  // rank among the surviving candidates = output slot
  for (int c = tid; c < nc; c += TEAM) {
    const int e = s.ce[c];
    if (e == 0x7fffffff) continue;
    const float v = s.csc[c];
    const int r = count_better(s.csc, s.ce, 0, ncp, v, e);
    if (r < K) {
      s.sel_e[r] = e;
      s.sel_ws[r] = s.ws[e];
      s.sel_sc[r] = v;
    }
  }
  team_sync<TEAM>();
  // weights: lanes k < K of the team's first wave, sums in k order
  float wk = 0.f;
  if (tid < K) wk = s.sel_ws[tid];
  int id = 0;
  float w = 0.f;
  if (MODE == 0) {
    const float lmax = s.sel_sc[0];
    const float ev = tid < K ? xtu_expf(wk - lmax) : 0.f;   // e^(l_k - lmax)
    float sum = 0.0f;
    if (renorm) {
      for (int k = 0; k < K; ++k) sum = sum + __shfl(ev, k, kWave);
    } else {
      team_sync<TEAM>();   // sel_* read before ws is rewritten
      if (valid)
        for (int e = tid; e < E; e += TEAM) s.ws[e] = xtu_expf(s.sc[e] - lmax);
      team_sync<TEAM>();
      if (tid == 0)
        for (int e = 0; e < E; ++e) sum = sum + s.ws[e];
      sum = __shfl(sum, 0, kWave);
    }
    if (tid < K) {
      id = s.sel_e[tid];
      w = __fdiv_rn(ev, sum);
    }
  } else {
    float sum = 0.0f;
    for (int k = 0; k < K; ++k) sum = sum + __shfl(wk, k, kWave);
    if (tid < K) {
      id = s.sel_e[tid];
      w = renorm ? __fdiv_rn(wk, sum) * scale : wk * scale;
    }
  }
  if (valid && tid < K) {
    ids_out[tid] = id;
    wts_out[tid] = w;
    if (ids_lds) {
      ids_lds[tid] = id;
      wts_lds[tid] = w;
    }
  }
  team_sync<TEAM>();   // the scratch may be reused for the next token
}

// 1024 / TEAM teams per workgroup, one token each: four 256-thread teams, or
// sixteen one-wave teams for at most 64 experts (wave syncs, no workgroup
// barrier).
template <int MODE, int TEAM = 256>
__global__ __launch_bounds__(1024) void route_kernel(const float* __restrict__ logits,
                                                     const float* __restrict__ bias, int T, int E,
                                                     int K, int n_group, int topk_group,
                                                     float scale, int renorm,
                                                     int32_t* __restrict__ ids,
                                                     float* __restrict__ wts) {
  extern __shared__ float route_lds[];
  constexpr int kTeams = 1024 / TEAM;
  const int team = threadIdx.x / TEAM, tid = threadIdx.x % TEAM;
  const long t = (long)blockIdx.x * kTeams + team;
  const int nc = (MODE == 1 ? n_group : (E + 31) / 32) * K;
  const RouteScratch s(route_lds + team * route_team_words(E, nc), E, nc);
  route_token<MODE, TEAM>(logits + t * E, bias, E, K, n_group, topk_group, scale, renorm, s, tid,
                          t < T, ids + t * K, wts + t * K);
}

// The team router's launch: one-wave teams for E <= 64.
template <int MODE>
void launch_route_teams(const float* logits, const float* bias, int T, int E, int K, int n_group,
                        int topk_group, float scale, int renorm, int nc, int32_t* ids,
                        float* wts, hipStream_t stream) {
  const size_t words = route_team_words(E, nc) * sizeof(float);
  if (E <= kWave)
    route_kernel<MODE, kWave><<<(T + 15) / 16, 1024, 16 * words, stream>>>(
        logits, bias, T, E, K, n_group, topk_group, scale, renorm, ids, wts);
  else
    route_kernel<MODE, 256><<<(T + 3) / 4, 1024, 4 * words, stream>>>(
        logits, bias, T, E, K, n_group, topk_group, scale, renorm, ids, wts);
}

// Batches of any size on E = 256 / 512 (tiny::wave_epl): one wave routes one
// token with tiny::route_token_wave (no workgroup barrier), four tokens per
// workgroup.  Same ids, order and fp32 sequences as route_kernel.
template <int MODE, int EPL>
__global__ __launch_bounds__(256) void route_wave_kernel(const float* __restrict__ logits,
                                                         const float* __restrict__ bias, int T,
                                                         int K, int n_group, int topk_group,
                                                         float scale, int renorm,
                                                         int32_t* __restrict__ ids,
                                                         float* __restrict__ wts) {
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const long t = (long)blockIdx.x * 4 + w;
  if (t >= T) return;   // whole wave
  tiny::route_token_wave<MODE, EPL>(logits + t * (kWave * EPL), bias, K, n_group, topk_group,
                                    scale, renorm, threadIdx.x % kWave, ids + t * K, wts + t * K,
                                    nullptr, nullptr);
}

template <int MODE>
void launch_route_wave(int epl, const float* logits, const float* bias, int T, int K,
                       int n_group, int topk_group, float scale, int renorm, int32_t* ids,
                       float* wts, hipStream_t stream) {
  const dim3 grid((unsigned)((T + 3) / 4));
  if (epl == 4)
    route_wave_kernel<MODE, 4><<<grid, 256, 0, stream>>>(logits, bias, T, K, n_group, topk_group,
                                                         scale, renorm, ids, wts);
  else
    route_wave_kernel<MODE, 8><<<grid, 256, 0, stream>>>(logits, bias, T, K, n_group, topk_group,
                                                         scale, renorm, ids, wts);
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
  const int nrounds = min(kSegRounds, (a.A - base + kSegThreads - 1) / kSegThreads);
  for (int r = 0; r < nrounds; ++r) {
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
  const int nbits = 32 - __builtin_clz(a.NB - 1);   // bits of the largest bucket id (NB >= 2)
  // rounds holding pairs only (uniform: a short batch skips the empty ones)
  const int nrounds = min(kSegRounds, (a.A - base + kSegThreads - 1) / kSegThreads);
  for (int r = 0; r < nrounds; ++r) {
    const int p = base + r * kSegThreads + threadIdx.x;
    const bool valid = p < a.A;
    float w = 0.f;
    int tok = 0;
    const int bk = valid ? bucket_of(a, p, &w, &tok) : -1;
    // lanes of this wave that share my bucket: the valid lanes that agree
    // with mine on every bit of the bucket id (one ballot per bit)
    uint64_t m = __ballot(valid);
    for (int bit = 0; bit < nbits; ++bit) {
      const bool on = (bk >> bit) & 1;
      const uint64_t b1 = __ballot(valid && on);
      m &= on ? b1 : ~b1;
    }
    const int rank = __builtin_popcountll(m & lt_mask);
    const int wcount = __builtin_popcountll(m);
    const bool leader = valid && lane == __builtin_ctzll(m);
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

// Inclusive prefix sum across the 64 lanes of a wave (DPP row shifts, then
// row broadcasts); lanes whose source is out of range add 0.
__device__ __forceinline__ int wave_incl_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);   // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);   // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);   // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);   // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);   // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);   // row_bcast:31
  return x;
}

constexpr int kFewNB = 64;   // bucket count of the ballot segmentation

struct SegSmem {
  int ids[kSmallMaxA];
  float w[kSmallMaxA];
  int bk[kSmallMaxA];
  int cnt[kSmallMaxNB];
  int wsum[3][16];
  int wc[kFewNB][16];          // ballot segmentation: pairs of bucket v in wave q
  int bstart[kFewNB];
};

// Stable counting sort of the A <= NT pairs (pair p in thread p) over NB <=
// kFewNB buckets: per wave, one ballot per bucket gives each pair its rank
// among the wave's pairs of its bucket and the wave's count; one wave scans
// the bucket totals.  Position = bucket start + the bucket's pairs in
// earlier waves + rank: the same stable order as the counting sort.
template <int NT>
__device__ __forceinline__ void segment_few_buckets(const SmallArgs& a, SegSmem& g, int A, int TK,
                                                    int NB) {
  constexpr int NW = NT / kWave;
  const int tid = threadIdx.x, lane = tid % kWave, wv = tid / kWave;
  const int K = a.K, E = a.E, NS = a.NS;
  int b = -1;
  float w = 1.0f;
  if (tid < A) {
    if (tid < TK) {
      int e = g.ids[tid];
      w = g.w[tid];
      if (a.id_map && e >= 0 && e < E) e = a.id_map[e];
      b = (e < 0 || e >= E) ? (E + NS) : e;
      if (a.drop_zero && w == 0.0f) b = E + NS;
    } else {
      b = E + (tid - TK) % NS;
    }
  }
  int rank = 0;
  for (int v = 0; v < NB; ++v) {
    const unsigned long long m = __ballot(b == v);
    if (lane == 0) g.wc[v][wv] = __popcll(m);
    if (b == v)
      rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                       __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
  }
  __syncthreads();
  if (wv == 0) {
    // lane v: bucket v's rows, its start; active entries and tile lists
    int c = 0;
    if (lane < NB)
      for (int q = 0; q < NW; ++q) c += g.wc[lane][q];
    const int start = wave_incl_scan(c) - c;
    const bool live = lane < NB - 1 && c > 0;
    const unsigned long long am = __ballot(live);
    const int ai = __builtin_amdgcn_mbcnt_hi((uint32_t)(am >> 32),
                                             __builtin_amdgcn_mbcnt_lo((uint32_t)am, 0u));
    const int nt = (lane < NB - 1) ? (c + a.bm - 1) / a.bm : 0;
    const int tinc = wave_incl_scan(nt);
    const int t0 = tinc - nt;
    if (lane < NB) {
      g.bstart[lane] = start;
      a.seg_start[lane] = start;
      a.expert_tile_start[lane] = t0;
    }
    if (live) {
      a.active[ai] = lane;
      for (int j = 0; j < nt; ++j) {
        a.tile_expert[t0 + j] = lane;
        a.tile_row0[t0 + j] = start + j * a.bm;
      }
    }
    if (lane == 0) {
      const int n_til = __builtin_amdgcn_readlane(tinc, 63);
      a.seg_start[NB] = A;
      a.expert_tile_start[NB] = n_til;
      a.n_active[0] = __popcll(am);
      a.n_tiles[0] = n_til;
    }
  }
  __syncthreads();
  if (tid < A) {
    int pos = g.bstart[b] + rank;
    for (int q = 0; q < wv; ++q) pos += g.wc[b][q];
    a.sorted_pair[pos] = tid;
    a.inv[tid] = pos;
    a.sorted_tok[pos] = tid < TK ? tid / K : (tid - TK) / NS;
    a.sorted_wts[pos] = tid < TK ? w : 1.0f;
  }
}

// Softmax top-K of one token by one thread, for at most kLaneE experts and
// kLaneK choices: the selection scan in (score desc, index asc) order and
// the weights in the same fp32 sequence as route_token (e^(l_k - lmax), the
// sum over the K chosen in selection order, or over all E in index order
// without renormalisation; one correctly rounded division each).
constexpr int kLaneE = 32, kLaneK = 8;

__device__ __forceinline__ void route_token_lane(const float* __restrict__ l, int E, int K,
                                                 int renorm, int32_t* ids_out, float* wts_out,
                                                 int32_t* ids_lds, float* wts_lds) {
  float v[kLaneE];
#pragma unroll
  for (int e = 0; e < kLaneE; ++e) v[e] = e < E ? l[e] : 0.f;
  int sel[kLaneK];
  float sv[kLaneK];
  uint32_t used = 0u;
#pragma unroll
  for (int k = 0; k < kLaneK; ++k) {
    if (k < K) {
      int best = -1;
      float bv = 0.f;
#pragma unroll
      for (int e = 0; e < kLaneE; ++e) {
        if (e < E && !((used >> e) & 1u) && (best < 0 || better(v[e], e, bv, best))) {
          best = e;
          bv = v[e];
        }
      }
      sel[k] = best;
      sv[k] = bv;
      used |= 1u << best;
    }
  }
  const float lmax = sv[0];
  float ev[kLaneK];
  float sum = 0.0f;
#pragma unroll
  for (int k = 0; k < kLaneK; ++k) {
    if (k < K) {
      ev[k] = xtu_expf(sv[k] - lmax);
      sum = sum + ev[k];
    }
  }
  if (!renorm) {
    sum = 0.0f;
#pragma unroll
    for (int e = 0; e < kLaneE; ++e)
      if (e < E) sum = sum + xtu_expf(v[e] - lmax);
  }
#pragma unroll
  for (int k = 0; k < kLaneK; ++k) {
    if (k < K) {
      const float w = __fdiv_rn(ev[k], sum);
      ids_out[k] = sel[k];
      wts_out[k] = w;
      ids_lds[k] = sel[k];
      wts_lds[k] = w;
    }
  }
}

// One workgroup of NT threads.  MODE 0: softmax routing, 1: grouped sigmoid
// routing (NT/256 teams route that many tokens at a time; LANE: softmax over
// at most kLaneE experts, one thread per token), 2: ids/wts given.  Then the
// whole segmentation.
template <int MODE, int NT, bool LANE = false, bool FEW = false>
__global__ __launch_bounds__(NT) void route_seg_small_kernel(SmallArgs a) {
  __shared__ SegSmem g;
  extern __shared__ float route_lds[];
  constexpr int NW = NT / kWave;
  const int tid = threadIdx.x;
  const int T = a.T, K = a.K, E = a.E, NS = a.NS;
  const int TK = T * K, A = TK + T * NS, NB = E + NS + 1;
  if (MODE == 0 && LANE) {
    for (int t = tid; t < T; t += NT)
      route_token_lane(a.logits + (long)t * E, E, K, a.renorm, a.ids + (long)t * K,
                       a.wts + (long)t * K, g.ids + t * K, g.w + t * K);
  } else if (MODE < 2) {
    // NT / 256 teams of 256 threads route that many tokens at a time
    constexpr int NTEAM = NT / 256;
    const int team = tid / 256, ttid = tid % 256;
    const int nc = (MODE == 1 ? a.n_group : (E + 31) / 32) * K;
    const RouteScratch s(route_lds + team * route_team_words(E, nc), E, nc);
    for (int t0 = 0; t0 < T; t0 += NTEAM) {
      const int t = t0 + team;
      const bool valid = t < T;
      route_token<MODE < 2 ? MODE : 0, 256>(a.logits + (long)t * E, a.bias, E, K, a.n_group,
                                             a.topk_group, a.scale, a.renorm, s, ttid, valid,
                                             a.ids + (long)t * K, a.wts + (long)t * K,
                                             g.ids + t * K, g.w + t * K);
    }
  } else {
    for (int p = tid; p < TK; p += NT) {
      g.ids[p] = a.ids[p];
      g.w[p] = a.wts[p];
    }
  }
  if constexpr (FEW) {   // A <= NT pairs over NB <= kFewNB buckets
    __syncthreads();
    segment_few_buckets<NT>(a, g, A, TK, NB);
    return;
  }
  for (int e = tid; e < NB; e += NT) g.cnt[e] = 0;
  __syncthreads();
  for (int p = tid; p < A; p += NT) {
    int b;
    if (p < TK) {
      int e = g.ids[p];
      if (a.id_map && e >= 0 && e < E) e = a.id_map[e];
      b = (e < 0 || e >= E) ? (E + NS) : e;
      if (a.drop_zero && g.w[p] == 0.0f) b = E + NS;
    } else {
      b = E + (p - TK) % NS;
    }
    g.bk[p] = b;
    atomicAdd(&g.cnt[b], 1);
  }
  for (int p = A + tid; p < ((A + 3) & ~3); p += NT) g.bk[p] = -1;   // pad for 4-wide reads
  __syncthreads();
  // one scan pass over the buckets for (rows, active flag, tiles): each thread
  // owns `per` consecutive buckets
  const int per = (NB + NT - 1) / NT;
  const int lane = tid % kWave, wv = tid / kWave;
  int c_loc[8], s_rows = 0, s_act = 0, s_til = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int e = tid * per + i;
    const int c = (i < per && e < NB) ? g.cnt[e] : 0;
    c_loc[i] = c;
    s_rows += c;
    s_act += (e < NB - 1 && c > 0) ? 1 : 0;
    s_til += (e < NB - 1) ? (c + a.bm - 1) / a.bm : 0;
  }
  const int i_rows = wave_incl_scan(s_rows), i_act = wave_incl_scan(s_act),
            i_til = wave_incl_scan(s_til);
  if (lane == kWave - 1) {
    g.wsum[0][wv] = i_rows;
    g.wsum[1][wv] = i_act;
    g.wsum[2][wv] = i_til;
  }
  __syncthreads();
  int b_rows = i_rows - s_rows, b_act = i_act - s_act, b_til = i_til - s_til;
  int n_act = 0, n_til = 0;
#pragma unroll
  for (int q = 0; q < NW; ++q) {
    if (q < wv) {
      b_rows += g.wsum[0][q];
      b_act += g.wsum[1][q];
      b_til += g.wsum[2][q];
    }
    n_act += g.wsum[1][q];
    n_til += g.wsum[2][q];
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int e = tid * per + i;
    if (i < per && e < NB) {
      const int c = c_loc[i];
      a.seg_start[e] = b_rows;
      a.expert_tile_start[e] = b_til;
      g.cnt[e] = b_rows;   // bucket start, for the scatter below
      if (e < NB - 1 && c > 0) {
        a.active[b_act++] = e;
        const int nt = (c + a.bm - 1) / a.bm;
        for (int j = 0; j < nt; ++j) {
          a.tile_expert[b_til + j] = e;
          a.tile_row0[b_til + j] = b_rows + j * a.bm;
        }
        b_til += nt;
      }
      b_rows += c;
      if (e == NB - 1) {
        a.seg_start[NB] = A;
        a.expert_tile_start[NB] = n_til;
      }
    }
  }
  if (tid == 0) {
    a.n_active[0] = n_act;
    a.n_tiles[0] = n_til;
  }
  __syncthreads();
  // stable scatter: position = bucket start + earlier pairs of the bucket
  for (int p = tid; p < A; p += NT) {
    const int b = g.bk[p];
    int r = 0;
    int q = 0;
#pragma unroll 4
    for (; q + 4 <= p; q += 4) {
      const i32x4_t v = *reinterpret_cast<const i32x4_t*>(g.bk + q);
      r += (v[0] == b) + (v[1] == b) + (v[2] == b) + (v[3] == b);
    }
    for (; q < p; ++q) r += g.bk[q] == b;
    const int pos = g.cnt[b] + r;
    a.sorted_pair[pos] = p;
    a.inv[p] = pos;
    if (p < TK) {
      a.sorted_tok[pos] = p / K;
      a.sorted_wts[pos] = g.w[p];
    } else {
      a.sorted_tok[pos] = (p - TK) / NS;
      a.sorted_wts[pos] = 1.0f;
    }
  }
}

// Tiny batches: the whole routing + segmentation in one workgroup
// (tiny::route_segment_block).
template <int MODE, int EPL>
__global__ __launch_bounds__(1024) void route_seg_tiny_kernel(SmallArgs a) {
  __shared__ __attribute__((aligned(16))) tiny::TinySmem g;
  tiny::route_segment_block<MODE, EPL>(a, g);
}

template <int MODE>
hipError_t launch_small(const SmallArgs& a, hipStream_t stream) {
  const int epl = tiny::tiny_epl(a, MODE);
  // one wave per token, and one thread per bucket start for the last pass
  const int nb_waves = (a.E + a.NS + 2 + kWave - 1) / kWave;
  int tiny_waves = a.T > 4 ? a.T : 4;
  if (tiny_waves < nb_waves) tiny_waves = nb_waves < 16 ? nb_waves : 16;
  const int tiny_threads = kWave * tiny_waves;
  if (epl != 0) {
    if constexpr (MODE == 2) {
      route_seg_tiny_kernel<2, 1><<<1, tiny_threads, 0, stream>>>(a);
    } else {
      if (epl == 4) route_seg_tiny_kernel<MODE, 4><<<1, tiny_threads, 0, stream>>>(a);
      else route_seg_tiny_kernel<MODE, 8><<<1, tiny_threads, 0, stream>>>(a);
    }
    return hipSuccess;
  }
  // few buckets: the ballot segmentation, one pair per thread
  const long A = (long)a.T * a.K + (long)a.T * a.NS;
  const bool few = a.E + a.NS + 1 <= kFewNB && A <= 1024;
  if constexpr (MODE == 2) {
    if (few && A <= 256) route_seg_small_kernel<2, 256, false, true><<<1, 256, 0, stream>>>(a);
    else if (few) route_seg_small_kernel<2, 1024, false, true><<<1, 1024, 0, stream>>>(a);
    else route_seg_small_kernel<MODE, 256><<<1, 256, 0, stream>>>(a);
  } else if (MODE == 0 && a.E <= kLaneE && a.K <= kLaneK && few) {
    // few experts and few buckets (shared experts included): one thread per
    // token, no routing barriers, the ballot segmentation
    if (A <= 256) route_seg_small_kernel<0, 256, true, true><<<1, 256, 0, stream>>>(a);
    else route_seg_small_kernel<0, 1024, true, true><<<1, 1024, 0, stream>>>(a);
  } else {
    const int nc = (MODE == 1 ? a.n_group : (a.E + 31) / 32) * a.K;
    const size_t team_lds = route_team_words(a.E, nc) * sizeof(float);
    if (a.T <= 2)   // one team: fewer waves in lockstep through the barriers
      route_seg_small_kernel<MODE, 256><<<1, 256, team_lds, stream>>>(a);
    else
      route_seg_small_kernel<MODE, 1024><<<1, 1024, 4 * team_lds, stream>>>(a);
  }
  return hipSuccess;
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
  if (const int epl = tiny::wave_epl(0, E, 1, renormalize, logits, nullptr)) {
    launch_route_wave<0>(epl, logits, nullptr, T, K, 1, 1, 1.0f, renormalize, topk_ids,
                         topk_weights, stream);
    return hipPeekAtLastError();
  }
  launch_route_teams<0>(logits, nullptr, T, E, K, 1, 1, 1.0f, renormalize, ((E + 31) / 32) * K,
                       topk_ids, topk_weights, stream);
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
  if (const int epl = tiny::wave_epl(1, E, n_group, renormalize, logits, bias)) {
    launch_route_wave<1>(epl, logits, bias, T, K, n_group, topk_group, routed_scaling,
                         renormalize, topk_ids, topk_weights, stream);
    return hipPeekAtLastError();
  }
  launch_route_teams<1>(logits, bias, T, E, K, n_group, topk_group, routed_scaling, renormalize,
                       n_group * K, topk_ids, topk_weights, stream);
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

}  // extern "C"

namespace xtu {
namespace {

// The three segmentation launches over a caller-supplied workspace of
// xtu_segment_workspace_bytes() bytes (every word written by seg_hist_kernel
// before seg_scan_kernel reads it, so it needs no clearing).
hipError_t segment_impl(const int32_t* topk_ids, const float* topk_weights,
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

// Device address of `scratch` on the current device, looked up once per
// device (hipGetSymbolAddress with that device current) and kept.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

hipError_t scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}

}  // namespace
}  // namespace xtu

extern "C" {

hipError_t xtu_segment(const int32_t* topk_ids, const float* topk_weights,
                       const int32_t* id_map, int T, int K, int E, int n_shared, int drop_zero,
                       int bm, void* workspace, int32_t* sorted_pair, int32_t* sorted_tok,
                       float* sorted_wts, int32_t* inv, int32_t* seg_start, int32_t* active,
                       int32_t* n_active, int32_t* tile_expert, int32_t* tile_row0,
                       int32_t* n_tiles, int32_t* expert_tile_start, hipStream_t stream) {
  return segment_impl(topk_ids, topk_weights, id_map, T, K, E, n_shared, drop_zero, bm,
                      workspace, sorted_pair, sorted_tok, sorted_wts, inv, seg_start, active,
                      n_active, tile_expert, tile_row0, n_tiles, expert_tile_start, stream);
}

hipError_t xtu_segment_noalloc(const int32_t* topk_ids, const float* topk_weights,
                               const int32_t* id_map, int T, int K, int E, int n_shared,
                               int drop_zero, int bm, int32_t* sorted_pair, int32_t* sorted_tok,
                               float* sorted_wts, int32_t* inv, int32_t* seg_start,
                               int32_t* active, int32_t* n_active, int32_t* tile_expert,
                               int32_t* tile_row0, int32_t* n_tiles, int32_t* expert_tile_start,
                               hipStream_t stream) {
  XTU_CHECK_ARG(T >= 0 && K >= 0 && E > 0 && n_shared >= 0);
  const size_t need = xtu_segment_workspace_bytes(T, K, E, n_shared);
  if (need > kNoAllocScratchBytes) {
    fprintf(stderr,
            "xtu_segment_noalloc: T=%d K=%d E=%d n_shared=%d needs %zu bytes of workspace, more "
            "than the %zu-byte static scratch; use xtu_segment with a workspace\n",
            T, K, E, n_shared, need, kNoAllocScratchBytes);
    return hipErrorInvalidValue;
  }
  void* ws = nullptr;
  const hipError_t e = scratch_address(&ws);
  if (e != hipSuccess) return e;
  return segment_impl(topk_ids, topk_weights, id_map, T, K, E, n_shared, drop_zero, bm, ws,
                      sorted_pair, sorted_tok, sorted_wts, inv, seg_start, active, n_active,
                      tile_expert, tile_row0, n_tiles, expert_tile_start, stream);
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
  if (mode < 2 && T == 0) mode = 2;   // nothing to route: segment the empty batch
  SmallArgs a{logits, bias, topk_ids, topk_weights, id_map, T, K, E, n_group, topk_group,
              renormalize, n_shared, drop_zero, bm, routed_scaling, sorted_pair, sorted_tok, inv,
              seg_start, active, n_active, sorted_wts, tile_expert, tile_row0, n_tiles,
              expert_tile_start};
  (void)hipGetLastError();
  hipError_t err;
  if (mode == 0) err = launch_small<0>(a, stream);
  else if (mode == 1) err = launch_small<1>(a, stream);
  else err = launch_small<2>(a, stream);
  return err != hipSuccess ? err : hipPeekAtLastError();
}

}  // extern "C"
