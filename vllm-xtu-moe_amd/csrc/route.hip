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

// wave argmax of (s, i) pairs under `better`; every lane gets the winner.
__device__ __forceinline__ void wave_argmax(float& s, int& i) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float os = __shfl_xor(s, off, kWave);
    const int oi = __shfl_xor(i, off, kWave);
    if (better(os, oi, s, i)) {
      s = os;
      i = oi;
    }
  }
}

// MODE 0: softmax top-k (renormalised or not).  MODE 1: grouped sigmoid.
template <int MODE>
__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits,
                                                    const float* __restrict__ bias, int T, int E,
                                                    int K, int n_group, int topk_group,
                                                    float scale, int renorm,
                                                    int32_t* __restrict__ ids,
                                                    float* __restrict__ wts) {
  __shared__ float sb[4][1024];   // selection score per expert, per wave
  const int wv = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int t = blockIdx.x * 4 + wv;
  if (t >= T) return;
  const float* l = logits + (size_t)t * E;
  const float NEG = -__builtin_inff();
  float sel_score[kMaxPerLane];   // selection score (logit, or sigmoid+bias)
  float wt_score[kMaxPerLane];    // weight score (sigmoid) for MODE 1
  const int nper = (E + kWave - 1) / kWave;
#pragma unroll
  for (int j = 0; j < kMaxPerLane; ++j) {
    const int e = lane + kWave * j;
    float v = NEG, w = 0.f;
    if (j < nper && e < E) {
      const float x = l[e];
      if (MODE == 0) {
        v = x;
      } else {
        w = xtu_sigmoid(x);
        v = w + (bias ? bias[e] : 0.0f);
      }
      sb[wv][e] = v;
    }
    sel_score[j] = v;
    wt_score[j] = w;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");

  // group mask (MODE 1): bit j set when group j is kept
  uint64_t gmask = ~0ull;
  int gsz = E;
  if (MODE == 1) {
    gsz = E / n_group;
    float g = NEG;
    if (lane < n_group) {
      int i1 = -1, i2 = -1;
      for (int q = 0; q < gsz; ++q) {
        const int e = lane * gsz + q;
        const float v = sb[wv][e];
        if (i1 < 0 || better(v, e, sb[wv][i1], i1)) {
          i2 = i1;
          i1 = e;
        } else if (i2 < 0 || better(v, e, sb[wv][i2], i2)) {
          i2 = e;
        }
      }
      g = (gsz >= 2) ? (sb[wv][i1] + sb[wv][i2]) : sb[wv][i1];
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

  float chosen_w[16];
  float chosen_s[16];
  int chosen_i[16];
  uint32_t used = 0;   // bit j: this lane's expert lane+64j already chosen
  for (int k = 0; k < K; ++k) {
    float s = NEG;
    int i = 0x7fffffff;
    float w = 0.f;
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j) {
      const int e = lane + kWave * j;
      if (j < nper && e < E && !((used >> j) & 1u) && ((gmask >> (e / gsz)) & 1ull)) {
        if (better(sel_score[j], e, s, i)) {
          s = sel_score[j];
          i = e;
          w = wt_score[j];
        }
      }
    }
    wave_argmax(s, i);
    // the owner of the winner marks it and broadcasts its weight score
    const int owner = i % kWave;
    if (lane == owner) used |= 1u << (i / kWave);
    float wsc = 0.f;
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j)
      if (lane == owner && lane + kWave * j == i) wsc = wt_score[j];
    wsc = __shfl(wsc, owner, kWave);
    (void)w;
    if (k < 16) {
      chosen_s[k] = s;
      chosen_w[k] = wsc;
      chosen_i[k] = i;
    }
  }
  if (lane != 0) return;
  {
#pragma clang fp contract(off)
  if (MODE == 0) {
    const float lmax = chosen_s[0];
    float ev[16];
    float sum = 0.0f;
    for (int k = 0; k < K; ++k) {
      ev[k] = xtu_expf(chosen_s[k] - lmax);
      sum = sum + ev[k];
    }
    if (!renorm) {
      sum = 0.0f;
      for (int e = 0; e < E; ++e) sum = sum + xtu_expf(l[e] - lmax);
    }
    for (int k = 0; k < K; ++k) {
      ids[(size_t)t * K + k] = chosen_i[k];
      wts[(size_t)t * K + k] = __fdiv_rn(ev[k], sum);
    }
  } else {
    float sum = 0.0f;
    for (int k = 0; k < K; ++k) sum = sum + chosen_w[k];
    for (int k = 0; k < K; ++k) {
      ids[(size_t)t * K + k] = chosen_i[k];
      wts[(size_t)t * K + k] =
          renorm ? __fdiv_rn(chosen_w[k], sum) * scale : chosen_w[k] * scale;
    }
  }
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
  route_kernel<0><<<(T + 3) / 4, 256, 0, stream>>>(logits, nullptr, T, E, K, 1, 1, 1.0f,
                                                   renormalize, topk_ids, topk_weights);
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
  route_kernel<1><<<(T + 3) / 4, 256, 0, stream>>>(logits, bias, T, E, K, n_group, topk_group,
                                                   routed_scaling, renormalize, topk_ids,
                                                   topk_weights);
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

}  // extern "C"
