// Routing and segmentation of tiny batches (at most 64 (token, expert)
// pairs) by one workgroup: the one-launch router (route.hip) and the decode
// launch that routes while other workgroups run the shared experts'
// gate/up (decode.hip).
#pragma once

#include "xtu_common.hpp"

namespace xtu {
namespace tiny {

constexpr int kWave = 64;

__device__ __forceinline__ bool better(float sa, int ia, float sb, int ib) {
  return (sa > sb) || (sa == sb && ia < ib);
}

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

// Arguments of the one-launch routing + segmentation (xtu_route_segment_small).
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

// ---------------------------------------------------------------------------
// Tiny batches (at most 64 pairs; routing for E = 64 * EPL, EPL = 4 or 8): one
// wave routes one token with no workgroup barrier.  Lane l holds experts
// [l*EPL, (l+1)*EPL) and sorts them by (score desc, index asc) once; the K
// choices are taken in K rounds of a wave-wide maximum of the lanes' first
// order-preserving score keys; equal scores go to the lowest lane, whose
// first entry is its lowest index among them, so the order is (score desc,
// index asc) as in route_token.  Group scores (top two over a group's lanes)
// and group ranks follow route_token's definitions; the weights use its fp32
// sequences.  The segmentation of the <= 64 pairs works on the pair buckets
// staged in LDS with fixed-length loops.
// ---------------------------------------------------------------------------
constexpr int kTinyMaxA = 64;

// Larger score -> larger key; -0 and +0 share a key.
__device__ __forceinline__ uint32_t score_key(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) == 0u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Maximum over the wave (DPP row shifts and broadcasts; lane 63 ends with
// the maximum of all lanes), returned to every lane.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xF, 0xF, false));
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xF, 0xF, false));
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xF, 0xF, false));
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xF, 0xF, false));
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xA, 0xF, false));
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xC, 0xF, false));
  return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}

// Order this wave's LDS writes before its later LDS reads by other lanes:
// a wave's LDS instructions execute in issue order, so only the compiler
// must not move them (no wait for outstanding global stores).
__device__ __forceinline__ void lds_wave_order() {
  __builtin_amdgcn_wave_barrier();
  __asm__ __volatile__("" ::: "memory");
}

// Top two of (v1 >= v2) pairs over aligned groups of lpg lanes (1..64).
__device__ __forceinline__ void top2_merge(float& v1, float& v2, float b1, float b2) {
  const float n1 = fmaxf(v1, b1), n2 = fmaxf(fminf(v1, b1), fmaxf(v2, b2));
  v1 = n1;
  v2 = n2;
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ void group_top2(float& v1, float& v2, int lpg) {
  // partner lanes within a quad (xor 1, xor 2), then the mirrored quad of the
  // 8-lane half row, then the mirrored half of the 16-lane row, then across rows
  if (lpg >= 2) top2_merge(v1, v2, dpp_f<0xB1>(v1), dpp_f<0xB1>(v2));     // quad_perm [1,0,3,2]
  if (lpg >= 4) top2_merge(v1, v2, dpp_f<0x4E>(v1), dpp_f<0x4E>(v2));     // quad_perm [2,3,0,1]
  if (lpg >= 8) top2_merge(v1, v2, dpp_f<0x141>(v1), dpp_f<0x141>(v2));   // row_half_mirror
  if (lpg >= 16) top2_merge(v1, v2, dpp_f<0x140>(v1), dpp_f<0x140>(v2));  // row_mirror
  for (int o = 16; o < lpg; o <<= 1) top2_merge(v1, v2, __shfl_xor(v1, o, 64), __shfl_xor(v2, o, 64));
}

__device__ __forceinline__ float readlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Compare-exchange for a descending order: a gets the larger word.
__device__ __forceinline__ void cas_desc(uint64_t& a, uint64_t& b) {
  const uint64_t hi = a > b ? a : b, lo = a > b ? b : a;
  a = hi;
  b = lo;
}

// Descending sort of EPL words in registers: the optimal networks for 4 and
// 8 (5 and 19 compare-exchanges), odd-even transposition otherwise.
template <int EPL>
__device__ __forceinline__ void sort_desc(uint64_t (&c)[EPL]) {
  if constexpr (EPL != 4 && EPL != 8) {
#pragma unroll
    for (int r = 0; r < EPL; ++r)
#pragma unroll
      for (int i = r % 2; i + 1 < EPL; i += 2) cas_desc(c[i], c[i + 1]);
  } else if constexpr (EPL == 4) {
    cas_desc(c[0], c[1]); cas_desc(c[2], c[3]);
    cas_desc(c[0], c[2]); cas_desc(c[1], c[3]);
    cas_desc(c[1], c[2]);
  } else {
    cas_desc(c[0], c[2]); cas_desc(c[1], c[3]); cas_desc(c[4], c[6]); cas_desc(c[5], c[7]);
    cas_desc(c[0], c[4]); cas_desc(c[1], c[5]); cas_desc(c[2], c[6]); cas_desc(c[3], c[7]);
    cas_desc(c[0], c[1]); cas_desc(c[2], c[3]); cas_desc(c[4], c[5]); cas_desc(c[6], c[7]);
    cas_desc(c[2], c[4]); cas_desc(c[3], c[5]);
    cas_desc(c[1], c[4]); cas_desc(c[3], c[6]);
    cas_desc(c[1], c[2]); cas_desc(c[3], c[4]); cas_desc(c[5], c[6]);
  }
}

template <int MODE, int EPL>
__device__ void route_token_wave(const float* __restrict__ l, const float* __restrict__ bias,
                                 int K, int n_group, int topk_group, float scale, int renorm,
                                 int lane, int32_t* ids_out, float* wts_out, int* ids_lds,
                                 float* wts_lds) {
#pragma clang fp contract(off)
  constexpr int E = kWave * EPL;
  const int e0 = lane * EPL;
  float x[EPL], bi[EPL], ws[EPL], sc[EPL];
  uint32_t key[EPL];
#pragma unroll
  for (int j = 0; j < EPL; j += 4) {
    const f32x4_t v = *reinterpret_cast<const f32x4_t*>(l + e0 + j);
    f32x4_t bv = {0.f, 0.f, 0.f, 0.f};
    if (MODE == 1 && bias) bv = *reinterpret_cast<const f32x4_t*>(bias + e0 + j);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      x[j + q] = v[q];
      bi[j + q] = bv[q];
    }
  }
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    if (MODE == 0) {
      ws[j] = x[j];
      sc[j] = x[j];
    } else {
      ws[j] = xtu_sigmoid(x[j]);
      sc[j] = ws[j] + bi[j];
    }
    key[j] = score_key(sc[j]);
  }
  if (MODE == 1) {
    // group score: best + second best over the group's lanes; keep the
    // topk_group best groups (rank under (score desc, group asc))
    const float NEG = -__builtin_inff();
    const int gsz = E / n_group, lpg = gsz / EPL;
    float v1 = NEG, v2 = NEG;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      if (sc[j] > v1) {
        v2 = v1;
        v1 = sc[j];
      } else if (sc[j] > v2) {
        v2 = sc[j];
      }
    }
    group_top2(v1, v2, lpg);
    const float gs = gsz >= 2 ? v1 + v2 : v1;
    const int my_g = lane / lpg;
    int r = 0;
    for (int j = 0; j < n_group; ++j) r += better(readlane_f(gs, j * lpg), j, gs, my_g) ? 1 : 0;
    if (r >= topk_group) {
#pragma unroll
      for (int j = 0; j < EPL; ++j) key[j] = 0u;
    }
  }
  // Each lane sorts its EPL entries by (key desc, index asc) once (a sorting
  // network over 64-bit (key, EPL - 1 - index) words), so a round takes the
  // lane's head instead of rescanning: round k takes the wave's largest head
  // (the lowest lane among equal ones), and the winning lane drops its head.
  uint64_t c[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) c[j] = (uint64_t)key[j] << 32 | (uint32_t)(EPL - 1 - j);
  sort_desc<EPL>(c);
  uint32_t hk[EPL];   // keys in order
  uint32_t jpk = 0u;  // index of entry i at bits [4i, 4i + 4)
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    hk[i] = (uint32_t)(c[i] >> 32);
    jpk |= (uint32_t)(EPL - 1 - (int)(uint32_t)c[i]) << (4 * i);
  }
  int my_e = 0;
  for (int k = 0; k < K; ++k) {
    const uint32_t gmax = wave_max_u32(hk[0]);
    const unsigned long long m = __ballot(hk[0] == gmax);
    const int wl = __builtin_ctzll(m);
    const int ek = wl * EPL + (__builtin_amdgcn_readlane((int)jpk, wl) & 15);
    if (lane == k) my_e = ek;
    if (lane == wl) {
#pragma unroll
      for (int i = 0; i + 1 < EPL; ++i) hk[i] = hk[i + 1];
      hk[EPL - 1] = 0u;
      jpk >>= 4;
    }
  }
  // the chosen expert's unbiased score, from the lane that holds it
  float my_ws = 0.f;
  {
    const int src = my_e / EPL, js = my_e % EPL;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const float v = __shfl(ws[j], src, kWave);
      if (j == js) my_ws = v;
    }
    if (lane >= K) my_ws = 0.f;
  }
  float w = 0.f;
  if (MODE == 0) {
    const float lmax = readlane_f(my_ws, 0);
    const float ev = lane < K ? xtu_expf(my_ws - lmax) : 0.f;
    float sum = 0.0f;
    for (int k = 0; k < K; ++k) sum = sum + readlane_f(ev, k);
    w = __fdiv_rn(ev, sum);
  } else {
    float sum = 0.0f;
    for (int k = 0; k < K; ++k) sum = sum + readlane_f(my_ws, k);
    w = renorm ? __fdiv_rn(my_ws, sum) * scale : my_ws * scale;
  }
  if (lane < K) {
    if (ids_out) {
      ids_out[lane] = my_e;
      wts_out[lane] = w;
    }
    if (ids_lds) {
      ids_lds[lane] = my_e;
      wts_lds[lane] = w;
    }
  }
}

// Entries of v[0, 4 NQ) below x (the words past the live ones hold INT_MAX,
// so only the first 4 NQ are read when the live ones are fewer).
template <int NQ>
__device__ __forceinline__ int count_below(const int* v, int x) {
  int n = 0;
#pragma unroll
  for (int q = 0; q < 4 * NQ; q += 4) {
    const i32x4_t u = *reinterpret_cast<const i32x4_t*>(v + q);
    n += (u[0] < x) + (u[1] < x) + (u[2] < x) + (u[3] < x);
  }
  return n;
}

struct TinySmem {
  int ids[kTinyMaxA];
  float w[kTinyMaxA];
  int bk[kTinyMaxA];          // sort key of pair p: bucket * 64 + p (INT_MAX past A)
  int sb[kTinyMaxA];          // bucket at sorted position j (INT_MAX past A)
  int act_b[kTinyMaxA + 4];   // active buckets, ascending (INT_MAX past n_act)
  int act_r[kTinyMaxA + 1];   // first row of active bucket i; [n_act] = trash start
  int act_t[kTinyMaxA + 1];   // first tile of active bucket i; [n_act] = all tiles
  int n_act;
  // the same segmentation as the global outputs, for the workgroup's own use
  int stok[kTinyMaxA];        // token of sorted row j
  int tile_e[kTinyMaxA];      // bucket of tile t
  int tile_r[kTinyMaxA];      // first sorted row of tile t
  int tile_n[kTinyMaxA];      // rows of tile t (at most bm)
  float sw[kTinyMaxA];        // weight of sorted row j (1 for a shared expert's)
};

// MODE 0/1: wave w routes tokens w, w + waves, ... (E = 64 * EPL), then the
// segmentation; MODE 2: ids/wts given.  One workgroup of at least one wave;
// the last pass writes one bucket start per thread (any block size is
// correct).
// STORE = false: nothing is written to global memory, only the segmentation
// in g (the LDS copy every caller gets: sorted tokens and the tile map),
// so any number of workgroups can route the same batch for themselves and
// agree (the same code on the same inputs).
template <int MODE, int EPL, bool STORE = true>
__device__ void route_segment_block(const SmallArgs& a, TinySmem& g) {
  const int tid = threadIdx.x, lane = tid % kWave, wv = tid / kWave;
  const int T = a.T, K = a.K, E = a.E, NS = a.NS;
  const int TK = T * K, A = TK + T * NS, NB = E + NS + 1, trash = E + NS;
  constexpr int BIG = 0x7fffffff;
  if (MODE < 2) {
    const int nw = blockDim.x / kWave;   // a wave routes tokens wv, wv + nw, ...
    for (int t = wv; t < T; t += nw)
      route_token_wave<MODE, EPL>(a.logits + (long)t * E, a.bias, K, a.n_group, a.topk_group,
                                  a.scale, a.renorm, lane,
                                  STORE ? a.ids + (long)t * K : nullptr,
                                  STORE ? a.wts + (long)t * K : nullptr, g.ids + t * K,
                                  g.w + t * K);
  } else {
    for (int p = tid; p < TK; p += blockDim.x) {
      g.ids[p] = a.ids[p];
      g.w[p] = a.wts[p];
    }
  }
  __syncthreads();
  if (wv == 0) {
    // token of pair `lane` (routed pairs t*K + k, then shared ones
    // TK + t*NS + s), counted over the batch's tokens instead of divided
    const int pr = lane < TK ? lane : lane - TK, per = lane < TK ? K : NS;
    int tk = 0;
    for (int t = 1; t < T; ++t) tk += pr >= t * per ? 1 : 0;
    // bucket of pair `lane`
    int b = BIG;
    float w = 1.0f;
    if (lane < TK) {
      int e = g.ids[lane];
      w = g.w[lane];
      if (a.id_map && e >= 0 && e < E) e = a.id_map[e];
      b = (e < 0 || e >= E) ? trash : e;
      if (a.drop_zero && w == 0.0f) b = trash;
    } else if (lane < A) {
      b = E + (pr - tk * per);
    }
    // stable position: rank of the unique key (bucket, pair) among the pairs
    const int key = lane < A ? b * kTinyMaxA + lane : BIG;
    g.bk[lane] = key;
    lds_wave_order();
    const int pos = A <= 16 ? count_below<4>(g.bk, key)
                            : A <= 32 ? count_below<8>(g.bk, key) : count_below<16>(g.bk, key);
    if (lane < A) {
      g.sb[pos] = b;
      g.stok[pos] = tk;
      g.sw[pos] = w;
      if constexpr (STORE) {
        a.sorted_pair[pos] = lane;
        a.inv[lane] = pos;
        a.sorted_tok[pos] = tk;
        a.sorted_wts[pos] = w;
      }
    } else {
      g.sb[lane] = BIG;
    }
    lds_wave_order();
    // sorted position `lane`: the first of its bucket opens an active entry;
    // the bucket's size runs to the next bucket's first row (or A)
    const int sbj = g.sb[lane];
    const int prev = lane > 0 ? g.sb[lane - 1] : -1;
    const bool start = lane < A && sbj != prev;
    const unsigned long long bnd = __ballot(start);
    const unsigned long long above = lane == 63 ? 0ull : bnd & (~0ull << (lane + 1));
    const int cnt = (above ? __builtin_ctzll(above) : A) - lane;
    const bool first = start && sbj != trash;
    const unsigned long long fm = __ballot(first);
    const int ai = __builtin_amdgcn_mbcnt_hi((uint32_t)(fm >> 32),
                                             __builtin_amdgcn_mbcnt_lo((uint32_t)fm, 0u));
    const int na = __popcll(fm);
    const int nt = !first ? 0 : A <= a.bm ? 1 : (cnt + a.bm - 1) / a.bm;
    const int incl = wave_incl_scan(nt);
    const int t0 = incl - nt;
    if (first) {
      g.act_b[ai] = sbj;
      g.act_r[ai] = lane;
      g.act_t[ai] = t0;
      if constexpr (STORE) a.active[ai] = sbj;
      for (int j = 0; j < nt; ++j) {
        if constexpr (STORE) {
          a.tile_expert[t0 + j] = sbj;
          a.tile_row0[t0 + j] = lane + j * a.bm;
        }
        if (t0 + j < kTinyMaxA) {   // bm >= 1: at most A <= 64 tiles
          g.tile_e[t0 + j] = sbj;
          g.tile_r[t0 + j] = lane + j * a.bm;
          g.tile_n[t0 + j] = min(a.bm, cnt - j * a.bm);
        }
      }
    }
    // rows before the trash bucket (= pairs in active buckets)
    const unsigned long long tm = __ballot(lane < A && sbj != trash);
    if (lane == 0) {
      const int tot = __builtin_amdgcn_readlane(incl, 63);
      g.n_act = na;
      g.act_r[na] = __popcll(tm);
      g.act_t[na] = tot;
      if constexpr (STORE) {
        a.n_active[0] = na;
        a.n_tiles[0] = tot;
      }
    }
    if (lane >= na && lane < kTinyMaxA + 4) g.act_b[lane] = BIG;
    if (lane < 4) g.act_b[kTinyMaxA + lane] = BIG;
  }
  __syncthreads();
  if constexpr (!STORE) return;
  // per-bucket starts: i = active buckets below e; rows and tiles before e
  const int na = g.n_act;
  for (int e = tid; e <= NB; e += blockDim.x) {
    const int i = na <= 16 ? count_below<4>(g.act_b, e)
                           : na <= 32 ? count_below<8>(g.act_b, e) : count_below<16>(g.act_b, e);
    a.seg_start[e] = e == NB ? A : g.act_r[i];
    a.expert_tile_start[e] = g.act_t[i];
  }
}

// Experts per lane of route_token_wave for this router (0: outside its
// envelope): E = 256 or 512, whole lanes per group, renormalised softmax,
// 16-byte-aligned logit and bias rows.
__host__ inline int wave_epl(int mode, int E, int n_group, int renorm, const float* logits,
                             const float* bias) {
  const int epl = E / kWave;
  if (E % kWave != 0 || (epl != 4 && epl != 8)) return 0;
  if (reinterpret_cast<uintptr_t>(logits) % 16 != 0 ||
      (bias && reinterpret_cast<uintptr_t>(bias) % 16 != 0))
    return 0;
  if (mode == 0) return renorm != 0 ? epl : 0;
  if (n_group <= 0 || E % n_group != 0) return 0;
  const int gsz = E / n_group;
  if (gsz % epl != 0) return 0;
  const int lpg = gsz / epl;
  return (lpg >= 1 && lpg <= kWave && (lpg & (lpg - 1)) == 0) ? epl : 0;
}

// The tiny path's envelope: at most 64 pairs and 16 tokens, and the wave
// router's (mode 2, ids given, routes nothing).
__host__ inline int tiny_epl(const SmallArgs& a, int mode) {
  const long A = (long)a.T * a.K + (long)a.T * a.NS;
  if (A > kTinyMaxA || a.T > 16) return 0;
  if (mode == 2) return 1;
  if (a.T < 1) return 0;
  return wave_epl(mode, a.E, a.n_group, a.renorm, a.logits, a.bias);
}


}  // namespace tiny
}  // namespace xtu
