// The one-launch decode layer (decode_layer_kernel): routing, gate/up, a
// grid barrier and the down projection with the weighted combine.
#include <map>
#include <mutex>
#include <tuple>

#include "decode.hpp"

namespace xtu {
namespace {

// ---------------------------------------------------------------------------
// A whole decode layer in one launch: route_gate_up_phase (every workgroup
// routes the batch in LDS; the shared-expert ones after their gate/up item),
// a grid-wide barrier, then the down projection with the weighted combine --
// decode_down_combine_kernel's arithmetic and summation order, its tables
// built from the routing each workgroup holds in LDS instead of the global
// segmentation.  The host launches one resident round (the occupancy query
// sizes the grid), so every workgroup reaches the barrier; each issues the
// weights of its first down panel's first D experts before it waits, so the
// down stream starts while the last gate/up items finish.  Workgroups past
// the down panels leave after the barrier.

// Grid barrier of the launch.  Words (uint32, each on its own 256-byte line):
// group arrival counters at 64 g (g = workgroup % 8, the XCD it runs on),
// the group count at 64 * 8, per-group generations at 64 (9 + g), and a flag
// at 64 * 17 set when a wait ran out.  A workgroup arrives on its group's
// counter; the group's last arrival arrives on the group count, whose last
// arrival bumps every group's generation; waiters poll their group's word.
// Few atomics meet on one address, and pollers spread over eight lines.
// Every counter is reset by its last arrival, so the words are back to zero
// (generations aside) after each use and need clearing once, before the
// first.  The data crossing the barrier (the act rows) is written and read
// with device-coherent accesses (agent scope), so no cache write-back or
// invalidation is needed: each wave's stores complete before its workgroup
// arrives, and the reads are issued after the generation changed.
constexpr int kBarWords = 64 * 18;
constexpr int kBarSpin = 1 << 17;   // polls of about 1 us each before giving up

// The group's generation before this launch's barrier, read by thread 0 at
// the start of the launch: it cannot move before every workgroup, this one
// included, has arrived, so reading it early keeps a memory round trip off
// the last arrival's path.
__device__ __forceinline__ unsigned barrier_generation(const unsigned* bar) {
  return threadIdx.x == 0 ? __hip_atomic_load(bar + 64 * (9 + blockIdx.x % 8), __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT)
                          : 0u;
}

__device__ __forceinline__ void barrier_arrive(unsigned* bar) {
  __builtin_amdgcn_s_waitcnt(0);   // this wave's act stores are complete
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned g = blockIdx.x % 8, ngroups = gridDim.x < 8 ? gridDim.x : 8;
    const unsigned in_g = (gridDim.x - g + 7) / 8;
    if (__hip_atomic_fetch_add(bar + 64 * g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
        in_g - 1) {
      __hip_atomic_store(bar + 64 * g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (__hip_atomic_fetch_add(bar + 64 * 8, 1u, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT) == ngroups - 1) {
        __hip_atomic_store(bar + 64 * 8, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (unsigned h = 0; h < ngroups; ++h)
          __hip_atomic_fetch_add(bar + 64 * (9 + h), 1u, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

// Thread 0 polls its group's generation until it moves past gen (bounded: a
// launch that could not be resident ends with a flag, not a hang).
__device__ __forceinline__ void barrier_wait(unsigned* bar, unsigned gen) {
  if (threadIdx.x == 0) {
    const unsigned* w = bar + 64 * (9 + blockIdx.x % 8);
    for (int n = 0; __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gen;
         ++n) {
      if (n == kBarSpin) {
        __hip_atomic_store(bar + 64 * 17, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  __syncthreads();
}

constexpr int kLayerStageSB = 8;   // act pieces per thread in flight while staging
constexpr int kAuxDevice = 16;     // buffer access cache policy: device scope (sc1)

template <int FMT, int MODE, int EPL, int XC, int NPER>
__global__ __launch_bounds__(512) void decode_layer_kernel(tiny::SmallArgs ra, DecodeArgs a,
                                                           DownCombineArgs d, void* act_sh,
                                                           int n_sh, int skip, unsigned* bar) {
  using F = WFmt<FMT>;
  // experts in flight per wave: as many as keep the kernel within 128 VGPRs
  // (four waves per SIMD), so most of a decode batch's experts are loaded
  // while the workgroup waits at the barrier
  constexpr int D = FMT == kMXFP4 ? (NPER == 1 ? 6 : 5) : (FMT == kBF16 ? 2 : 3);
  extern __shared__ __attribute__((aligned(16))) uint8_t dyn[];
  __shared__ f32x4_t red[8][kWave];
  __shared__ __attribute__((aligned(16))) tiny::TinySmem g;
  const unsigned gen = barrier_generation(bar);
  route_gate_up_phase<FMT, MODE, EPL, XC, true>(ra, a, act_sh, n_sh, skip,
                                               reinterpret_cast<uint16_t*>(dyn), red, g);

  const int tid = threadIdx.x, bd = blockDim.x;
  const int w = wave_id();
  const uint32_t lane = tid % kWave;
  const int q = lane / 16, m = lane % 16;
  const int pp = w / d.ks, kq = w - pp * d.ks;
  const int u0 = kq * NPER;
  const int npg = d.H / 16 / d.ppb;
  const int nact = g.n_act;
  const int e_sh = d.trash - d.n_shared;   // first shared bucket
  ExpLoad<FMT, NPER> ring[D];
  auto issue_first = [&](int pg) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const bool live = j < nact;
      const int e = __builtin_amdgcn_readfirstlane(live ? g.act_b[j] : 0);
      const int ws = a.slot_map ? a.slot_map[e] : e;
      issue_expert<FMT, NPER>(ring[j], d, ws, live, pg * d.ppb + pp, u0, lane);
    }
  };
  // arrive, then issue the first down panel's weights (their loads would
  // otherwise hold up the arrival's wait for the act stores) and build the
  // tables the routing in LDS gives, then wait
  barrier_arrive(bar);
  int pg = blockIdx.x;
  if (pg >= npg) return;   // whole workgroup: nothing after the barrier
  issue_first(pg);

  // act rows: the sorted rows before the trash bucket (only the routed ones
  // when the shared experts' rows come from act_sh), then the shared rows
  const int sh_rows = d.act_sh ? d.n_shared * d.T : 0;
  const int nrows = g.act_r[d.act_sh ? nact - d.n_shared : nact];
  const int ldx = d.I + 8;
  const int per_row = d.I / 8;
  uint16_t* xs = reinterpret_cast<uint16_t*>(dyn);
  int* rowof = reinterpret_cast<int*>(dyn + (size_t)(d.row_cap + sh_rows) * ldx * 2);
  float* wof = reinterpret_cast<float*>(rowof + tiny::kTinyMaxA * kDcTok);
  int* eslot = reinterpret_cast<int*>(wof + tiny::kTinyMaxA * kDcTok);
  // token -> act row and summed weight per active expert, in active order
  // (the gate/up phase is over in every wave: the arrival's barrier)
  for (int i = tid; i < nact * kDcTok; i += bd) {
    rowof[i] = 0;
    wof[i] = 0.f;
  }
  __syncthreads();
  for (int j = tid; j < nact; j += bd) {
    const int e = g.act_b[j];
    eslot[j] = a.slot_map ? a.slot_map[e] : e;
    if (d.act_sh && e >= e_sh) {
      for (int t = 0; t < d.T; ++t) {
        rowof[j * kDcTok + t] = d.row_cap + (e - e_sh) * d.T + t;
        wof[j * kDcTok + t] = 1.0f;
      }
      continue;
    }
    for (int r = g.act_r[j]; r < g.act_r[j + 1]; ++r) {
      const int t = g.stok[r];
      rowof[j * kDcTok + t] = r;
      wof[j * kDcTok + t] += g.sw[r];
    }
  }
  barrier_wait(bar, gen);   // ends with a workgroup barrier: the tables are visible

  const int pieces = (nrows + sh_rows) * per_row;
  // device-coherent loads: the rows other workgroups wrote before the barrier
  const __amdgpu_buffer_rsrc_t ract = __builtin_amdgcn_make_buffer_rsrc(
      (void*)d.act, 0, nrows * d.I * 2, kRawBufferFlags);
  const __amdgpu_buffer_rsrc_t rsh = __builtin_amdgcn_make_buffer_rsrc(
      (void*)d.act_sh, 0, sh_rows * d.I * 2, kRawBufferFlags);
  for (int c0 = tid; c0 < pieces; c0 += kLayerStageSB * bd) {
    u32x4_t v[kLayerStageSB];
#pragma unroll
    for (int k = 0; k < kLayerStageSB; ++k) {
      const int c = min(c0 + k * bd, pieces - 1);
      const int r = c / per_row, c8 = c - r * per_row;
      v[k] = __builtin_bit_cast(
          u32x4_t, r < nrows ? __builtin_amdgcn_raw_buffer_load_b128(ract, (r * d.I + c8 * 8) * 2,
                                                                     0, kAuxDevice)
                             : __builtin_amdgcn_raw_buffer_load_b128(
                                   rsh, ((r - nrows) * d.I + c8 * 8) * 2, 0, kAuxDevice));
    }
#pragma unroll
    for (int k = 0; k < kLayerStageSB; ++k) {
      const int c = c0 + k * bd;
      if (c < pieces) {
        const int r = c / per_row, c8 = c - r * per_row;
        const int lr = r < nrows ? r : d.row_cap + (r - nrows);
        *reinterpret_cast<u32x4_t*>(xs + lr * ldx + c8 * 8) = v[k];
      }
    }
  }
  __syncthreads();

  const int nit = (nact + D - 1) / D;
  while (true) {
    const int panel = pg * d.ppb + pp;
    f32x4_t tacc = {0.f, 0.f, 0.f, 0.f};   // tokens 4q + i, column m of the panel
    for (int it = 0; it < nit; ++it) {
#pragma unroll
      for (int dd = 0; dd < D; ++dd) {
        const int j = it * D + dd;
        const bool live = j < nact;
        const int jt = live ? j : 0;
        const uint16_t* xa = xs + rowof[jt * kDcTok + m] * ldx + q * F::kCK;
        f32x4_t pe = consume_expert<FMT, NPER>(ring[dd], u0, xa);
        if constexpr (FMT == kNVFP4) {
          const float gv = d.gs ? d.gs[eslot[jt]] : 1.0f;
          pe = pe * gv;
        }
        const f32x4_t wv = live ? *reinterpret_cast<const f32x4_t*>(wof + jt * kDcTok + 4 * q)
                                : f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i)
          tacc[i] = wv[i] != 0.f ? __builtin_fmaf(wv[i], pe[i], tacc[i]) : tacc[i];
        const int jn = j + D;
        const int wsn = __builtin_amdgcn_readfirstlane(eslot[jn < nact ? jn : 0]);
        issue_expert<FMT, NPER>(ring[dd], d, wsn, jn < nact, panel, u0, lane);
      }
    }
    red[w][lane] = tacc;
    __syncthreads();
    for (int t = tid; t < d.ppb * 256; t += bd) {   // tokens x 16 columns per panel
      const int pq = t / 256, tok = (t % 256) / 16, n = t % 16;
      if (tok < d.T) {
        const int l = (tok / 4) * 16 + n, i = tok % 4;
        float v = 0.f;
        for (int k = 0; k < d.ks; ++k) v += red[pq * d.ks + k][l][i];
        const long o = (long)tok * d.H + 16 * (pg * d.ppb + pq) + n;
        if (d.out_bf16) reinterpret_cast<uint16_t*>(d.out)[o] = f32_to_bf16(v);
        else reinterpret_cast<float*>(d.out)[o] = v;
      }
    }
    pg += gridDim.x;
    if (pg >= npg) break;
    __syncthreads();   // red is read back before the next panel writes it
    // the ring holds loads past the last expert (zero-length): reissue
    issue_first(pg);
  }
}

// Down shape of the one-launch layer: ks * ppb = the workgroup's waves nw,
// the K range of I split ks ways into NPER in {1, 2} units per wave (the
// fewest panels per workgroup that fit).
bool layer_down_shape(int nw, int H, int I, int& ks, int& ppb, int& nper) {
  const int nunits = I / 128, npan = H / 16;
  for (ppb = 1; ppb <= nw; ppb *= 2) {
    if (nw % ppb || npan % ppb) continue;
    ks = nw / ppb;
    if (nunits % ks) continue;
    nper = nunits / ks;
    if (nper == 1 || nper == 2) return true;
  }
  return false;
}

// Workgroup of the one-launch layer: the gate/up fast shape's K split,
// raised to a routing wave per token and to as many waves as the down's
// 128-k units (up to 8 waves), so the down runs one unit per wave where it
// can; xc for that workgroup size (at least 2).
template <int FMT>
bool route_phase_shape(int T, int H, int I, int& ksplit, int& xc) {
  if (!gate_up_fast_shape<FMT>(T, H, ksplit, xc)) return false;
  while (ksplit < 4 && (2 * ksplit < T || 2 * ksplit < I / 128)) ksplit *= 2;
  const long pieces = (long)T * (H / 8), bd = 128L * ksplit;
  xc = pieces <= 2 * bd ? 2 : pieces <= 4 * bd ? 4 : 8;
  return true;
}

// LDS of the one-launch layer: the x rows of the gate/up phase, or the down
// phase's act rows (row_cap sorted + sh_rows shared) and tables.
size_t layer_lds(int T, int H, int I, int row_cap, int sh_rows) {
  const size_t gu = (size_t)T * H * 2;
  const size_t dn = (size_t)(row_cap + sh_rows) * (I + 8) * 2 +
                    (size_t)tiny::kTinyMaxA * kDcTok * 8 + (size_t)tiny::kTinyMaxA * 4;
  return gu > dn ? gu : dn;
}
constexpr size_t kLayerLdsMax = 96 * 1024;

using LayerKernel = void (*)(tiny::SmallArgs, DecodeArgs, DownCombineArgs, void*, int, int,
                             unsigned*);

template <int FMT, int MODE, int EPL, int XC>
LayerKernel layer_kernel_nper(int nper) {
  return nper == 1 ? decode_layer_kernel<FMT, MODE, EPL, XC, 1>
                   : decode_layer_kernel<FMT, MODE, EPL, XC, 2>;
}

template <int FMT, int XC>
LayerKernel layer_kernel_mode(int mode, int epl, int nper) {
  if (mode == 2) return layer_kernel_nper<FMT, 2, 1, XC>(nper);
  if (mode == 1)
    return epl == 4 ? layer_kernel_nper<FMT, 1, 4, XC>(nper) : layer_kernel_nper<FMT, 1, 8, XC>(nper);
  return epl == 4 ? layer_kernel_nper<FMT, 0, 4, XC>(nper) : layer_kernel_nper<FMT, 0, 8, XC>(nper);
}

// Resident workgroups per CU of a kernel at (block, LDS), queried once per
// device and shape.
int resident_per_cu(const void* k, int bd, size_t lds) {
  static std::mutex mu;
  static std::map<std::tuple<int, const void*, int, size_t>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  const auto key = std::make_tuple(dev, k, bd, lds);
  std::lock_guard<std::mutex> lock(mu);
  const auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, bd, lds) != hipSuccess) n = 0;
  cache[key] = n;
  return n;
}

template <int FMT>
hipError_t launch_layer(int mode, int epl, const tiny::SmallArgs& ra, DecodeArgs a,
                        DownCombineArgs d, void* act_sh, int max_tiles, unsigned* bar,
                        hipStream_t stream) {
  using F = WFmt<FMT>;
  if (!a.w_estride) a.w_estride = F::w_bytes(2L * a.I, a.H);
  if (!a.s_estride) a.s_estride = F::s_bytes(2L * a.I, a.H);
  if (!d.w_estride) d.w_estride = F::w_bytes(a.H, a.I);
  if (!d.s_estride) d.s_estride = F::s_bytes(a.H, a.I);
  int ksplit = 0, xc = 0, ks = 0, ppb = 0, nper = 0;
  if (!route_phase_shape<FMT>(a.T, a.H, a.I, ksplit, xc)) return hipErrorInvalidValue;
  const int bd = 128 * ksplit;
  if (!layer_down_shape(bd / kWave, a.H, a.I, ks, ppb, nper)) return hipErrorInvalidValue;
  a.ksplit = ksplit;
  a.rows = a.T;
  d.ks = ks;
  d.ppb = ppb;
  const int npan = a.I / 16;
  const int n_sh = act_sh ? ra.NS * npan : 0;
  const int skip = act_sh ? ra.NS * ((a.T + ra.bm - 1) / ra.bm) : 0;
  const int A = a.T * (ra.K + ra.NS);
  const int sh_rows = act_sh ? ra.NS * a.T : 0;
  d.row_cap = std::max(A - sh_rows, 1);
  const size_t lds = layer_lds(a.T, a.H, a.I, d.row_cap, sh_rows);
  if (lds > kLayerLdsMax) return hipErrorInvalidValue;
  LayerKernel k = nullptr;
  switch (xc) {
    case 2: k = layer_kernel_mode<FMT, 2>(mode, epl, nper); break;
    case 4: k = layer_kernel_mode<FMT, 4>(mode, epl, nper); break;
    default: k = layer_kernel_mode<FMT, 8>(mode, epl, nper); break;
  }
  // one resident round: every workgroup must reach the grid barrier
  if (!k) return hipErrorInvalidValue;
  const int per_cu = resident_per_cu(reinterpret_cast<const void*>(k), bd, lds);
  const long resident = (long)per_cu * cu_count();
  const long want = std::max<long>(n_sh + (long)max_tiles * npan, a.H / 16 / ppb);
  const long grid = std::min(resident, want);
  if (grid < n_sh + 1) return hipErrorInvalidValue;
  k<<<dim3((unsigned)grid), bd, lds, stream>>>(ra, a, d, act_sh, n_sh, skip, bar);
  return hipPeekAtLastError();
}

}  // namespace
}  // namespace xtu

using namespace xtu;

extern "C" {

int xtu_decode_route_gate_up_ok(int fmt, int mode, int T, int E, int K, int n_group,
                                int n_shared, int H, int I);

int xtu_decode_layer_barrier_words(void) { return kBarWords; }

int xtu_decode_layer_ok(int fmt, int mode, int T, int E, int K, int n_group, int n_shared,
                        int H, int I) {
  if (!xtu_decode_route_gate_up_ok(fmt, mode, T, E, K, n_group, n_shared, H, I)) return 0;
  int ksplit = 0, xc = 0, ks = 0, ppb = 0, nper = 0;
  bool ok = false;
  switch (fmt) {
    case kMXFP4: ok = route_phase_shape<kMXFP4>(T, H, I, ksplit, xc); break;
    case kNVFP4: ok = route_phase_shape<kNVFP4>(T, H, I, ksplit, xc); break;
    case kFP8: ok = route_phase_shape<kFP8>(T, H, I, ksplit, xc); break;
    case kBF16: ok = route_phase_shape<kBF16>(T, H, I, ksplit, xc); break;
  }
  if (!ok || !layer_down_shape(2 * ksplit, H, I, ks, ppb, nper)) return 0;
  const int A = T * (K + n_shared);
  return layer_lds(T, H, I, A, n_shared * T) <= kLayerLdsMax;
}

hipError_t xtu_decode_layer(
    int mode, const float* logits, const float* bias, int32_t* topk_ids, float* topk_weights,
    int T, int E, int K, int n_group, int topk_group, float routed_scaling, int renormalize,
    const int32_t* id_map, int n_shared, int drop_zero, int bm, int32_t* sorted_pair,
    int32_t* sorted_tok, float* sorted_wts, int32_t* inv, int32_t* seg_start, int32_t* active,
    int32_t* n_active, int32_t* tile_expert, int32_t* tile_row0, int32_t* n_tiles,
    int32_t* expert_tile_start, int fmt, const void* x, int H, int I, const void* w13,
    const void* s13, const float* gs13, long w13_estride, long s13_estride,
    const int32_t* slot_map, int max_tiles, void* act, void* act_shared, float limit,
    float alpha, float beta, const void* w2, const void* s2, const float* gs2,
    long w2_estride, long s2_estride, void* out, int out_bf16, uint32_t* barrier,
    hipStream_t stream) {
  XTU_CHECK_ARG(xtu_decode_layer_ok(fmt, mode, T, E, K, n_group, n_shared, H, I));
  XTU_CHECK_ARG(bm >= 1 && bm <= kMaxTok && w13_estride >= 0 && s13_estride >= 0 &&
                w2_estride >= 0 && s2_estride >= 0);
  {
    const long A = (long)T * (K + n_shared);
    const long b = std::min<long>(std::min<long>(E, (long)T * K) + n_shared, A);
    XTU_CHECK_ARG(max_tiles >= std::min<long>(A, b + (A - b) / std::max(bm, 1)) &&
                  max_tiles >= 1 && max_tiles <= tiny::kTinyMaxA);
  }
  if (mode == 1)
    XTU_CHECK_ARG(topk_group > 0 && topk_group <= n_group && K <= topk_group * (E / n_group));
  XTU_CHECK_ARG(topk_ids && topk_weights && (mode == 2 || logits));
  XTU_CHECK_ARG(sorted_pair && sorted_tok && sorted_wts && inv && seg_start && active &&
                n_active && tile_expert && tile_row0 && n_tiles && expert_tile_start);
  XTU_CHECK_ARG(x && w13 && (fmt == kBF16 || s13) && act && (n_shared > 0 || !act_shared));
  XTU_CHECK_ARG(w2 && (fmt == kBF16 || s2) && out && barrier);
  tiny::SmallArgs ra{logits, bias, topk_ids, topk_weights, id_map, T, K, E, n_group,
                     topk_group, renormalize, n_shared, drop_zero, bm, routed_scaling,
                     sorted_pair, sorted_tok, inv, seg_start, active, n_active, sorted_wts,
                     tile_expert, tile_row0, n_tiles, expert_tile_start};
  const int epl = tiny::tiny_epl(ra, mode);   // also checks the logit / bias alignment
  XTU_CHECK_ARG(epl != 0);
  (void)hipGetLastError();
  DecodeArgs a{(const uint16_t*)x, (const uint8_t*)w13, (const uint8_t*)s13, gs13, nullptr,
               nullptr, nullptr, nullptr, slot_map, act, nullptr, T, H, I, w13_estride,
               s13_estride, limit, alpha, beta, 0, 1, 1, 0};
  DownCombineArgs d{(const uint16_t*)act, (const uint8_t*)w2, (const uint8_t*)s2, gs2,
                    nullptr, nullptr, nullptr, nullptr, nullptr, slot_map, out,
                    out_bf16 ? 1 : 0, T, H, I, E + n_shared, tiny::kTinyMaxA, 1, w2_estride,
                    s2_estride, 1, 1, (const uint16_t*)act_shared, n_shared};
  unsigned* bar = reinterpret_cast<unsigned*>(barrier);
  switch (fmt) {
    case kMXFP4: return launch_layer<kMXFP4>(mode, epl, ra, a, d, act_shared, max_tiles, bar, stream);
    case kNVFP4: return launch_layer<kNVFP4>(mode, epl, ra, a, d, act_shared, max_tiles, bar, stream);
    case kFP8: return launch_layer<kFP8>(mode, epl, ra, a, d, act_shared, max_tiles, bar, stream);
    case kBF16: return launch_layer<kBF16>(mode, epl, ra, a, d, act_shared, max_tiles, bar, stream);
  }
  return hipErrorInvalidValue;
}

}  // extern "C"
