// Skinny-M (decode) expert kernels: launch shapes and the C entries of the
// gate/up, down, fused down + combine and routing launches (the kernels and
// their layout are described in decode.hpp).
#include "decode.hpp"

namespace xtu {
namespace {

// Sorted act rows the fused down stages: all A, or, when the shared experts'
// rows come from act_sh, the A - shared_rows routed ones (the segmentation
// puts the T * n_shared shared pairs after every routed pair).
int dc_sorted_rows(int A, int shared_rows) {
  return shared_rows > 0 ? (A - shared_rows > 1 ? A - shared_rows : 1) : A;
}

// Launch shape of the fused down: (KS, NPER) with KS * NPER = I / 128 and
// NPER in {1, 2, 4}, KS <= 8; KS grows until the grid holds about 2048 waves.
// Returns false when the shape or the LDS stage does not fit.
bool dc_shape(int fmt, int T, int rows, int sh_rows, int H, int I, int trash, int max_active,
              int& ks, int& nper, int& ppb, size_t& lds) {
  if (T < 1 || T > kDcTok || fmt < 0 || fmt > 3 || trash < 0 || trash > 4096 || rows < 1 ||
      max_active < 1)
    return false;
  const int nunits = I / 128, npan = H / 16;
  ks = 1;
  while (ks < 8 && nunits % (2 * ks) == 0 && (long)npan * ks < XTU_DC_WAVES) ks *= 2;
  while (nunits / ks > 4 && ks < 8 && nunits % (2 * ks) == 0) ks *= 2;
  nper = nunits / ks;
  if (nunits % ks || (nper != 1 && nper != 2 && nper != 4)) return false;
  ppb = 1;
  while (ks * ppb * 2 <= 4 && npan % (ppb * 2) == 0) ppb *= 2;
  lds = (size_t)(rows + sh_rows) * (I + 8) * 2 + (size_t)max_active * (2 * kDcTok + 2) * 4 +
        (size_t)(trash + 2) * 4 + (size_t)rows * 8;
  const size_t red = (size_t)ks * ppb * kWave * 16;
  if (lds < red) lds = red;
  return lds <= kDcLds;
}

template <int FMT>
hipError_t launch_down_combine(DownCombineArgs a, int nper, size_t lds, hipStream_t stream) {
  using F = WFmt<FMT>;
  if (!a.w_estride) a.w_estride = F::w_bytes(a.H, a.I);
  if (!a.s_estride) a.s_estride = F::s_bytes(a.H, a.I);
  const dim3 grid(a.H / 16 / a.ppb);
  const int bd = kWave * a.ks * a.ppb;
  switch (nper) {
    case 1: decode_down_combine_kernel<FMT, 1><<<grid, bd, lds, stream>>>(a); break;
    case 2: decode_down_combine_kernel<FMT, 2><<<grid, bd, lds, stream>>>(a); break;
    case 4: decode_down_combine_kernel<FMT, 4><<<grid, bd, lds, stream>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipPeekAtLastError();
}

template <int FMT>
hipError_t launch_decode(int which, DecodeArgs a, int max_active, hipStream_t stream) {
  using F = WFmt<FMT>;
  constexpr int NU = round_units<FMT>();
  if (which == 0) {
    if (!a.w_estride) a.w_estride = F::w_bytes(2L * a.I, a.H);
    if (!a.s_estride) a.s_estride = F::s_bytes(2L * a.I, a.H);
    const int row_bytes = a.H * 2;
    const int cap = kLdsBudget / row_bytes;
    a.rows = a.T < cap ? a.T : cap;
    if (a.rows < 1) return hipErrorInvalidValue;
    a.ksplit = pick_ksplit(a.H / 128, NU, 4);
    a.ppb = 1;
    const long items = (long)max_active * (a.I / 16);
    const int bd = 128 * a.ksplit;
    const long pieces = (long)a.T * (a.H / 8);   // 16-byte pieces of the batch's rows
    const bool generic = a.T > a.rows || a.H / 128 > NU * a.ksplit || pieces > 8L * bd;
    const size_t lds = (size_t)a.rows * row_bytes;
    if (generic)
      decode_gate_up_kernel<FMT, true, 1><<<dim3(items), bd, lds, stream>>>(a);
    else if (pieces <= bd)
      decode_gate_up_kernel<FMT, false, 1><<<dim3(items), bd, lds, stream>>>(a);
    else if (pieces <= 2L * bd)
      decode_gate_up_kernel<FMT, false, 2><<<dim3(items), bd, lds, stream>>>(a);
    else if (pieces <= 4L * bd)
      decode_gate_up_kernel<FMT, false, 4><<<dim3(items), bd, lds, stream>>>(a);
    else
      decode_gate_up_kernel<FMT, false, 8><<<dim3(items), bd, lds, stream>>>(a);
  } else {
    if (!a.w_estride) a.w_estride = F::w_bytes(a.H, a.I);
    if (!a.s_estride) a.s_estride = F::s_bytes(a.H, a.I);
    const int row_bytes = a.I * 2;
    const int cap = kLdsBudget / row_bytes;
    const int tmax = a.T < kMaxTok ? a.T : kMaxTok;   // an expert holds at most T pairs
    a.rows = tmax < cap ? tmax : cap;
    if (a.rows < 1) return hipErrorInvalidValue;
    a.ksplit = pick_ksplit(a.I / 128, NU, 4);
    a.ppb = 4 / a.ksplit;
    if ((a.H / 16) % a.ppb) a.ppb = 1;
    const long items = (long)max_active * (a.H / 16 / a.ppb);
    const bool generic = tmax > a.rows || a.I / 128 > NU * a.ksplit;
    const size_t lds = (size_t)a.rows * row_bytes;
    if (generic)
      decode_down_kernel<FMT, true><<<dim3(items), 64 * a.ksplit * a.ppb, lds, stream>>>(a);
    else
      decode_down_kernel<FMT, false><<<dim3(items), 64 * a.ksplit * a.ppb, lds, stream>>>(a);
  }
  return hipPeekAtLastError();
}

bool gate_up_fast_shape_fmt(int fmt, int T, int H, int& ksplit, int& xc) {
  switch (fmt) {
    case kMXFP4: return gate_up_fast_shape<kMXFP4>(T, H, ksplit, xc);
    case kNVFP4: return gate_up_fast_shape<kNVFP4>(T, H, ksplit, xc);
    case kFP8: return gate_up_fast_shape<kFP8>(T, H, ksplit, xc);
    case kBF16: return gate_up_fast_shape<kBF16>(T, H, ksplit, xc);
  }
  return false;
}

template <int FMT, int XC>
void launch_route_shared_xc(int mode, int epl, dim3 grid, int bd, size_t lds,
                            const tiny::SmallArgs& ra, const DecodeArgs& a, hipStream_t stream) {
  if (mode == 2) {
    decode_route_shared_kernel<FMT, 2, 1, XC><<<grid, bd, lds, stream>>>(ra, a);
  } else if (mode == 1) {
    if (epl == 4) decode_route_shared_kernel<FMT, 1, 4, XC><<<grid, bd, lds, stream>>>(ra, a);
    else decode_route_shared_kernel<FMT, 1, 8, XC><<<grid, bd, lds, stream>>>(ra, a);
  } else {
    if (epl == 4) decode_route_shared_kernel<FMT, 0, 4, XC><<<grid, bd, lds, stream>>>(ra, a);
    else decode_route_shared_kernel<FMT, 0, 8, XC><<<grid, bd, lds, stream>>>(ra, a);
  }
}

template <int FMT>
hipError_t launch_route_shared(int mode, int epl, const tiny::SmallArgs& ra, DecodeArgs a,
                               hipStream_t stream) {
  using F = WFmt<FMT>;
  if (!a.w_estride) a.w_estride = F::w_bytes(2L * a.I, a.H);
  if (!a.s_estride) a.s_estride = F::s_bytes(2L * a.I, a.H);
  int ksplit = 0, xc = 0;
  if (!gate_up_fast_shape<FMT>(a.T, a.H, ksplit, xc)) return hipErrorInvalidValue;
  a.ksplit = ksplit;
  a.rows = a.T;
  const int bd = 128 * ksplit;
  if (a.T * kWave > bd) return hipErrorInvalidValue;   // one routing wave per token
  const dim3 grid(1 + ra.NS * (a.I / 16));
  const size_t lds = (size_t)a.T * a.H * 2;
  switch (xc) {
    case 1: launch_route_shared_xc<FMT, 1>(mode, epl, grid, bd, lds, ra, a, stream); break;
    case 2: launch_route_shared_xc<FMT, 2>(mode, epl, grid, bd, lds, ra, a, stream); break;
    case 4: launch_route_shared_xc<FMT, 4>(mode, epl, grid, bd, lds, ra, a, stream); break;
    default: launch_route_shared_xc<FMT, 8>(mode, epl, grid, bd, lds, ra, a, stream); break;
  }
  return hipPeekAtLastError();
}

template <int FMT, int XC>
void launch_route_gate_up_xc(int mode, int epl, dim3 grid, int bd, size_t lds,
                             const tiny::SmallArgs& ra, const DecodeArgs& a, void* act_sh,
                             int n_sh, int skip, hipStream_t stream) {
  if (mode == 2) {
    decode_route_gate_up_kernel<FMT, 2, 1, XC><<<grid, bd, lds, stream>>>(ra, a, act_sh, n_sh, skip);
  } else if (mode == 1) {
    if (epl == 4)
      decode_route_gate_up_kernel<FMT, 1, 4, XC><<<grid, bd, lds, stream>>>(ra, a, act_sh, n_sh, skip);
    else
      decode_route_gate_up_kernel<FMT, 1, 8, XC><<<grid, bd, lds, stream>>>(ra, a, act_sh, n_sh, skip);
  } else {
    if (epl == 4)
      decode_route_gate_up_kernel<FMT, 0, 4, XC><<<grid, bd, lds, stream>>>(ra, a, act_sh, n_sh, skip);
    else
      decode_route_gate_up_kernel<FMT, 0, 8, XC><<<grid, bd, lds, stream>>>(ra, a, act_sh, n_sh, skip);
  }
}

constexpr size_t kLdsCu = 160 * 1024;                                      // LDS per CU
constexpr size_t kStaticLds = 8 * kWave * 16 + sizeof(tiny::TinySmem);     // red + routing

// Grid: the split-off shared experts' panels (act_sh set), then about one
// resident round of routed workgroups looping over the batch's work items.
template <int FMT>
hipError_t launch_route_gate_up(int mode, int epl, const tiny::SmallArgs& ra, DecodeArgs a,
                                void* act_sh, int max_tiles, hipStream_t stream) {
  using F = WFmt<FMT>;
  if (!a.w_estride) a.w_estride = F::w_bytes(2L * a.I, a.H);
  if (!a.s_estride) a.s_estride = F::s_bytes(2L * a.I, a.H);
  int ksplit = 0, xc = 0;
  if (!gate_up_fast_shape<FMT>(a.T, a.H, ksplit, xc)) return hipErrorInvalidValue;
  // a routing wave per token where the workgroup can have one (at most 8
  // waves): the K range is split further, the routing not serialised
  while (ksplit < 4 && 2 * ksplit < a.T) ksplit *= 2;
  a.ksplit = ksplit;
  a.rows = a.T;
  const int bd = 128 * ksplit;
  const int npan = a.I / 16;
  const int n_sh = act_sh ? ra.NS * npan : 0;
  const int skip = act_sh ? ra.NS * ((a.T + ra.bm - 1) / ra.bm) : 0;
  const size_t lds = (size_t)a.T * a.H * 2;
  // routed workgroups: one resident round beside the shared ones (the
  // work items past it are looped over), never more than the items
  const int per_cu = std::max(1, std::min<int>(1024 / bd, (int)(kLdsCu / (lds + kStaticLds))));
  const int routed = (int)std::max<long>(
      1, std::min<long>((long)max_tiles * npan, (long)per_cu * cu_count() - n_sh));
  const dim3 grid(n_sh + routed);
  switch (xc) {
    case 1: launch_route_gate_up_xc<FMT, 1>(mode, epl, grid, bd, lds, ra, a, act_sh, n_sh, skip, stream); break;
    case 2: launch_route_gate_up_xc<FMT, 2>(mode, epl, grid, bd, lds, ra, a, act_sh, n_sh, skip, stream); break;
    case 4: launch_route_gate_up_xc<FMT, 4>(mode, epl, grid, bd, lds, ra, a, act_sh, n_sh, skip, stream); break;
    default: launch_route_gate_up_xc<FMT, 8>(mode, epl, grid, bd, lds, ra, a, act_sh, n_sh, skip, stream); break;
  }
  return hipPeekAtLastError();
}

hipError_t dispatch_decode(int fmt, int which, DecodeArgs a, int max_active, hipStream_t stream) {
  switch (fmt) {
    case kMXFP4: return launch_decode<kMXFP4>(which, a, max_active, stream);
    case kNVFP4: return launch_decode<kNVFP4>(which, a, max_active, stream);
    case kFP8: return launch_decode<kFP8>(which, a, max_active, stream);
    case kBF16: return launch_decode<kBF16>(which, a, max_active, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace
}  // namespace xtu

using namespace xtu;

extern "C" {

hipError_t xtu_decode_gate_up(int fmt, const void* x, int T, int H, int I, const void* w13,
                              const void* s13, const float* gs13, long w_estride,
                              long s_estride, const int32_t* slot_map,
                              const int32_t* sorted_tok, const int32_t* seg_start,
                              const int32_t* active, const int32_t* tile_row0,
                              const int32_t* n_active, int max_active, void* act, float limit,
                              float alpha, float beta, hipStream_t stream) {
  XTU_CHECK_ARG(shape_ok(fmt, H, I) && max_active >= 0 && max_active <= 65535 && T >= 0 &&
                T <= kMaxTok);
  XTU_CHECK_ARG(w_estride >= 0 && s_estride >= 0);
  XTU_CHECK_ARG(x && w13 && (fmt == kBF16 || s13) && sorted_tok && seg_start && active &&
                n_active && act);
  if (max_active == 0 || T == 0) return hipSuccess;
  (void)hipGetLastError();
  DecodeArgs a{(const uint16_t*)x, (const uint8_t*)w13, (const uint8_t*)s13, gs13, sorted_tok,
               seg_start, active, n_active, slot_map, act, tile_row0, T, H, I, w_estride,
               s_estride, limit, alpha, beta, 0, 1, 1};
  return dispatch_decode(fmt, 0, a, max_active, stream);
}

hipError_t xtu_decode_down(int fmt, const void* act, int T, int H, int I, const void* w2,
                           const void* s2, const float* gs2, long w_estride, long s_estride,
                           const int32_t* slot_map, const int32_t* seg_start,
                           const int32_t* active, const int32_t* tile_row0,
                           const int32_t* n_active, int max_active, float* y,
                           hipStream_t stream) {
  XTU_CHECK_ARG(shape_ok(fmt, H, I) && max_active >= 0 && max_active <= 65535 && T >= 0 &&
                T <= kMaxTok);
  XTU_CHECK_ARG(w_estride >= 0 && s_estride >= 0);
  XTU_CHECK_ARG(act && w2 && (fmt == kBF16 || s2) && seg_start && active && n_active && y);
  if (max_active == 0 || T == 0) return hipSuccess;
  (void)hipGetLastError();
  DecodeArgs a{(const uint16_t*)act, (const uint8_t*)w2, (const uint8_t*)s2, gs2, nullptr,
               seg_start, active, n_active, slot_map, y, tile_row0, T, H, I, w_estride,
               s_estride, 0.f, 1.f, 0.f, 0, 1, 1};
  return dispatch_decode(fmt, 1, a, max_active, stream);
}

hipError_t xtu_decode_down_by_pair(int fmt, const void* act, int T, int H, int I, const void* w2,
                                   const void* s2, const float* gs2, long w_estride,
                                   long s_estride, const int32_t* slot_map,
                                   const int32_t* seg_start, const int32_t* active,
                                   const int32_t* tile_row0, const int32_t* n_active,
                                   int max_active, const int32_t* sorted_pair, float* y,
                                   hipStream_t stream) {
  XTU_CHECK_ARG(shape_ok(fmt, H, I) && max_active >= 0 && max_active <= 65535 && T >= 0 &&
                T <= kMaxTok);
  XTU_CHECK_ARG(w_estride >= 0 && s_estride >= 0);
  XTU_CHECK_ARG(act && w2 && (fmt == kBF16 || s2) && seg_start && active && n_active && y &&
                sorted_pair);
  if (max_active == 0 || T == 0) return hipSuccess;
  (void)hipGetLastError();
  DecodeArgs a{(const uint16_t*)act, (const uint8_t*)w2, (const uint8_t*)s2, gs2, nullptr,
               seg_start, active, n_active, slot_map, y, tile_row0, T, H, I, w_estride,
               s_estride, 0.f, 1.f, 0.f, 0, 1, 1, 0, sorted_pair};
  return dispatch_decode(fmt, 1, a, max_active, stream);
}

int xtu_decode_route_shared_ok(int fmt, int mode, int T, int E, int K, int n_group,
                               int n_shared, int H, int I) {
  int ksplit = 0, xc = 0;
  if (!shape_ok(fmt, H, I) || mode < 0 || mode > 2 || K < 1 || K > 16 || K > E || E < 1 ||
      E > 1024 || n_shared < 1 || n_shared > 16 ||
      !gate_up_fast_shape_fmt(fmt, T, H, ksplit, xc) || T * kWave > 128 * ksplit)
    return 0;
  if (mode == 1 && (n_group <= 0 || n_group > 64 || E % n_group)) return 0;
  tiny::SmallArgs r{};
  r.T = T;
  r.K = K;
  r.E = E;
  r.NS = n_shared;
  r.n_group = n_group > 0 ? n_group : 1;
  r.renorm = 1;
  static const float probe[4] = {0.f, 0.f, 0.f, 0.f};   // a 16-byte-aligned row stands in
  r.logits = probe;
  return tiny::tiny_epl(r, mode) != 0;
}

hipError_t xtu_decode_route_shared(
    int mode, const float* logits, const float* bias, int32_t* topk_ids, float* topk_weights,
    int T, int E, int K, int n_group, int topk_group, float routed_scaling, int renormalize,
    const int32_t* id_map, int n_shared, int drop_zero, int bm, int32_t* sorted_pair,
    int32_t* sorted_tok, float* sorted_wts, int32_t* inv, int32_t* seg_start, int32_t* active,
    int32_t* n_active, int32_t* tile_expert, int32_t* tile_row0, int32_t* n_tiles,
    int32_t* expert_tile_start, int fmt, const void* x, int H, int I, const void* w13,
    const void* s13, const float* gs13, long w_estride, long s_estride, const int32_t* slot_map,
    void* act_shared, float limit, float alpha, float beta, hipStream_t stream) {
  XTU_CHECK_ARG(xtu_decode_route_shared_ok(fmt, mode, T, E, K, n_group, n_shared, H, I));
  XTU_CHECK_ARG(bm > 0 && w_estride >= 0 && s_estride >= 0);
  if (mode == 1)
    XTU_CHECK_ARG(topk_group > 0 && topk_group <= n_group && K <= topk_group * (E / n_group));
  XTU_CHECK_ARG(topk_ids && topk_weights && (mode == 2 || logits));
  XTU_CHECK_ARG(sorted_pair && sorted_tok && sorted_wts && inv && seg_start && active &&
                n_active && tile_expert && tile_row0 && n_tiles && expert_tile_start);
  XTU_CHECK_ARG(x && w13 && (fmt == kBF16 || s13) && act_shared);
  tiny::SmallArgs ra{logits, bias, topk_ids, topk_weights, id_map, T, K, E, n_group,
                     topk_group, renormalize, n_shared, drop_zero, bm, routed_scaling,
                     sorted_pair, sorted_tok, inv, seg_start, active, n_active, sorted_wts,
                     tile_expert, tile_row0, n_tiles, expert_tile_start};
  const int epl = tiny::tiny_epl(ra, mode);   // also checks the logit / bias alignment
  XTU_CHECK_ARG(epl != 0);
  (void)hipGetLastError();
  DecodeArgs a{(const uint16_t*)x, (const uint8_t*)w13, (const uint8_t*)s13, gs13, nullptr,
               nullptr, nullptr, nullptr, slot_map, act_shared, nullptr, T, H, I, w_estride,
               s_estride, limit, alpha, beta, 0, 1, 1, 0};
  switch (fmt) {
    case kMXFP4: return launch_route_shared<kMXFP4>(mode, epl, ra, a, stream);
    case kNVFP4: return launch_route_shared<kNVFP4>(mode, epl, ra, a, stream);
    case kFP8: return launch_route_shared<kFP8>(mode, epl, ra, a, stream);
    case kBF16: return launch_route_shared<kBF16>(mode, epl, ra, a, stream);
  }
  return hipErrorInvalidValue;
}

int xtu_decode_route_gate_up_ok(int fmt, int mode, int T, int E, int K, int n_group,
                                int n_shared, int H, int I) {
  int ksplit = 0, xc = 0;
  if (!shape_ok(fmt, H, I) || mode < 0 || mode > 2 || K < 1 || K > 16 || K > E || E < 1 ||
      E > 1024 || n_shared < 0 || n_shared > 16 || !gate_up_fast_shape_fmt(fmt, T, H, ksplit, xc))
    return 0;
  if (mode == 1 && (n_group <= 0 || n_group > 64 || E % n_group)) return 0;
  tiny::SmallArgs r{};
  r.T = T;
  r.K = K;
  r.E = E;
  r.NS = n_shared;
  r.n_group = n_group > 0 ? n_group : 1;
  r.renorm = 1;
  static const float probe[4] = {0.f, 0.f, 0.f, 0.f};   // a 16-byte-aligned row stands in
  r.logits = probe;
  return tiny::tiny_epl(r, mode) != 0;
}

hipError_t xtu_decode_route_gate_up(
    int mode, const float* logits, const float* bias, int32_t* topk_ids, float* topk_weights,
    int T, int E, int K, int n_group, int topk_group, float routed_scaling, int renormalize,
    const int32_t* id_map, int n_shared, int drop_zero, int bm, int32_t* sorted_pair,
    int32_t* sorted_tok, float* sorted_wts, int32_t* inv, int32_t* seg_start, int32_t* active,
    int32_t* n_active, int32_t* tile_expert, int32_t* tile_row0, int32_t* n_tiles,
    int32_t* expert_tile_start, int fmt, const void* x, int H, int I, const void* w13,
    const void* s13, const float* gs13, long w_estride, long s_estride, const int32_t* slot_map,
    int max_tiles, void* act, void* act_shared, float limit, float alpha, float beta,
    hipStream_t stream) {
  XTU_CHECK_ARG(xtu_decode_route_gate_up_ok(fmt, mode, T, E, K, n_group, n_shared, H, I));
  XTU_CHECK_ARG(bm >= 1 && bm <= kMaxTok && w_estride >= 0 && s_estride >= 0);
  // every tile of the batch needs a work item: b non-empty buckets of A
  // pairs hold at most b + (A - b) / bm tiles (ceil(n / bm) <= 1 + (n-1) / bm)
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
  tiny::SmallArgs ra{logits, bias, topk_ids, topk_weights, id_map, T, K, E, n_group,
                     topk_group, renormalize, n_shared, drop_zero, bm, routed_scaling,
                     sorted_pair, sorted_tok, inv, seg_start, active, n_active, sorted_wts,
                     tile_expert, tile_row0, n_tiles, expert_tile_start};
  const int epl = tiny::tiny_epl(ra, mode);   // also checks the logit / bias alignment
  XTU_CHECK_ARG(epl != 0);
  (void)hipGetLastError();
  DecodeArgs a{(const uint16_t*)x, (const uint8_t*)w13, (const uint8_t*)s13, gs13, nullptr,
               nullptr, nullptr, nullptr, slot_map, act, nullptr, T, H, I, w_estride,
               s_estride, limit, alpha, beta, 0, 1, 1, 0};
  switch (fmt) {
    case kMXFP4: return launch_route_gate_up<kMXFP4>(mode, epl, ra, a, act_shared, max_tiles, stream);
    case kNVFP4: return launch_route_gate_up<kNVFP4>(mode, epl, ra, a, act_shared, max_tiles, stream);
    case kFP8: return launch_route_gate_up<kFP8>(mode, epl, ra, a, act_shared, max_tiles, stream);
    case kBF16: return launch_route_gate_up<kBF16>(mode, epl, ra, a, act_shared, max_tiles, stream);
  }
  return hipErrorInvalidValue;
}

hipError_t xtu_decode_gate_up_routed(int fmt, const void* x, int T, int H, int I,
                                     const void* w13, const void* s13, const float* gs13,
                                     long w_estride, long s_estride, const int32_t* slot_map,
                                     const int32_t* sorted_tok, const int32_t* seg_start,
                                     const int32_t* active, const int32_t* tile_row0,
                                     const int32_t* n_active, int max_active, int n_shared,
                                     void* act, float limit, float alpha, float beta,
                                     hipStream_t stream) {
  int ksplit = 0, xc = 0;
  XTU_CHECK_ARG(shape_ok(fmt, H, I) && max_active >= 0 && max_active <= 65535 && T >= 0 &&
                T <= kMaxTok && n_shared >= 0 && n_shared <= max_active);
  XTU_CHECK_ARG(T == 0 || gate_up_fast_shape_fmt(fmt, T, H, ksplit, xc));
  XTU_CHECK_ARG(w_estride >= 0 && s_estride >= 0);
  XTU_CHECK_ARG(x && w13 && (fmt == kBF16 || s13) && sorted_tok && seg_start && active &&
                n_active && act);
  if (max_active == n_shared || T == 0) return hipSuccess;
  (void)hipGetLastError();
  DecodeArgs a{(const uint16_t*)x, (const uint8_t*)w13, (const uint8_t*)s13, gs13, sorted_tok,
               seg_start, active, n_active, slot_map, act, tile_row0, T, H, I, w_estride,
               s_estride, limit, alpha, beta, 0, 1, 1, n_shared};
  return dispatch_decode(fmt, 0, a, max_active - n_shared, stream);
}

int xtu_decode_down_combine_ok(int fmt, int T, int A, int H, int I, int trash, int max_active,
                               int shared_rows) {
  int ks, nper, ppb;
  size_t lds;
  return shape_ok(fmt, H, I) && A >= 0 && max_active >= 0 && max_active <= 65535 &&
         shared_rows >= 0 && shared_rows <= kDcTok * 16 &&
         dc_shape(fmt, T, dc_sorted_rows(A, shared_rows), shared_rows, H, I, trash, max_active,
                  ks, nper, ppb, lds);
}

hipError_t xtu_decode_down_combine(int fmt, const void* act, const void* act_shared, int n_shared,
                                   int T, int A, int H, int I,
                                   const void* w2, const void* s2, const float* gs2,
                                   long w_estride, long s_estride, const int32_t* slot_map,
                                   const int32_t* sorted_tok, const float* sorted_wts,
                                   const int32_t* seg_start, int trash, const int32_t* active,
                                   const int32_t* n_active, int max_active, void* out,
                                   int out_bf16, hipStream_t stream) {
  int ks = 0, nper = 0, ppb = 0;
  size_t lds = 0;
  XTU_CHECK_ARG(n_shared >= 0 && n_shared <= 16 && n_shared <= trash);
  const int sh_rows = act_shared ? n_shared * T : 0;
  const int rows = dc_sorted_rows(A, sh_rows);
  XTU_CHECK_ARG(shape_ok(fmt, H, I) && A >= 0 && max_active >= 0 && max_active <= 65535 &&
                trash >= 0 &&
                dc_shape(fmt, T, rows, sh_rows, H, I, trash, max_active, ks, nper, ppb, lds));
  XTU_CHECK_ARG(w_estride >= 0 && s_estride >= 0);
  XTU_CHECK_ARG(act && w2 && (fmt == kBF16 || s2) && sorted_tok && sorted_wts && seg_start &&
                active && n_active && out);
  (void)hipGetLastError();
  DownCombineArgs a{(const uint16_t*)act, (const uint8_t*)w2, (const uint8_t*)s2, gs2,
                    sorted_tok, sorted_wts, seg_start, active, n_active, slot_map, out,
                    out_bf16 ? 1 : 0, T, H, I, trash, max_active, rows, w_estride, s_estride,
                    ks, ppb, (const uint16_t*)act_shared, n_shared};
  switch (fmt) {
    case kMXFP4: return launch_down_combine<kMXFP4>(a, nper, lds, stream);
    case kNVFP4: return launch_down_combine<kNVFP4>(a, nper, lds, stream);
    case kFP8: return launch_down_combine<kFP8>(a, nper, lds, stream);
    case kBF16: return launch_down_combine<kBF16>(a, nper, lds, stream);
  }
  return hipErrorInvalidValue;
}

}  // extern "C"
