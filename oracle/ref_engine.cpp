// Test-infrastructure harness over the reference xiaotu-moe CPU engine.
//
// This file is part of the oracle, not the product: it is compiled (by
// oracle/build_ref.sh) against the reference engine headers where they lie in
// the reference checkout, into oracle/_ref/, and is only loaded by tests, the
// golden-fixture generator and bench.py's CPU-baseline leg.
//
// It exposes a plain C ABI over:
//   * MOE_V2<Traits, BF16Activation>::forward_many   (xiaotu_moe/csrc/moe/moe_v2.hpp:651)
//   * Traits::gate_up_slice_batched                   (xiaotu_moe/csrc/moe/moe_v2.hpp:300)
//   * xiaotu_int8::set_activation / set_cur_tokens    (xiaotu_moe/csrc/moe/xiaotu_int8_mode.h)
// Traits: BF16WeightTraits (moe_v2.hpp:343), FP8WeightTraits (moe_v2_fp8.hpp:549),
// MXFP4WeightTraits / NVFP4WeightTraits / WNA16WeightTraits (moe_v2_packed4_*.inc).
#include <cstdint>
#include <cstdio>
#include <exception>

#include "moe/moe_v2.hpp"
#include "moe/moe_v2_fp8.hpp"
#include "moe/moe_v2_packed4.hpp"
#include "moe/xiaotu_int8_mode.h"

using namespace xiaotu_moe;

namespace {

enum Kind { kBF16 = 0, kFP8 = 1, kMXFP4 = 2, kNVFP4 = 3, kWNA16 = 4 };

struct Handle {
  int kind;
  void* eng;
  MOEConfigV2 cfg;
};

template <class WT>
using Eng = MOE_V2<WT, BF16Activation>;

template <class WT>
void* make(const MOEConfigV2& cfg, const void* w13, const void* w2, const void* s13,
           const void* s2, const float* gs13, const float* gs2) {
  return new Eng<WT>(cfg, w13, w2, s13, s2, gs13, gs2);
}

template <class WT>
void fwd(void* e, int M, int K, const uint32_t* ids, const float* wts, const uint16_t* x,
         float* out) {
  static_cast<Eng<WT>*>(e)->forward_many(M, K, ids, wts, x, out);
}

template <class WT>
void del(void* e) { delete static_cast<Eng<WT>*>(e); }

}  // namespace

extern "C" {

// Returns the compiled ISA level: 2 = AVX-512 VNNI (INT8 ALIGN path present), 1 = AVX-512, 0 = scalar.
int xref_isa() {
#if defined(__AVX512VNNI__)
  return 2;
#elif defined(__AVX512F__)
  return 1;
#else
  return 0;
#endif
}

void* xref_create(int kind, int E, int topk, int H, int I, int group_n, int group_k,
                  float swiglu_limit, float swiglu_alpha, float swiglu_beta,
                  const void* w13, const void* w2, const void* s13, const void* s2,
                  const float* gs13, const float* gs2) {
  try {
    auto* h = new Handle();
    h->kind = kind;
    MOEConfigV2& c = h->cfg;
    c.expert_num = E;
    c.top_k = topk;
    c.hidden_size = H;
    c.intermediate_size = I;
    c.groupN = group_n;
    c.groupK = group_k;
    c.swiglu_limit = swiglu_limit;
    c.swiglu_alpha = swiglu_alpha;
    c.swiglu_beta = swiglu_beta;
    c.activation_type = swiglu_limit > 0.f ? 1 : 0;
    switch (kind) {
      case kBF16: h->eng = make<BF16WeightTraits>(c, w13, w2, nullptr, nullptr, nullptr, nullptr); break;
      case kFP8: h->eng = make<FP8WeightTraits>(c, w13, w2, s13, s2, nullptr, nullptr); break;
      case kMXFP4: h->eng = make<MXFP4WeightTraits>(c, w13, w2, s13, s2, nullptr, nullptr); break;
      case kNVFP4: h->eng = make<NVFP4WeightTraits>(c, w13, w2, s13, s2, gs13, gs2); break;
      case kWNA16: h->eng = make<WNA16WeightTraits>(c, w13, w2, s13, s2, nullptr, nullptr); break;
      default: delete h; return nullptr;
    }
    return h;
  } catch (const std::exception& ex) {
    std::fprintf(stderr, "[xref] create failed: %s\n", ex.what());
    return nullptr;
  }
}

int xref_forward(void* hv, int M, int K, const uint32_t* ids, const float* wts,
                 const uint16_t* x, float* out) {
  auto* h = static_cast<Handle*>(hv);
  if (!h) return -1;
  switch (h->kind) {
    case kBF16: fwd<BF16WeightTraits>(h->eng, M, K, ids, wts, x, out); break;
    case kFP8: fwd<FP8WeightTraits>(h->eng, M, K, ids, wts, x, out); break;
    case kMXFP4: fwd<MXFP4WeightTraits>(h->eng, M, K, ids, wts, x, out); break;
    case kNVFP4: fwd<NVFP4WeightTraits>(h->eng, M, K, ids, wts, x, out); break;
    case kWNA16: fwd<WNA16WeightTraits>(h->eng, M, K, ids, wts, x, out); break;
    default: return -1;
  }
  return 0;
}

void xref_destroy(void* hv) {
  auto* h = static_cast<Handle*>(hv);
  if (!h) return;
  switch (h->kind) {
    case kBF16: del<BF16WeightTraits>(h->eng); break;
    case kFP8: del<FP8WeightTraits>(h->eng); break;
    case kMXFP4: del<MXFP4WeightTraits>(h->eng); break;
    case kNVFP4: del<NVFP4WeightTraits>(h->eng); break;
    case kWNA16: del<WNA16WeightTraits>(h->eng); break;
  }
  delete h;
}

// INT8 activation mode of the engine (1 = ALIGN) and the token count its gate reads.
void xref_set_int8(int mode, int cur_tokens) {
  xiaotu_int8::set_activation(mode);
  xiaotu_int8::set_cur_tokens(cur_tokens);
}

// Gate/up of ONE expert for `me` rows through the MXFP4 traits (dense layout):
// both[me][2I] fp32 = xg[me][H] bf16 x dequant(w13[eid])^T.
int xref_mxfp4_gate_up(int me, const uint16_t* xg, const void* w13, const void* s13,
                       float* both, int I, int H, int eid) {
#if defined(__AVX512F__)
  MXFP4WeightTraits::gate_up_slice_batched(me, xg, w13, s13, nullptr, both, I, H,
                                           (size_t)eid, 1, 32, 0, I);
  return 0;
#else
  (void)me; (void)xg; (void)w13; (void)s13; (void)both; (void)I; (void)H; (void)eid;
  return -1;
#endif
}

// Down of ONE expert for `me` rows through the MXFP4 traits: out[me][H] = act[me][I] bf16 x dequant(w2[eid])^T.
int xref_mxfp4_down(int me, const uint16_t* act, const void* w2, const void* s2, float* out,
                    int H, int I, int eid) {
#if defined(__AVX512F__)
  MXFP4WeightTraits::down_slice_batched(me, act, w2, s2, nullptr, out, H, I, (size_t)eid, 1,
                                        32, 0, H);
  return 0;
#else
  (void)me; (void)act; (void)w2; (void)s2; (void)out; (void)H; (void)I; (void)eid;
  return -1;
#endif
}

}  // extern "C"
