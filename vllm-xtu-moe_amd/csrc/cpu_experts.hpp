// Host-side expert MLPs over the pinned host copy of a layer (the CPU half of
// the pool-miss split).
//
// The weights are read where the host store keeps them: the P16 panel layout
// the device kernels use (16-row panels, each (panel, super-block) 1 KiB as
// [4 chunk][16 row][16 B]), cut into NUMA-node shards (node n holds gate rows
// [n*I/ns, (n+1)*I/ns) and the matching up rows of w13, and rows
// [n*H/ns, (n+1)*H/ns) of w2, for every expert), with one copy of the packed
// scales.  No second host copy is made.
//
// Arithmetic: dequantised weights (exactly: e2m1 x e8m0, e2m1 x fp32(e4m3 x
// global), e4m3 x fp32 block scale, bf16, (int4 code - 8) x fp32 group scale)
// times fp32(x) summed in fp32; the
// clamped SwiGLU activation rounded to bf16 (as the reference engine stores
// it); down in fp32; out[t] = sum over the token's pairs of w * y, the pairs
// taken in ascending expert order (a fixed order: results do not depend on
// the thread count or schedule).
#pragma once
#include <cstddef>
#include <cstdint>
#include <string>

namespace xtu_cpu {

enum { kBF16 = 0, kFP8 = 1, kMXFP4 = 2, kNVFP4 = 3, kINT4 = 4 };
constexpr int kMaxShards = 8;

struct LayerDesc {
  int fmt = 0, H = 0, I = 0, n_experts = 0;
  float limit = 0.f, alpha = 1.f, beta = 0.f;
  int ns = 1;
  const uint8_t* w13[kMaxShards] = {};     // node n: [expert][gate rows | up rows], P16
  const uint8_t* w2[kMaxShards] = {};      // node n: [expert][rows], P16
  size_t w13_estride = 0, w2_estride = 0;  // bytes per expert inside a node buffer
  const uint8_t* s13 = nullptr;            // fp4: packed scale groups; fp8: fp32 [2I/128][H/128];
                                           // int4: fp32 [2I][H/group_k]
  const uint8_t* s2 = nullptr;             // likewise for [H][I]
  int group_k = 0;                         // int4: k per scale (32, 64 or 128)
  size_t s13_estride = 0, s2_estride = 0;  // bytes per expert
  const float* gs13 = nullptr;             // NVFP4 second-level scales [E][2]: gate, up
  const float* gs2 = nullptr;              // NVFP4 second-level scales [E]
};

// Empty string when the description is usable, else what is wrong.
std::string check_layer(const LayerDesc& d);

struct Engine;

// isa: -1 = best the host supports, 0 = portable scalar code, 2 = AVX-512.
Engine* engine_new(const LayerDesc& d, int n_threads, int isa);
void engine_free(Engine* e);
int engine_isa(const Engine* e);
int engine_threads(const Engine* e);

// out[T][H] (fp32, every element written) = sum over pairs (t, k) with
// 0 <= ids[t*K+k] < n_experts and wts[t*K+k] != 0 of wts * expert(x[t]).
// x: bf16 bits [T][H].  Not reentrant per engine.
void engine_forward(Engine* e, int T, int K, const uint16_t* x, const int32_t* ids,
                    const float* wts, float* out);

}  // namespace xtu_cpu
