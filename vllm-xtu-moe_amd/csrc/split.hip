// Pool-miss split: the pairs of a batch whose expert is resident in the GPU
// pool run on the device, the others on the host engine (cpu_experts.cpp),
// and the two results are added.
//
//   xtu_pin_split    one launch: per pair, the host part (id, weight; 0 for
//                    resident or invalid ids) and the device part (slot or
//                    -1, weight or 0), plus a device hit counter
//   xtu_cpu_*        the host engine over the pinned host copy of the layer
//   xtu_cpu_decode   the stream bridge: device -> pinned copies of the rows,
//                    ids and weights, a host-function node running the
//                    engine, pinned -> device copy of its fp32 output.  Every
//                    step is a stream operation with arguments fixed when it
//                    is issued, so the sequence can be captured into a HIP
//                    graph and replayed (the host node then reruns the engine
//                    on whatever the replayed copies brought).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>
#include <vector>

#include "cpu_experts.hpp"
#include "xtu_common.hpp"

namespace {

__global__ void __launch_bounds__(256) pin_split_kernel(
    const int32_t* __restrict__ ids, const float* __restrict__ wts, int n,
    const int32_t* __restrict__ slotmap, int n_local, int32_t* __restrict__ cpu_ids,
    float* __restrict__ cpu_w, int32_t* __restrict__ part_ids, float* __restrict__ part_w,
    unsigned long long* __restrict__ hits) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  bool res = false;
  if (i < n) {
    const int id = ids[i];
    const float w = wts[i];
    const bool bad = id < 0 || id >= n_local;
    const int sl = bad ? 0 : slotmap[id];
    res = !bad && sl >= n_local;
    cpu_ids[i] = (res || bad) ? 0 : id;
    cpu_w[i] = (res || bad) ? 0.f : w;
    part_ids[i] = res ? sl - n_local : -1;
    part_w[i] = res ? w : 0.f;
  }
  if (hits) {
    const unsigned long long m = __ballot(res);
    if ((threadIdx.x & 63) == 0 && m) atomicAdd(hits, (unsigned long long)__popcll(m));
  }
}

struct CpuEngineHandle;

struct DecodeCall {
  CpuEngineHandle* h;
  int T, K;
  bool kept;   // recorded into a graph: replayed until the engine is destroyed
};

struct CpuEngineHandle {
  xtu_cpu::Engine* eng = nullptr;
  int H = 0, max_tokens = 0, max_topk = 0;
  uint16_t* pin_x = nullptr;
  int32_t* pin_ids = nullptr;
  float* pin_w = nullptr;
  float* pin_out = nullptr;
  std::mutex mu;
  std::vector<DecodeCall*> kept;
};

void decode_host_fn(void* arg) {
  DecodeCall* c = static_cast<DecodeCall*>(arg);
  CpuEngineHandle* h = c->h;
  xtu_cpu::engine_forward(h->eng, c->T, c->K, h->pin_x, h->pin_ids, h->pin_w, h->pin_out);
  if (!c->kept) delete c;
}

void free_pinned(CpuEngineHandle* h) {
  if (h->pin_x) (void)hipHostFree(h->pin_x);
  if (h->pin_ids) (void)hipHostFree(h->pin_ids);
  if (h->pin_w) (void)hipHostFree(h->pin_w);
  if (h->pin_out) (void)hipHostFree(h->pin_out);
  h->pin_x = nullptr;
  h->pin_ids = nullptr;
  h->pin_w = nullptr;
  h->pin_out = nullptr;
}

}  // namespace

extern "C" {

// The pin mask of the pool path (vllm_xiaotu_moe/pin_mask_triton.py:53-70,
// torch form :73-85; caller mixed_experts.py:2970-3100): for each of the n
// pairs, with bad = id < 0 or id >= n_local, sl = slotmap[id] and
// res = !bad && sl >= n_local (resident in slot sl - n_local):
//   cpu_ids = res||bad ? 0 : id     cpu_w = res||bad ? 0 : w
//   part_ids = res ? sl - n_local : -1      part_w = res ? w : 0
// and *hits += number of resident pairs (hits may be NULL).  Invalid ids get
// weight 0 on the host side too, so they contribute nothing anywhere.
hipError_t xtu_pin_split(const int32_t* ids, const float* wts, int n, const int32_t* slotmap,
                         int n_local, int32_t* cpu_ids, float* cpu_w, int32_t* part_ids,
                         float* part_w, unsigned long long* hits, hipStream_t stream) {
  XTU_CHECK_ARG(n >= 0 && n_local >= 0);
  if (n == 0) return hipSuccess;
  XTU_CHECK_ARG(ids && wts && slotmap && cpu_ids && cpu_w && part_ids && part_w);
  hipLaunchKernelGGL(pin_split_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, ids, wts, n,
                     slotmap, n_local, cpu_ids, cpu_w, part_ids, part_w, hits);
  return hipGetLastError();
}

// Host engine over a layer's host copy (the reference engine's CPU decode,
// xiaotu_moe/csrc/python_binding/binding.cpp:859-1296, run_moe_and_ep).
// w13_nodes / w2_nodes: ns node buffers ([expert][gate rows | up rows] and
// [expert][rows] of the node, P16; strides in bytes per expert); s13 / s2:
// packed scale groups (fp4), fp32 block scales (fp8) or fp32 [N][K/group_k]
// row scales (int4, format 4), per expert stride; gs13 / gs2: NVFP4
// second-level scales ([E][2] gate, up / [E]); group_k: int4's k per scale
// (32, 64, 128; else ignored).  isa: -1 best available, 0 portable, 2
// AVX-512.  max_tokens > 0 allocates the pinned staging that xtu_cpu_decode
// uses (max_tokens rows, max_topk pairs per row); 0 makes a host-only engine.
// The weights are read in place: they must outlive the engine.
hipError_t xtu_cpu_engine_create(int fmt, int H, int I, int n_experts, int ns,
                                 const void* const* w13_nodes, long w13_estride,
                                 const void* const* w2_nodes, long w2_estride, const void* s13,
                                 long s13_estride, const void* s2, long s2_estride,
                                 const float* gs13, const float* gs2, int group_k, float limit,
                                 float alpha, float beta, int n_threads, int isa, int max_tokens,
                                 int max_topk, void** engine) {
  XTU_CHECK_ARG(engine && w13_nodes && w2_nodes && ns >= 1 && ns <= xtu_cpu::kMaxShards);
  XTU_CHECK_ARG(w13_estride > 0 && w2_estride > 0 && s13_estride >= 0 && s2_estride >= 0);
  XTU_CHECK_ARG(max_tokens >= 0 && max_topk >= 0 && (max_tokens == 0 || max_topk > 0));
  *engine = nullptr;
  xtu_cpu::LayerDesc d;
  d.fmt = fmt;
  d.H = H;
  d.I = I;
  d.n_experts = n_experts;
  d.limit = limit;
  d.alpha = alpha;
  d.beta = beta;
  d.ns = ns;
  for (int n = 0; n < ns; ++n) {
    d.w13[n] = static_cast<const uint8_t*>(w13_nodes[n]);
    d.w2[n] = static_cast<const uint8_t*>(w2_nodes[n]);
  }
  d.w13_estride = (size_t)w13_estride;
  d.w2_estride = (size_t)w2_estride;
  d.s13 = static_cast<const uint8_t*>(s13);
  d.s2 = static_cast<const uint8_t*>(s2);
  d.s13_estride = (size_t)s13_estride;
  d.s2_estride = (size_t)s2_estride;
  d.gs13 = gs13;
  d.gs2 = gs2;
  d.group_k = group_k;
  XTU_CHECK_ARG(xtu_cpu::check_layer(d).empty());
  xtu_cpu::Engine* eng = xtu_cpu::engine_new(d, n_threads, isa);
  XTU_CHECK_ARG(eng != nullptr);
  CpuEngineHandle* h = new CpuEngineHandle;
  h->eng = eng;
  h->H = H;
  h->max_tokens = max_tokens;
  h->max_topk = max_topk;
  if (max_tokens > 0) {
    const size_t rows = (size_t)max_tokens, pairs = rows * (size_t)max_topk;
    hipError_t e = hipHostMalloc((void**)&h->pin_x, rows * H * sizeof(uint16_t), hipHostMallocDefault);
    if (e == hipSuccess)
      e = hipHostMalloc((void**)&h->pin_ids, pairs * sizeof(int32_t), hipHostMallocDefault);
    if (e == hipSuccess)
      e = hipHostMalloc((void**)&h->pin_w, pairs * sizeof(float), hipHostMallocDefault);
    if (e == hipSuccess)
      e = hipHostMalloc((void**)&h->pin_out, rows * H * sizeof(float), hipHostMallocDefault);
    if (e != hipSuccess) {
      free_pinned(h);
      xtu_cpu::engine_free(eng);
      delete h;
      return e;
    }
  }
  *engine = h;
  return hipSuccess;
}

// isa in use (0 portable, 2 AVX-512) and worker threads (callers included)
hipError_t xtu_cpu_engine_info(const void* engine, int* isa, int* threads) {
  XTU_CHECK_ARG(engine && isa && threads);
  const CpuEngineHandle* h = static_cast<const CpuEngineHandle*>(engine);
  *isa = xtu_cpu::engine_isa(h->eng);
  *threads = xtu_cpu::engine_threads(h->eng);
  return hipSuccess;
}

// Synchronous host forward on host memory: out[T][H] fp32 (every element
// written) = sum over pairs with 0 <= id < n_experts and w != 0 of
// w * expert(x).  Must not overlap an xtu_cpu_decode of the same engine
// that is still queued (they share the engine's workspace).
hipError_t xtu_cpu_forward(void* engine, int T, int K, const void* x, const int32_t* ids,
                           const float* wts, float* out) {
  XTU_CHECK_ARG(engine && T >= 0 && K >= 1);
  XTU_CHECK_ARG(T == 0 || (x && ids && wts && out));
  CpuEngineHandle* h = static_cast<CpuEngineHandle*>(engine);
  xtu_cpu::engine_forward(h->eng, T, K, static_cast<const uint16_t*>(x), ids, wts, out);
  return hipSuccess;
}

// The stream bridge (reference cpu_decode, binding.cpp:859-1296): on
// `stream`, copy x [T][H] bf16, ids and wts [T][K] from the device to the
// engine's pinned staging, run the engine in a host-function node, copy its
// fp32 [T][H] result to `out` on the device.  T <= max_tokens, K <= max_topk
// of the engine.  Allocates nothing, so it may be issued under stream
// capture; a captured call is kept (and rerun by every replay) until the
// engine is destroyed, so destroy the engine after the graphs.  Calls on one
// engine share its staging: issue them on one stream (or order them).
hipError_t xtu_cpu_decode(void* engine, int T, int K, const void* x, const int32_t* ids,
                          const float* wts, float* out, hipStream_t stream) {
  XTU_CHECK_ARG(engine);
  CpuEngineHandle* h = static_cast<CpuEngineHandle*>(engine);
  XTU_CHECK_ARG(h->pin_x && T >= 0 && K >= 1 && T <= h->max_tokens && K <= h->max_topk);
  if (T == 0) return hipSuccess;
  XTU_CHECK_ARG(x && ids && wts && out);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(stream, &cs);
  if (e != hipSuccess) return e;
  const size_t H = (size_t)h->H;
  if ((e = hipMemcpyAsync(h->pin_x, x, (size_t)T * H * sizeof(uint16_t), hipMemcpyDefault,
                          stream)) != hipSuccess)
    return e;
  if ((e = hipMemcpyAsync(h->pin_ids, ids, (size_t)T * K * sizeof(int32_t), hipMemcpyDefault,
                          stream)) != hipSuccess)
    return e;
  if ((e = hipMemcpyAsync(h->pin_w, wts, (size_t)T * K * sizeof(float), hipMemcpyDefault,
                          stream)) != hipSuccess)
    return e;
  DecodeCall* c = new DecodeCall{h, T, K, cs != hipStreamCaptureStatusNone};
  if (c->kept) {
    std::lock_guard<std::mutex> g(h->mu);
    h->kept.push_back(c);
  }
  e = hipLaunchHostFunc(stream, decode_host_fn, c);
  if (e != hipSuccess) {
    if (!c->kept) delete c;
    return e;
  }
  return hipMemcpyAsync(out, h->pin_out, (size_t)T * H * sizeof(float), hipMemcpyDefault, stream);
}

// Frees the engine, its pinned staging and its captured calls.  The caller
// has synchronised every stream that ran its xtu_cpu_decode calls and
// destroyed the graphs that captured them.
hipError_t xtu_cpu_engine_destroy(void* engine) {
  if (!engine) return hipSuccess;
  CpuEngineHandle* h = static_cast<CpuEngineHandle*>(engine);
  free_pinned(h);
  for (DecodeCall* c : h->kept) delete c;
  xtu_cpu::engine_free(h->eng);
  delete h;
  return hipSuccess;
}

}  // extern "C"
