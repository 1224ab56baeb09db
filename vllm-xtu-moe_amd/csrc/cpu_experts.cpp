// Host-side expert MLPs over the P16 host copy of a layer; the interface and
// arithmetic are described in cpu_experts.hpp.
//
// Work split: (1) the pairs are grouped by expert (ascending), (2) the token
// rows are widened to fp32 once, in the order the weight decoder produces k
// (fp4: even k of a 32-k chunk, then odd k), (3) gate/up items = (expert,
// run of 16-row panels): both panels of the same output columns, SwiGLU,
// bf16 rounding, act rows written in that same k order, (4) down items = run
// of output panels over all experts, so every output element is owned by one
// item and summed in expert order (no atomics, a fixed order).
//
// Inner kernel: one 16-row panel against a tile of token rows.  The AVX-512
// build decodes 16 weights per instruction group (e2m1 by a 16-entry
// in-register table, e4m3 through the fp16 converter, bf16 by a shift), scales
// them and feeds fp32 FMAs; the portable build decodes a row at a time.
#include "cpu_experts.hpp"

#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstring>
#include <functional>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

namespace xtu_cpu {
namespace {

// ---------------------------------------------------------------------------
// number formats
// ---------------------------------------------------------------------------
alignas(64) const float kE2M1[16] = {0.f,  0.5f,  1.f,  1.5f,  2.f,  3.f,  4.f,  6.f,
                                     -0.f, -0.5f, -1.f, -1.5f, -2.f, -3.f, -4.f, -6.f};
// int4 centred at 8 (WNA16): code c is worth c - 8
alignas(64) const float kI4[16] = {-8.f, -7.f, -6.f, -5.f, -4.f, -3.f, -2.f, -1.f,
                                   0.f,  1.f,  2.f,  3.f,  4.f,  5.f,  6.f,  7.f};
constexpr bool is_nib(int fmt) { return fmt == kMXFP4 || fmt == kNVFP4 || fmt == kINT4; }

struct Tables {
  float e4m3[256];   // OCP e4m3fn
  float e8m0[256];   // 2^(b - 127), 255 = NaN
  Tables() {
    for (int b = 0; b < 256; ++b) {
      const int s = b >> 7, e = (b >> 3) & 15, m = b & 7;
      float v;
      if (e == 15 && m == 7)
        v = NAN;
      else if (e == 0)
        v = std::ldexp((float)m, -9);
      else
        v = std::ldexp(1.f + (float)m / 8.f, e - 7);
      e4m3[b] = s ? -v : v;
      if (b == 255) {
        e8m0[b] = NAN;
      } else {
        const uint32_t bits = b ? ((uint32_t)b << 23) : 0x00400000u;
        std::memcpy(&e8m0[b], &bits, 4);
      }
    }
  }
};
const Tables kTab;

inline float bf16_value(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

inline float bf16_round(float f) {   // round to nearest even (NaN stays NaN)
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u)
    u |= 0x00400000u;
  else
    u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  std::memcpy(&f, &u, 4);
  return f;
}

inline float silu_gate(float g, float u, float limit, float alpha, float beta) {
  if (limit > 0.f) {
    g = std::min(g, limit);
    u = std::min(std::max(u, -limit), limit);
  }
  return (g / (1.f + std::exp(-alpha * g))) * (u + beta);
}

// k per super-block (one 1 KiB block of a 16-row panel) and bytes per row
constexpr int sb_k(int fmt) { return fmt == kBF16 ? 32 : (fmt == kFP8 ? 64 : 128); }
inline size_t row_bytes(int fmt, int K) {
  return fmt == kBF16 ? 2 * (size_t)K : (fmt == kFP8 ? (size_t)K : (size_t)K / 2);
}
// super-blocks per scale group of 1 KiB (fp4) and the groups of a K
constexpr int scale_ug(int fmt) { return fmt == kMXFP4 ? 16 : 8; }
inline int scale_groups(int fmt, int K) {
  return (K / 128 + scale_ug(fmt) - 1) / scale_ug(fmt);
}

// position of k in the decoder's order (fp4: a 32-k chunk is its 16 even k,
// then its 16 odd k; other formats: k order)
inline int kpos(int fmt, int k) {
  if (is_nib(fmt)) return (k & ~31) | ((k & 1) << 4) | ((k & 31) >> 1);
  return k;
}

// one 16-row panel of a [N][K] matrix of one expert
struct PanelRef {
  const uint8_t* w;   // 16 rows, K/sb_k super-blocks of 1 KiB
  const uint8_t* s;   // fp4: the panel's scale groups; fp8: fp32 scales of its 128-row block;
                      // int4: fp32 scales of its first row ([16][K/gk])
  float gs;           // NVFP4 second-level scale of the panel's rows
  int K;
  int gk;             // int4: k per scale
};

// int4: the fp32 scale of row r for the 32-k chunk starting at k0
inline float i4_scale(const PanelRef& P, int r, int k0) {
  return reinterpret_cast<const float*>(P.s)[(size_t)r * (P.K / P.gk) + k0 / P.gk];
}

// ---------------------------------------------------------------------------
// portable panel kernel: a row at a time
// ---------------------------------------------------------------------------
template <int FMT>
void decode_row(const PanelRef& P, int r, float* w) {
  const int nsb = P.K / sb_k(FMT);
  for (int sb = 0; sb < nsb; ++sb) {
    const uint8_t* blk = P.w + (size_t)sb * 1024;
    if constexpr (FMT == kINT4) {
      for (int q = 0; q < 4; ++q) {
        const uint8_t* c = blk + q * 256 + r * 16;
        const float sc = i4_scale(P, r, sb * 128 + q * 32);
        float* o = w + sb * 128 + q * 32;
        for (int j = 0; j < 16; ++j) {
          o[j] = kI4[c[j] & 15] * sc;
          o[16 + j] = kI4[c[j] >> 4] * sc;
        }
      }
    } else if constexpr (FMT == kMXFP4 || FMT == kNVFP4) {
      const uint8_t* sg = P.s + (size_t)(sb / scale_ug(FMT)) * 1024;
      for (int q = 0; q < 4; ++q) {
        const uint8_t* c = blk + q * 256 + r * 16;
        float s0, s1;
        if constexpr (FMT == kMXFP4) {
          s0 = s1 = kTab.e8m0[sg[(q * 16 + r) * 16 + sb % 16]];
        } else {
          const uint8_t* sp = sg + (q * 16 + r) * 16 + (sb % 8) * 2;
          s0 = kTab.e4m3[sp[0]] * P.gs;
          s1 = kTab.e4m3[sp[1]] * P.gs;
        }
        float* o = w + sb * 128 + q * 32;
        for (int j = 0; j < 16; ++j) {
          const float sc = j < 8 ? s0 : s1;
          o[j] = kE2M1[c[j] & 15] * sc;
          o[16 + j] = kE2M1[c[j] >> 4] * sc;
        }
      }
    } else if constexpr (FMT == kFP8) {
      const float sc = reinterpret_cast<const float*>(P.s)[sb / 2];
      for (int q = 0; q < 4; ++q) {
        const uint8_t* c = blk + q * 256 + r * 16;
        for (int j = 0; j < 16; ++j) w[sb * 64 + q * 16 + j] = kTab.e4m3[c[j]] * sc;
      }
    } else {
      for (int q = 0; q < 4; ++q) {
        const uint8_t* c = blk + q * 256 + r * 16;
        for (int j = 0; j < 8; ++j) {
          uint16_t h;
          std::memcpy(&h, c + 2 * j, 2);
          w[sb * 32 + q * 8 + j] = bf16_value(h);
        }
      }
    }
  }
}

template <int FMT>
void panel_scalar(const PanelRef& P, const float* const* xt, int nt, float* out) {
  thread_local std::vector<float> w;
  if ((int)w.size() < P.K) w.resize(P.K);
  for (int r = 0; r < 16; ++r) {
    decode_row<FMT>(P, r, w.data());
    for (int t = 0; t < nt; ++t) {
      const float* x = xt[t];
      float s = 0.f;
      for (int k = 0; k < P.K; ++k) s += w[k] * x[k];
      out[t * 16 + r] = s;
    }
  }
}

// ---------------------------------------------------------------------------
// AVX-512 panel kernel: RR rows x TT token rows in zmm accumulators
// ---------------------------------------------------------------------------
#pragma GCC push_options
#pragma GCC target("avx512f,avx512bw,avx512dq,avx512vl")

template <int FMT, int TT, int RR>
void tile512(const PanelRef& P, const float* const* xt, int r0, float* out) {
  __m512 acc[RR][TT];
  for (int a = 0; a < RR; ++a)
    for (int t = 0; t < TT; ++t) acc[a][t] = _mm512_setzero_ps();
  const int nsb = P.K / sb_k(FMT);
  if constexpr (is_nib(FMT)) {
    const __m512 lut = _mm512_load_ps(FMT == kINT4 ? kI4 : kE2M1);
    const __m512i m15 = _mm512_set1_epi32(15);
    for (int sb = 0; sb < nsb; ++sb) {
      const uint8_t* blk = P.w + (size_t)sb * 1024;
      const uint8_t* sg = FMT == kINT4 ? nullptr : P.s + (size_t)(sb / scale_ug(FMT)) * 1024;
      for (int q = 0; q < 4; ++q) {
        const int k0 = sb * 128 + q * 32;
        __m512 xa[TT], xb[TT];
        for (int t = 0; t < TT; ++t) {
          xa[t] = _mm512_loadu_ps(xt[t] + k0);
          xb[t] = _mm512_loadu_ps(xt[t] + k0 + 16);
        }
        for (int a = 0; a < RR; ++a) {
          const int r = r0 + a;
          const __m512i v = _mm512_cvtepu8_epi32(
              _mm_loadu_si128(reinterpret_cast<const __m128i*>(blk + q * 256 + r * 16)));
          __m512 wl = _mm512_permutexvar_ps(_mm512_and_si512(v, m15), lut);
          __m512 wh = _mm512_permutexvar_ps(_mm512_srli_epi32(v, 4), lut);
          __m512 sc;
          if constexpr (FMT == kINT4) {
            sc = _mm512_set1_ps(i4_scale(P, r, k0));
          } else if constexpr (FMT == kMXFP4) {
            sc = _mm512_set1_ps(kTab.e8m0[sg[(q * 16 + r) * 16 + sb % 16]]);
          } else {
            const uint8_t* sp = sg + (q * 16 + r) * 16 + (sb % 8) * 2;
            sc = _mm512_mask_blend_ps((__mmask16)0xff00, _mm512_set1_ps(kTab.e4m3[sp[0]] * P.gs),
                                      _mm512_set1_ps(kTab.e4m3[sp[1]] * P.gs));
          }
          wl = _mm512_mul_ps(wl, sc);
          wh = _mm512_mul_ps(wh, sc);
          for (int t = 0; t < TT; ++t) {
            acc[a][t] = _mm512_fmadd_ps(wl, xa[t], acc[a][t]);
            acc[a][t] = _mm512_fmadd_ps(wh, xb[t], acc[a][t]);
          }
        }
      }
    }
  } else if constexpr (FMT == kFP8) {
    // e4m3 -> fp16 bits (exponent and mantissa moved up 7 bits, sign to bit
    // 15): the fp16 value is the e4m3 value / 256, subnormals included; the
    // 256 is folded into the block scale (a power of two: no extra rounding)
    const __m512i m7f = _mm512_set1_epi32(0x7f), m80 = _mm512_set1_epi32(0x80);
    for (int sb = 0; sb < nsb; ++sb) {
      const uint8_t* blk = P.w + (size_t)sb * 1024;
      const __m512 sc = _mm512_set1_ps(256.f * reinterpret_cast<const float*>(P.s)[sb / 2]);
      for (int q = 0; q < 4; ++q) {
        const int k0 = sb * 64 + q * 16;
        __m512 xa[TT];
        for (int t = 0; t < TT; ++t) xa[t] = _mm512_loadu_ps(xt[t] + k0);
        for (int a = 0; a < RR; ++a) {
          const int r = r0 + a;
          const __m512i v = _mm512_cvtepu8_epi32(
              _mm_loadu_si128(reinterpret_cast<const __m128i*>(blk + q * 256 + r * 16)));
          const __m512i h = _mm512_or_si512(_mm512_slli_epi32(_mm512_and_si512(v, m7f), 7),
                                            _mm512_slli_epi32(_mm512_and_si512(v, m80), 8));
          const __m512 w = _mm512_mul_ps(_mm512_cvtph_ps(_mm512_cvtepi32_epi16(h)), sc);
          for (int t = 0; t < TT; ++t) acc[a][t] = _mm512_fmadd_ps(w, xa[t], acc[a][t]);
        }
      }
    }
  } else {
    for (int sb = 0; sb < nsb; ++sb) {
      const uint8_t* blk = P.w + (size_t)sb * 1024;
      for (int q2 = 0; q2 < 2; ++q2) {   // chunks 2*q2 and 2*q2+1: 16 consecutive k
        const int k0 = sb * 32 + q2 * 16;
        __m512 xa[TT];
        for (int t = 0; t < TT; ++t) xa[t] = _mm512_loadu_ps(xt[t] + k0);
        for (int a = 0; a < RR; ++a) {
          const int r = r0 + a;
          const __m128i c0 =
              _mm_loadu_si128(reinterpret_cast<const __m128i*>(blk + (2 * q2) * 256 + r * 16));
          const __m128i c1 =
              _mm_loadu_si128(reinterpret_cast<const __m128i*>(blk + (2 * q2 + 1) * 256 + r * 16));
          const __m512i v = _mm512_cvtepu16_epi32(
              _mm256_inserti128_si256(_mm256_castsi128_si256(c0), c1, 1));
          const __m512 w = _mm512_castsi512_ps(_mm512_slli_epi32(v, 16));
          for (int t = 0; t < TT; ++t) acc[a][t] = _mm512_fmadd_ps(w, xa[t], acc[a][t]);
        }
      }
    }
  }
  for (int a = 0; a < RR; ++a)
    for (int t = 0; t < TT; ++t) out[t * 16 + r0 + a] = _mm512_reduce_add_ps(acc[a][t]);
}

template <int FMT>
void panel512(const PanelRef& P, const float* const* xt, int nt, float* out) {
  int t = 0;
  for (; t + 4 <= nt; t += 4)
    for (int r0 = 0; r0 < 16; r0 += 4) tile512<FMT, 4, 4>(P, xt + t, r0, out + t * 16);
  for (; t + 2 <= nt; t += 2)
    for (int r0 = 0; r0 < 16; r0 += 8) tile512<FMT, 2, 8>(P, xt + t, r0, out + t * 16);
  for (; t < nt; ++t) tile512<FMT, 1, 16>(P, xt + t, 0, out + t * 16);
}

#pragma GCC pop_options

using PanelFn = void (*)(const PanelRef&, const float* const*, int, float*);

PanelFn pick_panel(int fmt, int isa) {
  if (isa == 2) {
    switch (fmt) {
      case kBF16: return panel512<kBF16>;
      case kFP8: return panel512<kFP8>;
      case kMXFP4: return panel512<kMXFP4>;
      case kINT4: return panel512<kINT4>;
      default: return panel512<kNVFP4>;
    }
  }
  switch (fmt) {
    case kBF16: return panel_scalar<kBF16>;
    case kFP8: return panel_scalar<kFP8>;
    case kMXFP4: return panel_scalar<kMXFP4>;
    case kINT4: return panel_scalar<kINT4>;
    default: return panel_scalar<kNVFP4>;
  }
}

bool host_has_avx512() {
  __builtin_cpu_init();
  return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
         __builtin_cpu_supports("avx512dq") && __builtin_cpu_supports("avx512vl");
}

// MXCSR with flush-to-zero and denormals-are-zero off: subnormal weights and
// products keep their value whatever mode the calling thread runs in
inline unsigned fp_mode_enter() {
  const unsigned old = _mm_getcsr();
  _mm_setcsr(old & ~0x8040u);
  return old;
}

// ---------------------------------------------------------------------------
// thread pool: run(n, f) calls f(0..n-1) on the workers and the caller
// ---------------------------------------------------------------------------
class Pool {
 public:
  explicit Pool(int n) : n_(std::max(1, n)) {
    for (int i = 1; i < n_; ++i) th_.emplace_back([this] { loop(); });
  }
  ~Pool() {
    {
      std::lock_guard<std::mutex> g(mu_);
      stop_ = true;
    }
    cv_.notify_all();
    for (auto& t : th_) t.join();
  }
  int size() const { return n_; }

  // one job at a time: engines of several layers (or streams) share a pool
  void run(int n, const std::function<void(int)>& f) {
    if (n <= 0) return;
    if (th_.empty() || n == 1) {
      for (int i = 0; i < n; ++i) f(i);
      return;
    }
    std::lock_guard<std::mutex> one(run_mu_);
    {
      std::lock_guard<std::mutex> g(mu_);
      job_ = &f;
      items_ = n;
      next_.store(0, std::memory_order_relaxed);
      busy_ = (int)th_.size();
      ++gen_;
    }
    cv_.notify_all();
    work();
    std::unique_lock<std::mutex> lk(mu_);
    done_.wait(lk, [&] { return busy_ == 0; });
    job_ = nullptr;
  }

 private:
  void work() {
    for (;;) {
      const int i = next_.fetch_add(1, std::memory_order_relaxed);
      if (i >= items_) break;
      (*job_)(i);
    }
  }
  void loop() {
    fp_mode_enter();
    uint64_t seen = 0;
    for (;;) {
      {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, [&] { return stop_ || gen_ != seen; });
        if (stop_) return;
        seen = gen_;
      }
      work();
      std::lock_guard<std::mutex> g(mu_);
      if (--busy_ == 0) done_.notify_one();
    }
  }

  const int n_;
  std::vector<std::thread> th_;
  std::mutex run_mu_, mu_;
  std::condition_variable cv_, done_;
  const std::function<void(int)>* job_ = nullptr;
  std::atomic<int> next_{0};
  int items_ = 0, busy_ = 0;
  uint64_t gen_ = 0;
  bool stop_ = false;
};

// Process-wide pools by thread count: every layer's engine would otherwise
// hold its own idle workers (58 layers x 16 threads).
std::shared_ptr<Pool> shared_pool(int n) {
  static std::mutex mu;
  static std::vector<std::pair<int, std::weak_ptr<Pool>>> pools;
  std::lock_guard<std::mutex> g(mu);
  for (auto& pw : pools)
    if (pw.first == n)
      if (auto p = pw.second.lock()) return p;
  auto p = std::make_shared<Pool>(n);
  pools.erase(std::remove_if(pools.begin(), pools.end(),
                             [](const std::pair<int, std::weak_ptr<Pool>>& q) {
                               return q.second.expired();
                             }),
              pools.end());
  pools.emplace_back(n, p);
  return p;
}

}  // namespace

// ---------------------------------------------------------------------------
// engine
// ---------------------------------------------------------------------------
struct Engine {
  LayerDesc d;
  int isa = 0;
  PanelFn panel = nullptr;
  size_t rb13 = 0, rb2 = 0, sg13 = 0, sg2 = 0;   // row bytes; scale bytes per panel
  std::shared_ptr<Pool> pool_;
  Pool& pool() { return *pool_; }
  // per-call workspace (grows, never shrinks)
  std::vector<int> cnt, start, ex, ptok;
  std::vector<float> pw, xp, act;

  Engine(const LayerDesc& desc, int threads, int isa_)
      : d(desc), isa(isa_), pool_(shared_pool(std::max(1, threads))) {
    panel = pick_panel(d.fmt, isa);
    rb13 = row_bytes(d.fmt, d.H);
    rb2 = row_bytes(d.fmt, d.I);
    if (d.fmt == kMXFP4 || d.fmt == kNVFP4) {
      sg13 = (size_t)scale_groups(d.fmt, d.H) * 1024;
      sg2 = (size_t)scale_groups(d.fmt, d.I) * 1024;
    }
  }

  // panel p (16 rows) of expert e's w13 ([2I][H]: gate panels, then up panels)
  PanelRef w13_panel(int e, int p) const {
    const int ipan = d.I / 16, ppn = ipan / d.ns;
    const bool up = p >= ipan;
    const int pp = up ? p - ipan : p, node = pp / ppn, lp = pp % ppn;
    PanelRef P;
    P.w = d.w13[node] + (size_t)e * d.w13_estride + (up ? (size_t)ppn * 16 * rb13 : 0) +
          (size_t)lp * 16 * rb13;
    P.s = scale_of(d.s13, d.s13_estride, sg13, e, p, d.H);
    P.gs = d.gs13 ? d.gs13[2 * (size_t)e + (up ? 1 : 0)] : 1.f;   // [E][2]: gate, up
    P.K = d.H;
    P.gk = d.group_k;
    return P;
  }
  // panel p of expert e's w2 ([H][I])
  PanelRef w2_panel(int e, int p) const {
    const int ppn = (d.H / 16) / d.ns, node = p / ppn, lp = p % ppn;
    PanelRef P;
    P.w = d.w2[node] + (size_t)e * d.w2_estride + (size_t)lp * 16 * rb2;
    P.s = scale_of(d.s2, d.s2_estride, sg2, e, p, d.I);
    P.gs = d.gs2 ? d.gs2[e] : 1.f;
    P.K = d.I;
    P.gk = d.group_k;
    return P;
  }
  const uint8_t* scale_of(const uint8_t* s, size_t estride, size_t sg, int e, int p, int K) const {
    if (!s) return nullptr;
    const uint8_t* base = s + (size_t)e * estride;
    if (d.fmt == kFP8) return base + (size_t)((16 * p) / 128) * (K / 128) * sizeof(float);
    if (d.fmt == kINT4) return base + (size_t)16 * p * (K / d.group_k) * sizeof(float);
    return base + (size_t)p * sg;
  }
};

std::string check_layer(const LayerDesc& d) {
  if (d.fmt < kBF16 || d.fmt > kINT4) return "unknown weight format";
  if (d.H <= 0 || d.I <= 0 || d.n_experts <= 0) return "H, I and the expert count must be positive";
  if (d.ns < 1 || d.ns > kMaxShards) return "shard count must be in [1, 8]";
  if (d.H % (16 * d.ns) || d.I % (16 * d.ns)) return "H and I must split into 16-row panels per shard";
  const int kq = sb_k(d.fmt);
  if (d.H % kq || d.I % kq) return "H and I must be whole super-blocks of k";
  if (d.fmt == kFP8 && (d.H % 128 || d.I % 128)) return "FP8 needs H and I multiples of 128";
  for (int n = 0; n < d.ns; ++n)
    if (!d.w13[n] || !d.w2[n]) return "missing weight shard";
  if (d.fmt != kBF16 && (!d.s13 || !d.s2)) return "missing scales";
  if (d.fmt == kNVFP4 && (!d.gs13 || !d.gs2)) return "missing NVFP4 global scales";
  if (d.fmt == kINT4 && !(d.group_k == 32 || d.group_k == 64 || d.group_k == 128))
    return "INT4 scale groups must be 32, 64 or 128 k";
  if (d.fmt == kINT4 && (d.H % d.group_k || d.I % d.group_k))
    return "H and I must be whole INT4 scale groups";
  return "";
}

Engine* engine_new(const LayerDesc& d, int n_threads, int isa) {
  if (!check_layer(d).empty()) return nullptr;
  const bool avx = host_has_avx512();
  if (isa == 2 && !avx) return nullptr;
  if (isa < 0) isa = avx ? 2 : 0;
  if (isa != 0 && isa != 2) return nullptr;
  if (n_threads <= 0) n_threads = (int)std::max(1u, std::thread::hardware_concurrency());
  return new Engine(d, n_threads, isa);
}

void engine_free(Engine* e) { delete e; }
int engine_isa(const Engine* e) { return e->isa; }
int engine_threads(const Engine* e) { return e->pool_->size(); }

void engine_forward(Engine* E, int T, int K, const uint16_t* x, const int32_t* ids,
                    const float* wts, float* out) {
  const LayerDesc& d = E->d;
  const int H = d.H, I = d.I, NE = d.n_experts;
  const unsigned csr = fp_mode_enter();
  if (T <= 0) {
    _mm_setcsr(csr);
    return;
  }
  // (1) pairs grouped by expert, ascending; (t, k) order inside an expert
  E->cnt.assign(NE, 0);
  int P = 0;
  for (int i = 0; i < T * K; ++i)
    if (ids[i] >= 0 && ids[i] < NE && wts[i] != 0.f) {
      ++E->cnt[ids[i]];
      ++P;
    }
  E->ex.clear();
  E->start.assign(1, 0);
  for (int e = 0; e < NE; ++e)
    if (E->cnt[e]) {
      E->ex.push_back(e);
      E->start.push_back(E->start.back() + E->cnt[e]);
    }
  const int nex = (int)E->ex.size();
  if (nex == 0) {
    std::memset(out, 0, sizeof(float) * (size_t)T * H);
    _mm_setcsr(csr);
    return;
  }
  {
    std::vector<int>& fill = E->cnt;   // reused as the write cursor of each expert
    for (int j = 0; j < nex; ++j) fill[E->ex[j]] = E->start[j];
    if ((int)E->ptok.size() < P) {
      E->ptok.resize(P);
      E->pw.resize(P);
    }
    for (int i = 0; i < T * K; ++i)
      if (ids[i] >= 0 && ids[i] < NE && wts[i] != 0.f) {
        const int at = fill[ids[i]]++;
        E->ptok[at] = i / K;
        E->pw[at] = wts[i];
      }
  }
  if (E->xp.size() < (size_t)T * H) E->xp.resize((size_t)T * H);
  if (E->act.size() < (size_t)P * I) E->act.resize((size_t)P * I);
  const int fmt = d.fmt;
  float* xp = E->xp.data();
  float* act = E->act.data();
  const int nthr = E->pool().size();

  // (2) token rows to fp32 in the decoder's k order
  E->pool().run(T, [&](int t) {
    const uint16_t* xr = x + (size_t)t * H;
    float* o = xp + (size_t)t * H;
    for (int k = 0; k < H; ++k) o[kpos(fmt, k)] = bf16_value(xr[k]);
  });

  // (3) gate/up + SwiGLU: items of `pg` panels of one expert
  const int ipan = I / 16;
  const int pg = std::max(1, std::min(8, (nex * ipan) / (4 * nthr)));
  const int gchunks = (ipan + pg - 1) / pg;
  E->pool().run(nex * gchunks, [&](int item) {
    const int j = item / gchunks, c = item % gchunks;
    const int e = E->ex[j], p0 = E->start[j], nt = E->start[j + 1] - p0;
    thread_local std::vector<const float*> xt;
    thread_local std::vector<float> g, u;
    xt.resize(nt);
    g.resize((size_t)nt * 16);
    u.resize((size_t)nt * 16);
    for (int i = 0; i < nt; ++i) xt[i] = xp + (size_t)E->ptok[p0 + i] * H;
    for (int p = c * pg; p < std::min(ipan, (c + 1) * pg); ++p) {
      E->panel(E->w13_panel(e, p), xt.data(), nt, g.data());
      E->panel(E->w13_panel(e, ipan + p), xt.data(), nt, u.data());
      for (int i = 0; i < nt; ++i) {
        float* ar = act + (size_t)(p0 + i) * I;
        for (int r = 0; r < 16; ++r)
          ar[kpos(fmt, 16 * p + r)] =
              bf16_round(silu_gate(g[i * 16 + r], u[i * 16 + r], d.limit, d.alpha, d.beta));
      }
    }
  });

  // (4) down + weighted sum: items of `pd` output panels over all experts
  const int hpan = H / 16;
  const int pd = std::max(1, std::min(8, hpan / (4 * nthr)));
  const int dchunks = (hpan + pd - 1) / pd;
  E->pool().run(dchunks, [&](int c) {
    const int q0 = c * pd, q1 = std::min(hpan, (c + 1) * pd);
    for (int t = 0; t < T; ++t)
      std::memset(out + (size_t)t * H + 16 * q0, 0, sizeof(float) * 16 * (q1 - q0));
    thread_local std::vector<const float*> at;
    thread_local std::vector<float> y;
    for (int j = 0; j < nex; ++j) {
      const int e = E->ex[j], p0 = E->start[j], nt = E->start[j + 1] - p0;
      at.resize(nt);
      y.resize((size_t)nt * 16);
      for (int i = 0; i < nt; ++i) at[i] = act + (size_t)(p0 + i) * I;
      for (int p = q0; p < q1; ++p) {
        E->panel(E->w2_panel(e, p), at.data(), nt, y.data());
        for (int i = 0; i < nt; ++i) {
          float* o = out + (size_t)E->ptok[p0 + i] * H + 16 * p;
          const float w = E->pw[p0 + i];
          for (int r = 0; r < 16; ++r) o[r] += w * y[i * 16 + r];
        }
      }
    }
  });
  _mm_setcsr(csr);
}

}  // namespace xtu_cpu
