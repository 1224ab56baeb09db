/*
 * xtu_oracle.c -- CPU restatement of the quantized MoE expert path (TEST
 * INFRASTRUCTURE ONLY).
 *
 * This file is the checker, never the product.  Only tests/, the smoke check
 * and bench.py's CPU-baseline leg load it.  Every function cites the
 * reference file:line whose behaviour it restates.
 *
 * Build: oracle/build_ref.sh (gcc -O2 -ffp-contract=off; no fast-math, so the
 * fp32 operation sequence below is exactly what executes).
 *
 * Parity status of each function (how it is pinned; tests/test_oracle_*.py):
 *   codecs (e2m1/e8m0/e4m3/bf16)     exhaustive closed forms + torch float8 decode
 *   xo_expf / xo_sigmoid             within 2 ulp of libm expf over a dense sweep
 *   routers                          brute force (sort-based) on tiny E; textbook
 *   xo_segment                       numpy stable argsort restatement + brute force
 *   xo_moe_layer (bf16/fp8/mxfp4/nvfp4/int4) vs the compiled reference
 *                                    engine (oracle/_ref) forward_many, rel
 *                                    err ~1e-6 (int4: MOE_WNA16 traits)
 *   xo_i8_* (INT8 ALIGN)             int32 accumulators bit-exact against an
 *                                    int64 closed form built from the codec
 *                                    tables (brute force); the layer (marked
 *                                    rows' fp32 fallback included) against the
 *                                    compiled reference engine with the ALIGN
 *                                    gate on, within the layer tolerance (the
 *                                    engine's lane-sum order differs, so C is
 *                                    not bit-exact); the offset guard's fp32
 *                                    rows against an engine fixture whose every
 *                                    tile fails that guard
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* codecs                                                                    */
/* ------------------------------------------------------------------------ */

/* e2m1 table, low nibble = even k (vllm_xiaotu_moe/gpu_prefill.py:45-48,
 * xiaotu_moe/csrc/moe/moe_v2_packed4_w4a8.inc:195-199). */
static const float kE2M1[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                                -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

float xo_e2m1(int nib) { return kE2M1[nib & 15]; }

/* e8m0: 2^(b-127) (moe_v2_packed4_w4a8.inc:258-262; b=255 gives +inf there). */
float xo_e8m0(int b) { return ldexpf(1.0f, (b & 255) - 127); }

/* e4m3fn byte -> f32 (vllm_xiaotu_moe/gpu_prefill_fp8.py:33-48): normal =
 * bits ((e+120)<<23)|(m<<20); subnormal m*2^-9; 0x7f/0xff (NaN) are never fed. */
float xo_e4m3(int b) {
  const uint32_t i = (uint32_t)b & 255u;
  const uint32_t e = (i >> 3) & 15u, m = i & 7u;
  float v;
  if (e == 0) {
    v = (float)m * 1.953125e-03f;
  } else {
    uint32_t bits = ((e + 120u) << 23) | (m << 20);
    memcpy(&v, &bits, 4);
  }
  return (i >> 7) ? -v : v;
}

float xo_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* Round-to-nearest-even f32 -> bf16, NaN kept quiet
 * (xiaotu_moe/csrc/kernels/bf16_gemm.hpp convert_f32_to_bf16). */
uint16_t xo_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static float bf16_round(float f) { return xo_bf16_to_f32(xo_f32_to_bf16(f)); }

/* ------------------------------------------------------------------------ */
/* exp / sigmoid: the build's own fp32 formula, restated operation by        */
/* operation from the device code (vllm-xtu-moe_amd/csrc/xtu_common.hpp,    */
/* xtu_expf / xtu_sigmoid).                                                  */
/* Cody-Waite reduction x = k ln2 + r, |r| <= ln2/2, degree-7 Taylor in r,   */
/* Horner with fused multiply-add, scale by 2^k through the exponent field.  */
/* ------------------------------------------------------------------------ */
float xo_expf(float x) {
  if (!(x == x)) return x;
  if (x > 88.5f) return INFINITY;
  if (x < -87.0f) return 0.0f;
  const float kLog2e = 1.44269504088896341f;
  const float kLn2Hi = 0.693145751953125f;     /* 12 significant bits: k*hi exact */
  const float kLn2Lo = 1.42860682030941723e-06f;
  const float k = rintf(x * kLog2e);
  float r = fmaf(-k, kLn2Hi, x);
  r = fmaf(-k, kLn2Lo, r);
  float p = 1.98412698412698413e-04f;          /* 1/5040 */
  p = fmaf(p, r, 1.38888888888888889e-03f);    /* 1/720 */
  p = fmaf(p, r, 8.33333333333333333e-03f);    /* 1/120 */
  p = fmaf(p, r, 4.16666666666666667e-02f);    /* 1/24 */
  p = fmaf(p, r, 1.66666666666666667e-01f);    /* 1/6 */
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int ki = (int)k;                       /* in [-126, 128) here */
  /* 2^k split in two factors so k = -126 .. 127 stays normal. */
  const int k1 = ki / 2, k2 = ki - k1;
  uint32_t b1 = (uint32_t)(k1 + 127) << 23, b2 = (uint32_t)(k2 + 127) << 23;
  float s1, s2;
  memcpy(&s1, &b1, 4);
  memcpy(&s2, &b2, 4);
  return (p * s1) * s2;
}

float xo_sigmoid(float x) { return 1.0f / (1.0f + xo_expf(-x)); }

/* ------------------------------------------------------------------------ */
/* routers (a1).  The reference hands routing to vLLM's router factory      */
/* (vllm_xiaotu_moe/mixed_experts.py:994-1078, hybrid_model.py:1877), which  */
/* is not vendored; these are the textbook formulas with a fixed fp32        */
/* sequence and a fixed tie-break (larger score first, then lower index).    */
/* ------------------------------------------------------------------------ */

/* a better than b under (score desc, index asc) */
static int better(float sa, int ia, float sb, int ib) {
  return (sa > sb) || (sa == sb && ia < ib);
}

/* Mixtral / Qwen3: softmax over E, top-K, renormalised over the K chosen.
 * Selection on logits (monotone in the softmax); weights
 *   e_i = exp(l_i - l_max),  w_i = e_i / (e_0 + e_1 + ... + e_{K-1})
 * summed in selection order.  renormalize == 0: w_i = e_i / sum_all where
 * sum_all adds e_0..e_{E-1} in index order. */
int xo_route_softmax_topk(const float* logits, int T, int E, int K, int renormalize,
                          int32_t* ids, float* wts) {
  if (E < 1 || K < 1 || K > 64 || K > E) return -1;
  int sel[64];
  for (int t = 0; t < T; ++t) {
    const float* l = logits + (size_t)t * E;
    for (int k = 0; k < K; ++k) {
      int best = -1;
      for (int e = 0; e < E; ++e) {
        int used = 0;
        for (int j = 0; j < k; ++j) used |= (sel[j] == e);
        if (used) continue;
        if (best < 0 || better(l[e], e, l[best], best)) best = e;
      }
      sel[k] = best;
    }
    const float lmax = l[sel[0]];
    float ev[64];
    float s = 0.0f;
    for (int k = 0; k < K; ++k) {
      ev[k] = xo_expf(l[sel[k]] - lmax);
      s = s + ev[k];
    }
    if (!renormalize) {
      s = 0.0f;
      for (int e = 0; e < E; ++e) s = s + xo_expf(l[e] - lmax);
    }
    for (int k = 0; k < K; ++k) {
      ids[(size_t)t * K + k] = sel[k];
      wts[(size_t)t * K + k] = ev[k] / s;
    }
  }
  return 0;
}

/* DeepSeek-V3 grouped sigmoid routing:
 *   s_i = sigmoid(l_i); b_i = s_i + bias_i (selection only)
 *   group score g_j = (largest b in group j) + (second largest)
 *   keep the topk_group best groups, then the K best b_i inside them
 *   w_i = s_i / (s_0 + ... + s_{K-1}) * routed_scaling   (renormalize)
 *   w_i = s_i * routed_scaling                          (renormalize == 0) */
int xo_route_grouped_sigmoid(const float* logits, const float* bias, int T, int E,
                             int n_group, int topk_group, int K, float routed_scaling,
                             int renormalize, int32_t* ids, float* wts) {
  if (E < 1 || E > 1024 || n_group < 1 || n_group > 64 || E % n_group || K < 1 || K > 64 ||
      topk_group < 1 || topk_group > n_group || K > topk_group * (E / n_group))
    return -1;
  const int gsz = E / n_group;
  float s[1024], b[1024], g[64];
  int gsel[64], sel[64];
  for (int t = 0; t < T; ++t) {
    const float* l = logits + (size_t)t * E;
    for (int e = 0; e < E; ++e) {
      s[e] = xo_sigmoid(l[e]);
      b[e] = s[e] + (bias ? bias[e] : 0.0f);
    }
    for (int j = 0; j < n_group; ++j) {
      int i1 = -1, i2 = -1;
      for (int q = 0; q < gsz; ++q) {
        const int e = j * gsz + q;
        if (i1 < 0 || better(b[e], e, b[i1], i1)) {
          i2 = i1;
          i1 = e;
        } else if (i2 < 0 || better(b[e], e, b[i2], i2)) {
          i2 = e;
        }
      }
      g[j] = (gsz >= 2) ? (b[i1] + b[i2]) : b[i1];
    }
    for (int k = 0; k < topk_group; ++k) {
      int best = -1;
      for (int j = 0; j < n_group; ++j) {
        int used = 0;
        for (int q = 0; q < k; ++q) used |= (gsel[q] == j);
        if (used) continue;
        if (best < 0 || better(g[j], j, g[best], best)) best = j;
      }
      gsel[k] = best;
    }
    for (int k = 0; k < K; ++k) {
      int best = -1;
      for (int e = 0; e < E; ++e) {
        int ok = 0;
        for (int q = 0; q < topk_group; ++q) ok |= (gsel[q] == e / gsz);
        if (!ok) continue;
        for (int q = 0; q < k; ++q) ok &= (sel[q] != e);
        if (!ok) continue;
        if (best < 0 || better(b[e], e, b[best], best)) best = e;
      }
      sel[k] = best;
    }
    float sum = 0.0f;
    for (int k = 0; k < K; ++k) sum = sum + s[sel[k]];
    for (int k = 0; k < K; ++k) {
      ids[(size_t)t * K + k] = sel[k];
      wts[(size_t)t * K + k] =
          renormalize ? (s[sel[k]] / sum) * routed_scaling : s[sel[k]] * routed_scaling;
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* permutation / segmentation (a2), vllm_xiaotu_moe/gpu_prefill.py:849-887.  */
/* Flat pair a = t*K + k for routed pairs; shared-expert pairs follow as     */
/* a = T*K + t*n_shared + s with bucket E + s and weight 1.  Invalid ids     */
/* (<0 or >=E) -- and, when drop_zero, zero-weight pairs -- go to the trash  */
/* bucket E + n_shared.  Stable order by bucket.  Outputs:                   */
/*   sorted_pair[A]  flat pair at each sorted position                       */
/*   sorted_tok[A], sorted_wts[A]                                            */
/*   inv[A]          sorted position of each flat pair                       */
/*   seg_start[NB+1] exclusive cumsum of bucket counts, NB = E+n_shared+1    */
/* ------------------------------------------------------------------------ */
int xo_segment(const int32_t* ids, const float* wts, int T, int K, int E, int n_shared,
               int drop_zero, int32_t* sorted_pair, int32_t* sorted_tok, float* sorted_wts,
               int32_t* inv, int32_t* seg_start) {
  const int A = T * K + T * n_shared;
  const int NB = E + n_shared + 1;
  int32_t* bucket = (int32_t*)malloc(sizeof(int32_t) * (size_t)(A > 0 ? A : 1));
  int32_t* cnt = (int32_t*)calloc((size_t)NB, sizeof(int32_t));
  if (!bucket || !cnt) {
    free(bucket);
    free(cnt);
    return -1;
  }
  for (int a = 0; a < A; ++a) {
    int bk;
    if (a < T * K) {
      const int e = ids[a];
      bk = (e < 0 || e >= E) ? (E + n_shared) : e;
      if (drop_zero && wts[a] == 0.0f) bk = E + n_shared;
    } else {
      bk = E + (a - T * K) % (n_shared > 0 ? n_shared : 1);
    }
    bucket[a] = bk;
    cnt[bk]++;
  }
  seg_start[0] = 0;
  for (int b = 0; b < NB; ++b) seg_start[b + 1] = seg_start[b] + cnt[b];
  for (int b = 0; b < NB; ++b) cnt[b] = seg_start[b];
  for (int a = 0; a < A; ++a) {
    const int p = cnt[bucket[a]]++;
    sorted_pair[p] = a;
    inv[a] = p;
    if (a < T * K) {
      sorted_tok[p] = a / K;
      sorted_wts[p] = wts[a];
    } else {
      sorted_tok[p] = (a - T * K) / (n_shared > 0 ? n_shared : 1);
      sorted_wts[p] = 1.0f;
    }
  }
  free(bucket);
  free(cnt);
  return A;
}

/* ------------------------------------------------------------------------ */
/* expert math (a3-a5, a7): MOE_V2::forward_many semantics                   */
/* (xiaotu_moe/csrc/moe/moe_v2.hpp:651-957):                                 */
/*   gate/up fp32 = x . dequant(W13) (gate rows [0,I), up rows [I,2I))       */
/*   act = silu_gate_one(g, u, limit, alpha, beta) (moe_v2.hpp:180-188)      */
/*   act rounded to bf16 (moe_v2.hpp:906,955)                                */
/*   down fp32 = bf16(act) . dequant(W2)                                     */
/*   out[t] += w * down, r = 0..K-1 in order, skipping id >= E or w == 0     */
/*   (moe_v2.hpp:920-930); shared experts are extra pairs of weight 1 added  */
/*   after the routed ones.                                                  */
/* Dot products accumulate in double (the exact dequantized-fp32 result up   */
/* to one final rounding).                                                   */
/* Weight formats, dense checkpoint layout:                                  */
/*   0 BF16 : w13 [E][2I][H] bf16, w2 [E][H][I] bf16                         */
/*   1 FP8  : w13 [E][2I][H] e4m3, s13 [E][2I/128][H/128] f32 (w2 alike)     */
/*   2 MXFP4: w13 [E][2I][H/2] e2m1 (low nibble even k), s13 [E][2I][H/32]   */
/*            e8m0 (moe_v2_packed4_w4a8.inc:1966-2003)                        */
/*   3 NVFP4: as MXFP4 with s13 [E][2I][H/16] e4m3 bytes and fp32 second-   */
/*            level scales gs13 [E][2] (gate rows, up rows) and gs2 [E]      */
/*            (hybrid_model.py:1546-1561 folds them into the group scales;   */
/*            gpu_prefill.py:111-127, 290-297)                               */
/*   4 INT4 (WNA16): nibbles as MXFP4, value = nibble - 8, times an fp32     */
/*            scale s13 [E][2I][H/gk] (moe_v2_packed4_base.inc:4-16, :1594)  */
/* ------------------------------------------------------------------------ */
enum { XO_BF16 = 0, XO_FP8 = 1, XO_MXFP4 = 2, XO_NVFP4 = 3, XO_INT4 = 4 };

/* dequantize row n (of N) of one expert's [N][K] weight into out[K]; gk is
 * INT4's k per scale, g the row's NVFP4 second-level scale */
static void deq_row(int fmt, int gk, const void* w, const void* s, float g, int e, int N,
                    int K, int n, float* out) {
  if (fmt == XO_INT4) {
    const uint8_t* r = (const uint8_t*)w + ((size_t)e * N + n) * (K / 2);
    const float* sc = (const float*)s + ((size_t)e * N + n) * (K / gk);
    for (int k = 0; k < K; ++k) {
      const int nib = (k & 1) ? (r[k / 2] >> 4) : (r[k / 2] & 15);
      out[k] = (float)(nib - 8) * sc[k / gk];
    }
    return;
  }
  if (fmt == XO_BF16) {
    const uint16_t* r = (const uint16_t*)w + ((size_t)e * N + n) * K;
    for (int k = 0; k < K; ++k) out[k] = xo_bf16_to_f32(r[k]);
  } else if (fmt == XO_FP8) {
    const uint8_t* r = (const uint8_t*)w + ((size_t)e * N + n) * K;
    const float* sc = (const float*)s + (size_t)e * (N / 128) * (K / 128) + (size_t)(n / 128) * (K / 128);
    for (int k = 0; k < K; ++k) out[k] = xo_e4m3(r[k]) * sc[k / 128];
  } else {
    const uint8_t* r = (const uint8_t*)w + ((size_t)e * N + n) * (K / 2);
    const int gk = (fmt == XO_MXFP4) ? 32 : 16;
    const uint8_t* sc = (const uint8_t*)s + ((size_t)e * N + n) * (K / gk);
    for (int k = 0; k < K; ++k) {
      const int nib = (k & 1) ? (r[k / 2] >> 4) : (r[k / 2] & 15);
      const float scale = (fmt == XO_MXFP4) ? xo_e8m0(sc[k / gk]) : xo_e4m3(sc[k / gk]) * g;
      out[k] = kE2M1[nib] * scale;
    }
  }
}

/* silu_gate_one (moe_v2.hpp:180-188): gate clamped above only, up both sides */
float xo_silu_gate(float g, float u, float limit, float alpha, float beta) {
  if (limit > 0.f) {
    if (g > limit) g = limit;
    if (u > limit) u = limit;
    else if (u < -limit) u = -limit;
  }
  return (g / (1.f + expf(-alpha * g))) * (u + beta);
}

/* One expert applied to one bf16 row x[H]: y[H] (fp32). Also returns the bf16
 * activation row (act_out[I], may be NULL). */
static void expert_row(int fmt, int gk, const void* w13, const void* s13, const float* gs13,
                       const void* w2, const void* s2, const float* gs2, int e, int H, int I,
                       const float* xf, float limit, float alpha, float beta, float* wrow,
                       float* actf, float* y) {
  const int nv = fmt == XO_NVFP4;
  const float g_gate = nv && gs13 ? gs13[2 * (size_t)e] : 1.0f;
  const float g_up = nv && gs13 ? gs13[2 * (size_t)e + 1] : 1.0f;
  const float g_down = nv && gs2 ? gs2[e] : 1.0f;
  for (int i = 0; i < I; ++i) {
    double g = 0.0, u = 0.0;
    deq_row(fmt, gk, w13, s13, g_gate, e, 2 * I, H, i, wrow);
    for (int k = 0; k < H; ++k) g += (double)xf[k] * wrow[k];
    deq_row(fmt, gk, w13, s13, g_up, e, 2 * I, H, I + i, wrow);
    for (int k = 0; k < H; ++k) u += (double)xf[k] * wrow[k];
    actf[i] = bf16_round(xo_silu_gate((float)g, (float)u, limit, alpha, beta));
  }
  for (int h = 0; h < H; ++h) {
    double d = 0.0;
    deq_row(fmt, gk, w2, s2, g_down, e, H, I, h, wrow);
    for (int i = 0; i < I; ++i) d += (double)actf[i] * wrow[i];
    y[h] = (float)d;
  }
}

/* Full layer: out[T][H] fp32.  Experts [0,E) routed, [E, E+n_shared) shared
 * (weight 1, after the routed pairs).  gk: INT4's k per scale (ignored for
 * the other formats).  Returns 0 on success. */
int xo_moe_layer_g(int fmt, int gk, int T, int K, int E, int n_shared, int H, int I,
                   const uint16_t* x, const int32_t* ids, const float* wts, const void* w13,
                   const void* s13, const float* gs13, const void* w2, const void* s2,
                   const float* gs2, float limit, float alpha, float beta, float* out) {
  if (fmt == XO_INT4 && (gk <= 0 || H % gk || I % gk)) return -1;
  const int mx = H > I ? H : I;
  float* xf = (float*)malloc(sizeof(float) * (size_t)H);
  float* wrow = (float*)malloc(sizeof(float) * (size_t)mx);
  float* actf = (float*)malloc(sizeof(float) * (size_t)I);
  float* y = (float*)malloc(sizeof(float) * (size_t)H);
  if (!xf || !wrow || !actf || !y) {
    free(xf); free(wrow); free(actf); free(y);
    return -1;
  }
  for (int t = 0; t < T; ++t) {
    float* o = out + (size_t)t * H;
    for (int h = 0; h < H; ++h) o[h] = 0.f;
    for (int k = 0; k < H; ++k) xf[k] = xo_bf16_to_f32(x[(size_t)t * H + k]);
    for (int r = 0; r < K + n_shared; ++r) {
      int e;
      float w;
      if (r < K) {
        e = ids[(size_t)t * K + r];
        w = wts[(size_t)t * K + r];
        if (e < 0 || e >= E || w == 0.f) continue;
      } else {
        e = E + (r - K);
        w = 1.0f;
      }
      expert_row(fmt, gk, w13, s13, gs13, w2, s2, gs2, e, H, I, xf, limit, alpha, beta, wrow,
                 actf, y);
      for (int h = 0; h < H; ++h) o[h] += w * y[h];
    }
  }
  free(xf); free(wrow); free(actf); free(y);
  return 0;
}

int xo_moe_layer(int fmt, int T, int K, int E, int n_shared, int H, int I,
                 const uint16_t* x, const int32_t* ids, const float* wts, const void* w13,
                 const void* s13, const float* gs13, const void* w2, const void* s2,
                 const float* gs2, float limit, float alpha, float beta, float* out) {
  return xo_moe_layer_g(fmt, 0, T, K, E, n_shared, H, I, x, ids, wts, w13, s13, gs13, w2, s2,
                        gs2, limit, alpha, beta, out);
}

/* ------------------------------------------------------------------------ */
/* INT8-activation x FP4-code ALIGN path (a6),                               */
/* xiaotu_moe/csrc/moe/moe_v2_packed4_w4a8.inc:                              */
/*   row exponent  :661-676  crow = (ef-127) - 6 + [mant(m) > 0x7E0000],     */
/*                           clamp [-120,120]; m = max|a| over the row       */
/*   a8            :676-714  clamp(rne(a * 2^-crow), -127, 127)              */
/*   w4            :448-456  2*e2m1 in {0,+-1,+-2,+-3,+-4,+-6,+-8,+-12}      */
/*   shift         :545-556  w8' = w4 << (b - emin_j), emin_j = min_g b      */
/*   accumulate    :811-858  ACC = sum a8*w8' (int32 exact)                  */
/*   output        :855-858  C = float(ACC) * (gs * 2^(emin-128)) * 2^crow   */
/* ------------------------------------------------------------------------ */
static const int kW4[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

int xo_i8_quant_row(const float* a, int K, int8_t* a8) {
  float m = 0.f;
  for (int k = 0; k < K; ++k) {
    const float v = fabsf(a[k]);
    if (v > m) m = v;
  }
  int crow = 0;
  if (m > 0.f) {
    uint32_t b;
    memcpy(&b, &m, 4);
    const int ef = (int)((b >> 23) & 0xFFu);
    if (ef == 0xFF) crow = 120;
    else if (ef == 0) crow = -120;
    else crow = (ef - 127) - 6 + (((b & 0x7FFFFFu) > 8257536u) ? 1 : 0);
    if (crow < -120) crow = -120;
    if (crow > 120) crow = 120;
  }
  uint32_t pb = (uint32_t)(127 - crow) << 23;
  float inv;
  memcpy(&inv, &pb, 4);
  for (int k = 0; k < K; ++k) {
    float q = rintf(a[k] * inv);
    if (q < -127.f) q = -127.f;
    if (q > 127.f) q = 127.f;
    a8[k] = (int8_t)q;
  }
  return crow;
}

/* Weight row n of one MXFP4 expert matrix [N][K/2] + e8m0 [N][K/32]:
 * w8'[K] and emin; returns the row's largest shift d (ALIGN needs <= 3). */
int xo_i8_weight_row(const uint8_t* wrow, const uint8_t* srow, int K, int8_t* w8, int* emin) {
  int mn = 255, dmax = 0;
  for (int g = 0; g < K / 32; ++g)
    if (srow[g] < mn) mn = srow[g];
  for (int g = 0; g < K / 32; ++g) {
    const int d = srow[g] - mn;
    if (d > dmax) dmax = d;
    for (int q = 0; q < 32; ++q) {
      const int k = g * 32 + q;
      const int nib = (k & 1) ? (wrow[k / 2] >> 4) : (wrow[k / 2] & 15);
      w8[k] = (int8_t)(kW4[nib] * (1 << d));
    }
  }
  *emin = mn;
  return dmax;
}

/* One INT8 GEMM of M activation rows against N MXFP4 weight rows:
 *   acc[M][N] int32 (exact), c[M][N] fp32.  a: [M][K] fp32 values, w: [N][K/2],
 *   s: [N][K/32].  Returns the largest row shift seen (ALIGN gate: <= 3). */
int xo_i8_gemm(const float* a, int M, const uint8_t* w, const uint8_t* s, int N, int K,
               float gs, int32_t* acc, float* c) {
  int8_t* a8 = (int8_t*)malloc((size_t)M * K);
  int* crow = (int*)malloc(sizeof(int) * (size_t)M);
  int8_t* w8 = (int8_t*)malloc((size_t)K);
  int dmax = 0;
  if (!a8 || !crow || !w8) {
    free(a8); free(crow); free(w8);
    return -1;
  }
  for (int m = 0; m < M; ++m) crow[m] = xo_i8_quant_row(a + (size_t)m * K, K, a8 + (size_t)m * K);
  for (int n = 0; n < N; ++n) {
    int emin;
    const int d = xo_i8_weight_row(w + (size_t)n * (K / 2), s + (size_t)n * (K / 32), K, w8, &emin);
    if (d > dmax) dmax = d;
    const float dw = gs * ldexpf(1.0f, emin - 128);
    for (int m = 0; m < M; ++m) {
      int64_t sacc = 0;
      const int8_t* ar = a8 + (size_t)m * K;
      for (int k = 0; k < K; ++k) sacc += (int64_t)ar[k] * w8[k];
      acc[(size_t)m * N + n] = (int32_t)sacc;
      c[(size_t)m * N + n] = (float)sacc * (dw * ldexpf(1.0f, crow[m]));
    }
  }
  free(a8); free(crow); free(w8);
  return dmax;
}

/* e8m0 spread of one MXFP4 weight row (its K/32 scale bytes): max - min. */
int xo_i8_row_spread(const uint8_t* srow, int K) {
  int mn = 255, mx = 0;
  for (int g = 0; g < K / 32; ++g) {
    if (srow[g] < mn) mn = srow[g];
    if (srow[g] > mx) mx = srow[g];
  }
  return mx - mn;
}

/* fp32-path dot of a[K] with dequantized MXFP4 weight row n of [N][K] */
static float i8_fallback_dot(const float* a, const uint8_t* w, const uint8_t* s, int N, int K,
                             int n, float* wrow) {
  double d = 0.0;
  deq_row(XO_MXFP4, 0, w, s, 1.0f, 0, N, K, n, wrow);
  for (int k = 0; k < K; ++k) d += (double)a[k] * wrow[k];
  return (float)d;
}

/* Smallest e8m0 byte of one MXFP4 expert matrix [N][K/32]. */
static int i8_emin_min(const uint8_t* s, int N, int K) {
  int mn = 255;
  for (size_t i = 0; i < (size_t)N * (K / 32); ++i)
    if (s[i] < mn) mn = s[i];
  return mn;
}

/* Full MXFP4 layer with INT8 activations for both GEMMs (the engine with
 * int8_activation ALIGN on, moe_v2_packed4_w4a8.inc:1341-1362): gate/up from
 * int8(x), act fp32 -> bf16, down from int8(bf16(act)).
 * Fallbacks to the fp32 path (bf16 activation times the dequantized weights):
 *  - the spread guard (wtmax <= 3, :1344-1366, a tile whose weight rows spread
 *    more than 3 e8m0 steps takes the fp32 path): a gate/up column pair i
 *    whose gate row i or up row i spreads more than 3, and a down column h
 *    whose row spreads more than 3 (the reference decides per CPU tile of
 *    output columns; this build decides per column);
 *  - the offset guard (cmin + emin - 128 >= -24, :436, :1361-1364): a pair
 *    whose activation row exponent crow plus the smallest e8m0 byte of the
 *    expert's matrix, minus 128, is below -24 takes the whole gate/up (or
 *    down) row on the fp32 path (the reference decides per block of its rows
 *    -- one row in its per-token loop, six in the grouped one -- and over its
 *    thread's column range; this build decides per row over the expert). */
int xo_moe_layer_i8(int T, int K, int E, int n_shared, int H, int I, const uint16_t* x,
                    const int32_t* ids, const float* wts, const uint8_t* w13,
                    const uint8_t* s13, const uint8_t* w2, const uint8_t* s2, float limit,
                    float alpha, float beta, float* out) {
  float* xf = (float*)malloc(sizeof(float) * (size_t)H);
  float* gu = (float*)malloc(sizeof(float) * (size_t)2 * I);
  int32_t* accb = (int32_t*)malloc(sizeof(int32_t) * (size_t)(2 * I > H ? 2 * I : H));
  float* actf = (float*)malloc(sizeof(float) * (size_t)I);
  float* y = (float*)malloc(sizeof(float) * (size_t)H);
  float* wrow = (float*)malloc(sizeof(float) * (size_t)(H > I ? H : I));
  int8_t* a8b = (int8_t*)malloc((size_t)(H > I ? H : I));
  if (!xf || !gu || !accb || !actf || !y || !wrow || !a8b) {
    free(xf); free(gu); free(accb); free(actf); free(y); free(wrow); free(a8b);
    return -1;
  }
  for (int t = 0; t < T; ++t) {
    float* o = out + (size_t)t * H;
    for (int h = 0; h < H; ++h) o[h] = 0.f;
    for (int k = 0; k < H; ++k) xf[k] = xo_bf16_to_f32(x[(size_t)t * H + k]);
    for (int r = 0; r < K + n_shared; ++r) {
      int e;
      float w;
      if (r < K) {
        e = ids[(size_t)t * K + r];
        w = wts[(size_t)t * K + r];
        if (e < 0 || e >= E || w == 0.f) continue;
      } else {
        e = E + (r - K);
        w = 1.0f;
      }
      const uint8_t* w13e = w13 + (size_t)e * 2 * I * (H / 2);
      const uint8_t* s13e = s13 + (size_t)e * 2 * I * (H / 32);
      const uint8_t* w2e = w2 + (size_t)e * H * (I / 2);
      const uint8_t* s2e = s2 + (size_t)e * H * (I / 32);
      xo_i8_gemm(xf, 1, w13e, s13e, 2 * I, H, 1.0f, accb, gu);
      const int g2_13 = xo_i8_quant_row(xf, H, a8b) + i8_emin_min(s13e, 2 * I, H) - 128 < -24;
      for (int i = 0; i < I; ++i) {
        if (g2_13 || xo_i8_row_spread(s13e + (size_t)i * (H / 32), H) > 3 ||
            xo_i8_row_spread(s13e + (size_t)(I + i) * (H / 32), H) > 3) {
          gu[i] = i8_fallback_dot(xf, w13e, s13e, 2 * I, H, i, wrow);
          gu[I + i] = i8_fallback_dot(xf, w13e, s13e, 2 * I, H, I + i, wrow);
        }
        actf[i] = bf16_round(xo_silu_gate(gu[i], gu[I + i], limit, alpha, beta));
      }
      xo_i8_gemm(actf, 1, w2e, s2e, H, I, 1.0f, accb, y);
      const int g2_2 = xo_i8_quant_row(actf, I, a8b) + i8_emin_min(s2e, H, I) - 128 < -24;
      for (int h = 0; h < H; ++h)
        if (g2_2 || xo_i8_row_spread(s2e + (size_t)h * (I / 32), I) > 3)
          y[h] = i8_fallback_dot(actf, w2e, s2e, H, I, h, wrow);
      for (int h = 0; h < H; ++h) o[h] += w * y[h];
    }
  }
  free(xf); free(gu); free(accb); free(actf); free(y); free(wrow); free(a8b);
  return 0;
}
