/*
 * xtu_moe_amd.h -- C ABI of the MI355X (gfx950) quantized MoE expert path.
 *
 * Plain pointers (device addresses as integers on the Python side), sizes and
 * a hipStream_t; every entry point returns a hipError_t (0 = success,
 * hipErrorInvalidValue = 1 for rejected arguments, otherwise the launch
 * status from hipPeekAtLastError; execution errors surface at the next
 * synchronisation).  The caller owns all buffers.  Entry points never
 * allocate and never synchronise, so they may be recorded into a HIP graph.
 *
 * Weight formats (fmt): 0 BF16, 1 FP8 e4m3 + 128x128 fp32 block scales,
 * 2 MXFP4 (e2m1 + e8m0 per 32 k), 3 NVFP4 (e2m1 + e4m3 per 16 k + fp32
 * second-level scales: gs13 [E][2] = gate, up -- the checkpoint's
 * w13_weight_scale_2 [E][2], hybrid_model.py:1546-1561 -- and gs2 [E],
 * indexed by weight slot).  Weights are in the P16 panel layout: per
 * expert, a [N][K] matrix is stored as
 * [N/16][K/SB][4][16][16 B] with SB = 128 (fp4), 64 (fp8), 32 (bf16) k per
 * super-block; fp4 scales in groups of UG super-blocks per 16-row panel,
 * [N/16][ceil((K/128)/UG)][64 lanes][16 B], lane 16q+r holding the scales of
 * row r, k-chunk q for UG consecutive super-blocks (MXFP4: UG = 16, 1 B
 * each; NVFP4: UG = 8, 2 B each; the last group zero-padded); fp8 block
 * scales as [N/128][K/128] fp32.
 * w13 rows [0, I) are the gate projection, [I, 2I) the up projection.
 *
 * Citations are to the reference (yeungtuzi/vllm-xtu-moe) interface each
 * entry point replaces.
 */
#ifndef XTU_MOE_AMD_H
#define XTU_MOE_AMD_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- library */
const char* xtu_version(void);
const char* xtu_error_string(int err);

/* ---------------------------------------------------------------- routing
 * Replaces the router the hook obtains from vLLM's router factory
 * (vllm_xiaotu_moe/mixed_experts.py:991-1078 _get_router/_select_topk;
 * hybrid_model.py:1877 fused_topk_bias).  A 256-thread team per token (four
 * per workgroup); ties broken toward the lower expert index.  logits [T][E] fp32; outputs [T][K].
 *   softmax:  w = exp(l - lmax) / sum over the K chosen (renormalize=1)
 *   grouped:  s = sigmoid(l), selection by s + bias, group score = sum of the
 *             two best in the group, topk_group groups kept, then
 *             w = s / sum(s of chosen) * routed_scaling (renormalize=1). */
hipError_t xtu_route_softmax_topk(const float* logits, int T, int E, int K, int renormalize,
                                  int32_t* topk_ids, float* topk_weights, hipStream_t stream);
hipError_t xtu_route_grouped_sigmoid(const float* logits, const float* bias, int T, int E,
                                     int n_group, int topk_group, int K, float routed_scaling,
                                     int renormalize, int32_t* topk_ids, float* topk_weights,
                                     hipStream_t stream);

/* ----------------------------------------------------------- segmentation
 * Replaces _build_segmentation / _build_segmentation_reuse
 * (vllm_xiaotu_moe/gpu_prefill.py:800-887) and moe4_smallm._segmentation
 * (vllm_xiaotu_moe/moe4_smallm.py:97-129).  Flat pairs a = t*K + k, then the
 * shared-expert pairs a = T*K + t*n_shared + s (bucket E + s, weight 1).
 * Invalid ids (< 0 or >= E) -- and zero weights when drop_zero -- go to the
 * trash bucket E + n_shared.  Stable order by bucket.  id_map (nullable,
 * int32 [E]) translates ids before bucketing (pool slots / ring order).
 * Outputs (device): sorted_pair/sorted_tok/sorted_wts/inv [A];
 * seg_start [NB+1] (NB = E + n_shared + 1); active [NB] + n_active[1] (the
 * non-empty non-trash buckets, ascending); tile_expert/tile_row0
 * [xtu_segment_max_tiles] + n_tiles[1] (bm-row tiles per bucket);
 * expert_tile_start [NB+1] (first tile of each bucket).
 * workspace: xtu_segment_workspace_bytes(T, K, E, n_shared) bytes. */
size_t xtu_segment_workspace_bytes(int T, int K, int E, int n_shared);
int xtu_segment_max_tiles(int T, int K, int E, int n_shared, int bm);
hipError_t xtu_segment(const int32_t* topk_ids, const float* topk_weights, const int32_t* id_map,
                       int T, int K, int E, int n_shared, int drop_zero, int bm, void* workspace,
                       int32_t* sorted_pair, int32_t* sorted_tok, float* sorted_wts, int32_t* inv,
                       int32_t* seg_start, int32_t* active, int32_t* n_active,
                       int32_t* tile_expert, int32_t* tile_row0, int32_t* n_tiles,
                       int32_t* expert_tile_start, hipStream_t stream);

/* xtu_segment without the workspace argument: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc): the
 * workspace is a static device array of 4 MiB per GPU, held until the process
 * ends, so the call allocates nothing.  Outputs and their meaning are
 * xtu_segment's.  Shapes whose xtu_segment_workspace_bytes() exceeds 4 MiB
 * (1M per-block bucket counts, e.g. up to 16.6M pairs at 258 buckets, 2M at
 * 2048) are rejected with hipErrorInvalidValue and a message on stderr.  The
 * array is shared by every call on a GPU and holds the last call's counts
 * (each call rewrites every word it reads, so nothing needs clearing): calls
 * that overlap on one GPU (different streams) race -- serialise them.  The
 * stream must belong to the current device. */
hipError_t xtu_segment_noalloc(const int32_t* topk_ids, const float* topk_weights,
                               const int32_t* id_map, int T, int K, int E, int n_shared,
                               int drop_zero, int bm, int32_t* sorted_pair, int32_t* sorted_tok,
                               float* sorted_wts, int32_t* inv, int32_t* seg_start,
                               int32_t* active, int32_t* n_active, int32_t* tile_expert,
                               int32_t* tile_row0, int32_t* n_tiles, int32_t* expert_tile_start,
                               hipStream_t stream);

/* Small batches (A = T*K + T*n_shared <= xtu_route_segment_small_max_pairs()):
 * routing and the whole segmentation in one launch, same outputs as
 * xtu_route_* followed by xtu_segment.  mode 0 = softmax routing, 1 = grouped
 * sigmoid routing (topk_ids/topk_weights are written; up to 16 waves route
 * one token each at a time), 2 = ids/weights given (read).  One workgroup.  Replaces, for decode, the router call plus _build_segmentation
 * (gpu_prefill.py:849-887) and the in-kernel dispatch scan of
 * moe4_smallm_gu2/dn2 (moe4_smallm.cu:193-206, :266-281). */
int xtu_route_segment_small_max_pairs(void);
hipError_t xtu_route_segment_small(int mode, const float* logits, const float* bias,
                                   int32_t* topk_ids, float* topk_weights, int T, int E, int K,
                                   int n_group, int topk_group, float routed_scaling,
                                   int renormalize, const int32_t* id_map, int n_shared,
                                   int drop_zero, int bm, int32_t* sorted_pair,
                                   int32_t* sorted_tok, float* sorted_wts, int32_t* inv,
                                   int32_t* seg_start, int32_t* active, int32_t* n_active,
                                   int32_t* tile_expert, int32_t* tile_row0, int32_t* n_tiles,
                                   int32_t* expert_tile_start, hipStream_t stream);

/* --------------------------------------------------- skinny-M (decode) path
 * Replaces moe4_smallm_gu2 / moe4_smallm_dn2 (xiaotu_moe/csrc/moe4_smallm.cu:
 * 395-430) and the FP8 pair kernels _gate_up_pairs_kernel / _act_pairs_kernel
 * / _down_pairs_kernel (vllm_xiaotu_moe/decode_moe_fp8.py:23-101).  Batches
 * of T <= 16 tokens.  Work slots are either the active experts (tile_row0 =
 * NULL: slot j is expert active[j], rows from seg_start, at most 16 of them
 * computed) or the segmentation's 16-row tiles (xtu_segment with bm = 16:
 * active = tile_expert, tile_row0, n_active = n_tiles), which cover every
 * row of every bucket -- an expert listed twice by a token, or zero-weight
 * pairs kept with drop_zero = 0, may hold more than 16 rows.  One workgroup
 * per (work slot, weight panel group); slots beyond *n_active exit at once;
 * max_active bounds the grid.
 * gate_up writes act bf16 [A][I] = SwiGLU-clamp(x W_gate^T, x W_up^T) per
 * sorted pair row; down writes y fp32 [A][H].  T = tokens of the batch (up
 * to 72 KiB of an expert's activation rows are staged in LDS, the rest read
 * from global memory).
 * w/s_estride: bytes between experts (0 = dense); slot_map (nullable):
 * expert -> weight slot. */
hipError_t xtu_decode_gate_up(int fmt, const void* x, int T, int H, int I, const void* w13,
                              const void* s13, const float* gs13, long w_estride, long s_estride,
                              const int32_t* slot_map, const int32_t* sorted_tok,
                              const int32_t* seg_start, const int32_t* active,
                              const int32_t* tile_row0, const int32_t* n_active, int max_active,
                              void* act, float limit, float alpha, float beta,
                              hipStream_t stream);
hipError_t xtu_decode_down(int fmt, const void* act, int T, int H, int I, const void* w2, const void* s2,
                           const float* gs2, long w_estride, long s_estride,
                           const int32_t* slot_map, const int32_t* seg_start,
                           const int32_t* active, const int32_t* tile_row0,
                           const int32_t* n_active, int max_active, float* y,
                           hipStream_t stream);
/* xtu_decode_down with y row sorted_pair[position] (the flat pair index:
 * t*K + k, shared T*K + t*n_shared + s) instead of the sorted position, for
 * xtu_combine_by_pair.  Same replaced code as xtu_decode_down
 * (moe4_smallm.cu:395-430).  y holds T*(K + n_shared) rows; rows of pairs in
 * the trash bucket are not written. */
hipError_t xtu_decode_down_by_pair(int fmt, const void* act, int T, int H, int I, const void* w2,
                                   const void* s2, const float* gs2, long w_estride,
                                   long s_estride, const int32_t* slot_map,
                                   const int32_t* seg_start, const int32_t* active,
                                   const int32_t* tile_row0, const int32_t* n_active,
                                   int max_active, const int32_t* sorted_pair, float* y,
                                   hipStream_t stream);

/* Routing + segmentation and the shared experts' gate/up in one launch
 * (tiny batches, n_shared >= 1): workgroup 0 does exactly what
 * xtu_route_segment_small does (same outputs, same order; mode 0 softmax /
 * 1 grouped sigmoid from fp32 logits, 2 ids given), workgroups 1.. run the
 * shared experts' gate/up for all T tokens -- they need no routing -- and
 * write act_shared bf16 [n_shared][T][I] in token order.  The argument list
 * is xtu_route_segment_small's followed by the gate/up weights.  Then
 * xtu_decode_gate_up_routed runs the routed experts (the last n_shared
 * active slots, the shared buckets, left out) and xtu_decode_down_combine
 * takes the shared rows from act_shared.  Replaces, for decode, the router
 * call plus _build_segmentation (gpu_prefill.py:849-887) and the shared
 * expert's share of moe4_smallm_gu2 (moe4_smallm.cu:395-413).
 * xtu_decode_route_shared_ok: the shape fits (the tiny router's envelope,
 * one wave per token in the gate/up workgroup, the gate/up fast path: every
 * token row staged in LDS, one round per wave); logits / bias rows must
 * also be 16-byte aligned (hipErrorInvalidValue otherwise). */
int xtu_decode_route_shared_ok(int fmt, int mode, int T, int E, int K, int n_group,
                               int n_shared, int H, int I);
hipError_t xtu_decode_route_shared(
    int mode, const float* logits, const float* bias, int32_t* topk_ids, float* topk_weights,
    int T, int E, int K, int n_group, int topk_group, float routed_scaling, int renormalize,
    const int32_t* id_map, int n_shared, int drop_zero, int bm, int32_t* sorted_pair,
    int32_t* sorted_tok, float* sorted_wts, int32_t* inv, int32_t* seg_start, int32_t* active,
    int32_t* n_active, int32_t* tile_expert, int32_t* tile_row0, int32_t* n_tiles,
    int32_t* expert_tile_start, int fmt, const void* x, int H, int I, const void* w13,
    const void* s13, const float* gs13, long w_estride, long s_estride, const int32_t* slot_map,
    void* act_shared, float limit, float alpha, float beta, hipStream_t stream);
/* xtu_decode_gate_up for the routed experts only: the last n_shared work
 * slots (the shared buckets, one 16-row tile each) are left out; the gate/up
 * fast-path shape is required. */
hipError_t xtu_decode_gate_up_routed(int fmt, const void* x, int T, int H, int I,
                                     const void* w13, const void* s13, const float* gs13,
                                     long w_estride, long s_estride, const int32_t* slot_map,
                                     const int32_t* sorted_tok, const int32_t* seg_start,
                                     const int32_t* active, const int32_t* tile_row0,
                                     const int32_t* n_active, int max_active, int n_shared,
                                     void* act, float limit, float alpha, float beta,
                                     hipStream_t stream);

/* Routing, segmentation and every gate/up of a tiny decode batch in one
 * launch (the routing launch and the gate/up launch above folded together).
 * The routing arguments are xtu_decode_route_shared's and its outputs the
 * same (topk_ids / topk_weights and the segmentation with tiles of bm <= 16
 * rows, for the down pass); act bf16 [A][I] gets the routed experts' SwiGLU
 * rows in sorted order.  act_shared non-null (n_shared >= 1): the shared
 * experts' rows go there ([n_shared][T][I], token order) from workgroups
 * that need no routing, and the down pass is xtu_decode_down_combine with
 * act_shared; act_shared null: the shared experts' rows are ordinary sorted
 * rows of act.  Every routed workgroup routes the batch in LDS for itself
 * (the same code on the same inputs, so all agree) instead of reading the
 * routing back from memory.  max_tiles: work items per gate panel, at least
 * b + (A - b) / bm for A = T (K + n_shared) pairs in b <= min(E, T K) +
 * n_shared buckets, at most 64.  Replaces, for decode, the router call,
 * _build_segmentation (gpu_prefill.py:849-887) and moe4_smallm_gu2
 * (moe4_smallm.cu:395-413).
 * xtu_decode_route_gate_up_ok: the shape fits (the tiny router's envelope
 * and the gate/up fast path, as xtu_decode_route_shared_ok, but a routing
 * wave may take several tokens and n_shared may be 0). */
int xtu_decode_route_gate_up_ok(int fmt, int mode, int T, int E, int K, int n_group,
                                int n_shared, int H, int I);
hipError_t xtu_decode_route_gate_up(
    int mode, const float* logits, const float* bias, int32_t* topk_ids, float* topk_weights,
    int T, int E, int K, int n_group, int topk_group, float routed_scaling, int renormalize,
    const int32_t* id_map, int n_shared, int drop_zero, int bm, int32_t* sorted_pair,
    int32_t* sorted_tok, float* sorted_wts, int32_t* inv, int32_t* seg_start, int32_t* active,
    int32_t* n_active, int32_t* tile_expert, int32_t* tile_row0, int32_t* n_tiles,
    int32_t* expert_tile_start, int fmt, const void* x, int H, int I, const void* w13,
    const void* s13, const float* gs13, long w_estride, long s_estride, const int32_t* slot_map,
    int max_tiles, void* act, void* act_shared, float limit, float alpha, float beta,
    hipStream_t stream);

/* A whole decode layer in one launch: xtu_decode_route_gate_up's routing,
 * segmentation and gate/up (same arguments, same outputs), then, after a
 * barrier across the launch's workgroups, xtu_decode_down_combine's down
 * projection with the weighted combine (w2 / s2 / gs2 as there, W2 strides
 * w2_estride / s2_estride, out bf16 or fp32 [T][H] written whole, the same
 * per-token summation order).  The launch is one resident round of
 * workgroups (sized by the occupancy query) so the barrier completes;
 * barrier: xtu_decode_layer_barrier_words() words of device memory, zero
 * before the first call; every call leaves its counters zero (the last
 * 64-word line's first word becomes 1 if a wait ever ran out, about 0.1 s,
 * instead of hanging).  Calls that overlap on one device must not share
 * the barrier words.  Replaces, for decode, the router call,
 * _build_segmentation (gpu_prefill.py:849-887), moe4_smallm_gu2 and
 * moe4_smallm_dn2 (moe4_smallm.cu:260-333, 395-430) -- one launch instead
 * of four.  xtu_decode_layer_ok: xtu_decode_route_gate_up_ok and the down's
 * shape (I / 128 = 2 x the K split of the gate/up workgroup's waves over
 * one or more panels, the act rows within 96 KiB of LDS). */
int xtu_decode_layer_barrier_words(void);
int xtu_decode_layer_ok(int fmt, int mode, int T, int E, int K, int n_group, int n_shared,
                        int H, int I);
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
    hipStream_t stream);

/* Down projection with the weighted combine fused: out[t] = sum over t's live
 * pairs (t, e) of w * (act_row W2_e^T), bf16 (out_bf16 = 1) or fp32 [T][H],
 * every row written.  Replaces moe4_smallm_dn2 (moe4_smallm.cu:260-333,
 * 416-430), which scatters the same sums with atomics; here each token's sum
 * runs over its experts in active-slot order (deterministic).  sorted_wts:
 * the segmentation's per-row weights (1 for shared rows); trash = E + NS.
 * act_shared (nullable): the shared experts' rows [n_shared][T][I] written
 * by xtu_decode_route_shared, used for buckets trash - n_shared .. trash - 1
 * instead of their rows in act.  xtu_decode_down_combine_ok reports whether
 * a batch fits (T <= 16, I a multiple of 128 with I/128 splitting into waves
 * of 1, 2 or 4 units, the A = T*(K+NS) act rows plus shared_rows =
 * n_shared*T (when act_shared is given) within the LDS stage); the entry
 * returns hipErrorInvalidValue otherwise. */
int xtu_decode_down_combine_ok(int fmt, int T, int A, int H, int I, int trash, int max_active,
                               int shared_rows);
hipError_t xtu_decode_down_combine(int fmt, const void* act, const void* act_shared, int n_shared,
                                   int T, int A, int H, int I,
                                   const void* w2, const void* s2, const float* gs2,
                                   long w_estride, long s_estride, const int32_t* slot_map,
                                   const int32_t* sorted_tok, const float* sorted_wts,
                                   const int32_t* seg_start, int trash, const int32_t* active,
                                   const int32_t* n_active, int max_active, void* out,
                                   int out_bf16, hipStream_t stream);

/* ------------------------------------------------ grouped GEMM (prefill) path
 * Replaces _gate_up_kernel / _down_kernel (vllm_xiaotu_moe/gpu_prefill.py:
 * 232-390) and gate_up_kernel_fp8 / down_kernel_fp8
 * (vllm_xiaotu_moe/gpu_prefill_fp8.py:101-205) plus the bmm FP8 path
 * (gpu_prefill_fp8.py:1172).  M tiles of xtu_gemm_tile_m(fmt) rows from the
 * segmentation tile list, range [*tile_lo, *tile_hi) (device pointers, e.g.
 * expert_tile_start + e0 / + e1); max_tiles bounds the grid.
 * Requires H % 256 == 0, I % 128 == 0. */
int xtu_gemm_tile_m(int fmt);
hipError_t xtu_gemm_gate_up(int fmt, const void* x, const int32_t* sorted_tok, int H, int I,
                            const void* w13, const void* s13, const float* gs13, long w_estride,
                            long s_estride, const int32_t* slot_map, const int32_t* seg_start,
                            const int32_t* tile_expert, const int32_t* tile_row0,
                            const int32_t* tile_lo, const int32_t* tile_hi, int max_tiles,
                            void* act, float limit, float alpha, float beta, hipStream_t stream);
hipError_t xtu_gemm_down(int fmt, const void* act, int H, int I, const void* w2, const void* s2,
                         const float* gs2, long w_estride, long s_estride,
                         const int32_t* slot_map, const int32_t* seg_start,
                         const int32_t* tile_expert, const int32_t* tile_row0,
                         const int32_t* tile_lo, const int32_t* tile_hi, int max_tiles, float* y,
                         hipStream_t stream);

/* Weighted unpermute.  Replaces the atomic_add epilogue of _down_kernel
 * (gpu_prefill.py:380-385) and the per-token ordered sum of MOE_V2::forward_many
 * (xiaotu_moe/csrc/moe/moe_v2.hpp:920-930): out[t] = sum_k w[t,k] * y[inv[t*K+k]]
 * in k order over pairs whose sorted position is below *trash_start (the
 * segmentation's seg_start[E + n_shared]) and whose weight is non-zero, plus
 * the shared rows.  out is bf16 (out_bf16 = 1) or fp32 [T][H]. */
hipError_t xtu_combine(const float* y, const int32_t* inv, const float* topk_weights,
                       const int32_t* trash_start, int T, int K, int n_shared, int H, void* out,
                       int out_bf16, hipStream_t stream);
/* xtu_combine over y rows in flat pair order (as xtu_decode_down_by_pair
 * writes them): the same sum, skip rule and order, the row addresses taken
 * from the pair index instead of inv (inv still decides the skip).  K in
 * {1, 2, 4, 6, 8, 10}, n_shared <= 2; other shapes are rejected. */
hipError_t xtu_combine_by_pair(const float* y, const int32_t* inv, const float* topk_weights,
                               const int32_t* trash_start, int T, int K, int n_shared, int H,
                               void* out, int out_bf16, hipStream_t stream);

/* ------------------------------------------------- exact FP8 prefill GEMMs
 * FP8-weight grouped GEMMs on the scaled fp8 MFMA (16x16x128 e4m3 x e4m3),
 * the dequantised-fp32 product up to fp32 summation order.  Replace the
 * reference's Triton FP8 prefill kernels (gpu_prefill_fp8.py:101-205,
 * gate_up_kernel_fp8 / down_kernel_fp8), which round e4m3 * block scale to a
 * bf16 operand.  Activation rows are first split by xtu_fp8pair_quant into
 * e4m3 pairs (hi, lo) with per-32-k e8m0 scales (shi, slo) such that
 * x = hi * 2^(shi-127) + lo * 2^(slo-127) exactly (bf16 x); planes hi, lo
 * [M][K] bytes, shi, slo [M][K/32] bytes.  The GEMMs take the pairs of x
 * (gate/up, rows gathered through sorted_tok) or of act (down), the e4m3
 * P16 weights and their [N/128][K/128] fp32 block scales, and M tiles of
 * xtu_gemm8_tile_m() rows from xtu_segment(bm = that) (and its
 * expert_tile_start, which orders the work items); outputs as
 * xtu_gemm_gate_up / xtu_gemm_down. */
int xtu_gemm8_tile_m(void);
hipError_t xtu_fp8pair_quant(const void* x, int M, int K, uint8_t* hi, uint8_t* lo, uint8_t* shi,
                             uint8_t* slo, hipStream_t stream);
hipError_t xtu_gemm8_gate_up(const uint8_t* hi, const uint8_t* lo, const uint8_t* shi,
                             const uint8_t* slo, const int32_t* sorted_tok, int H, int I,
                             const void* w13, const float* s13, long w_estride, long s_estride,
                             const int32_t* slot_map, const int32_t* seg_start,
                             const int32_t* tile_expert, const int32_t* tile_row0,
                             const int32_t* expert_tile_start, const int32_t* tile_lo,
                             const int32_t* tile_hi, int max_tiles, void* act, float limit,
                             float alpha, float beta, hipStream_t stream);
hipError_t xtu_gemm8_down(const uint8_t* hi, const uint8_t* lo, const uint8_t* shi,
                          const uint8_t* slo, int H, int I, const void* w2, const float* s2,
                          long w_estride, long s_estride, const int32_t* slot_map,
                          const int32_t* seg_start, const int32_t* tile_expert,
                          const int32_t* tile_row0, const int32_t* expert_tile_start,
                          const int32_t* tile_lo, const int32_t* tile_hi, int max_tiles,
                          float* y, hipStream_t stream);


/* The same exact-pair GEMMs with the weight format as an argument: fmt 1
 * (FP8, s = fp32 [N/128][K/128] block scales) or 2 (MXFP4, s = the packed
 * e8m0 scale groups).  MXFP4 codes enter v_mfma_scale_f32_16x16x128_f8f6f4
 * as fp4 B operands straight from P16 (lane 16q + r: k = 32q..32q+31 of row
 * r) with their e8m0 byte as the B scale, so the product is exact with no
 * dequantisation.  M tiles of xtu_gemm8_tile_m() rows.  Replace
 * _gate_up_kernel / _down_kernel (vllm_xiaotu_moe/gpu_prefill.py:232-390)
 * for MXFP4 prefill; xtu_mx_pair_* below is the faster form where it fits. */
hipError_t xtu_gemm_pair_gate_up(int fmt, const uint8_t* hi, const uint8_t* lo,
                                 const uint8_t* shi, const uint8_t* slo,
                                 const int32_t* sorted_tok, int H, int I, const void* w13,
                                 const void* s13, long w_estride, long s_estride,
                                 const int32_t* slot_map, const int32_t* seg_start,
                                 const int32_t* tile_expert, const int32_t* tile_row0,
                                 const int32_t* expert_tile_start, const int32_t* tile_lo,
                                 const int32_t* tile_hi, int max_tiles, void* act, float limit,
                                 float alpha, float beta, hipStream_t stream);
hipError_t xtu_gemm_pair_down(int fmt, const uint8_t* hi, const uint8_t* lo, const uint8_t* shi,
                              const uint8_t* slo, int H, int I, const void* w2, const void* s2,
                              long w_estride, long s_estride, const int32_t* slot_map,
                              const int32_t* seg_start, const int32_t* tile_expert,
                              const int32_t* tile_row0, const int32_t* expert_tile_start,
                              const int32_t* tile_lo, const int32_t* tile_hi, int max_tiles,
                              float* y, hipStream_t stream);

/* --------------------------------------- MXFP4 exact-pair GEMMs (32x32x64)
 * The MXFP4 prefill GEMMs of the reference (vllm_xiaotu_moe/gpu_prefill.py:
 * 232-390, _gate_up_kernel / _down_kernel) on v_mfma_scale_f32_32x32x64_
 * f8f6f4 with operand layouts made for it:
 *   xtu_pair_quant_il: bf16 rows [M][K] -> interleaved e4m3 pairs hilo
 *     [M][2K] (per 64 k: 64 bytes hi, 64 bytes lo) and e8m0 shi [M][K/32];
 *     x = hi * 2^(shi-127) + lo * 2^(max(shi-4,0)-127) exactly (bf16 x).
 *   xtu_mx_pair_scales: packed MXFP4 scale groups (E slots of s_estride
 *     bytes, N rows, K) -> step-major [E][K/64][N/16][16][2] bytes.
 *   xtu_mx_pair_gate_up / _down: as xtu_gemm_pair_* for fmt 2, with hilo,
 *     shi and the step-major scales (s_estride 0: N * K / 32), M tiles of
 *     xtu_mx_pair_tile_m() rows; shapes where xtu_mx_pair_fits(H, I). */
int xtu_mx_pair_fits(int H, int I);
int xtu_mx_pair_tile_m(void);
hipError_t xtu_pair_quant_il(const void* x, int M, int K, uint8_t* hilo, uint8_t* shi,
                             hipStream_t stream);
hipError_t xtu_mx_pair_scales(const uint8_t* s, int E, int N, int K, long s_estride, uint8_t* out,
                              hipStream_t stream);
hipError_t xtu_mx_pair_gate_up(const uint8_t* hilo, const uint8_t* shi, const int32_t* sorted_tok,
                               int H, int I, const void* w13, const uint8_t* s13p,
                               long w_estride, long s_estride, const int32_t* slot_map,
                               const int32_t* seg_start, const int32_t* tile_expert,
                               const int32_t* tile_row0, const int32_t* expert_tile_start,
                               const int32_t* tile_lo, const int32_t* tile_hi, int max_tiles,
                               void* act, float limit, float alpha, float beta,
                               hipStream_t stream);
hipError_t xtu_mx_pair_down(const uint8_t* hilo, const uint8_t* shi, int H, int I, const void* w2,
                            const uint8_t* s2p, long w_estride, long s_estride,
                            const int32_t* slot_map, const int32_t* seg_start,
                            const int32_t* tile_expert, const int32_t* tile_row0,
                            const int32_t* expert_tile_start, const int32_t* tile_lo,
                            const int32_t* tile_hi, int max_tiles, float* y, hipStream_t stream);

/* The same MXFP4 GEMMs on the double-rate fp6 / fp4 MFMA (fp6 or fp4 A
 * operand against fp4 B runs at twice the fp8 x fp4 rate on 32x32x64):
 *   xtu_tri_quant_il: bf16 rows [M][K] -> activation triples q [M][2K]
 *     (per 64 k and 32-k half h: 64 bytes at 64h, [p1 24 B | p2 24 B |
 *     p3 16 B], p1 p2 e2m3 codes packed 6 bits each, p3 e2m1 codes 4 bits
 *     each, k order) and e8m0 sq [M][K/32] = e + 127;
 *     x ~= 2^e (p1 + p2/16 + p3/256), each piece the round-to-nearest-even
 *     of the remainder of the previous ones, e the smallest exponent with
 *     max|x| <= 7.5 * 2^e; |error| <= 2^(e-9) < 2^-10.9 * max|x| of the
 *     32-k block (pieces whose scale byte would be negative are zero).
 *   xtu_mx_tri_gate_up / _down: as xtu_mx_pair_gate_up / _down (same
 *     arguments, tiles, shapes), on q and sq: three MFMAs per block and
 *     step (scales sq, sq-4, sq-8) instead of the pair's two.
 * No counterpart in the reference: its Triton kernels run these GEMMs on
 * bf16 operands; the triples are this library's operand format. */
hipError_t xtu_tri_quant_il(const void* x, int M, int K, uint8_t* q, uint8_t* sq,
                            hipStream_t stream);
hipError_t xtu_mx_tri_gate_up(const uint8_t* q, const uint8_t* sq, const int32_t* sorted_tok,
                              int H, int I, const void* w13, const uint8_t* s13p, long w_estride,
                              long s_estride, const int32_t* slot_map, const int32_t* seg_start,
                              const int32_t* tile_expert, const int32_t* tile_row0,
                              const int32_t* expert_tile_start, const int32_t* tile_lo,
                              const int32_t* tile_hi, int max_tiles, void* act, float limit,
                              float alpha, float beta, hipStream_t stream);
hipError_t xtu_mx_tri_down(const uint8_t* q, const uint8_t* sq, int H, int I, const void* w2,
                           const uint8_t* s2p, long w_estride, long s_estride,
                           const int32_t* slot_map, const int32_t* seg_start,
                           const int32_t* tile_expert, const int32_t* tile_row0,
                           const int32_t* expert_tile_start, const int32_t* tile_lo,
                           const int32_t* tile_hi, int max_tiles, float* y, hipStream_t stream);
/* xtu_mx_{pair,tri,duo}_gate_up with the activation written straight in the
 * down pass's operand layout (mode 0 pairs as xtu_pair_quant_il writes
 * them, 1 and 2 triples as xtu_tri_quant_il does): act_q [A][2I] and its
 * e8m0 bytes act_sq [A][I/32], the bytes the separate quantiser would make
 * of the bf16 rows, which are never written.  Replaces the gate/up kernel's
 * bf16 inter rows plus the down kernel's in-loop activation handling
 * (gpu_prefill.py:311-390). */
hipError_t xtu_mx_gate_up_q(int mode, const uint8_t* q, const uint8_t* sq,
                            const int32_t* sorted_tok, int H, int I, const void* w13,
                            const uint8_t* s13p, long w_estride, long s_estride,
                            const int32_t* slot_map, const int32_t* seg_start,
                            const int32_t* tile_expert, const int32_t* tile_row0,
                            const int32_t* expert_tile_start, const int32_t* tile_lo,
                            const int32_t* tile_hi, int max_tiles, uint8_t* act_q,
                            uint8_t* act_sq, float limit, float alpha, float beta,
                            hipStream_t stream);
/*   xtu_mx_duo_gate_up / _down: the same on the first two pieces of the
 *     triples only (x ~= 2^e (p1 + p2/16), |error| <= 2^(e-6) of the 32-k
 *     block, rms ~7.5e-4 of the values for N(0,1) rows): two double-rate
 *     MFMAs per block and step.  No counterpart in the reference either. */
hipError_t xtu_mx_duo_gate_up(const uint8_t* q, const uint8_t* sq, const int32_t* sorted_tok,
                              int H, int I, const void* w13, const uint8_t* s13p, long w_estride,
                              long s_estride, const int32_t* slot_map, const int32_t* seg_start,
                              const int32_t* tile_expert, const int32_t* tile_row0,
                              const int32_t* expert_tile_start, const int32_t* tile_lo,
                              const int32_t* tile_hi, int max_tiles, void* act, float limit,
                              float alpha, float beta, hipStream_t stream);
hipError_t xtu_mx_duo_down(const uint8_t* q, const uint8_t* sq, int H, int I, const void* w2,
                           const uint8_t* s2p, long w_estride, long s_estride,
                           const int32_t* slot_map, const int32_t* seg_start,
                           const int32_t* tile_expert, const int32_t* tile_row0,
                           const int32_t* expert_tile_start, const int32_t* tile_lo,
                           const int32_t* tile_hi, int max_tiles, float* y, hipStream_t stream);

/* -------------------------------------- INT8-activation x FP4-code (ALIGN) path
 * Replaces the engine's ALIGN integer path (xiaotu_moe/csrc/moe/
 * moe_v2_packed4_w4a8.inc:478-586 xiaotu_predecode_block, :661-715
 * xiaotu_quant_row_align_into, :811-858 xiaotu_i8_align_tile).
 * xtu_i8_prepare expands MXFP4 weights (P16) of E experts into shifted int8
 * w8' (P16 with 16 int8 per chunk, N*K bytes per expert) and emin [E][N];
 * *dmax (zero on entry) receives the largest shift.  A row whose shift
 * exceeds 3 is marked (emin 0xFF, int8 weights 0): the integer GEMMs leave
 * its output column unwritten (gate/up: act column n when gate row n or up
 * row n is marked) and xtu_i8_fallback computes it in fp32 -- the reference
 * sends such tiles to its fp32 path (moe_v2_packed4_w4a8.inc:1344-1366).
 * xtu_i8_quant_rows: per-row power-of-two int8 quantisation of bf16 rows.
 * The GEMMs accumulate in int32 (optionally stored to acc_out [A][N]) and
 * apply 2^(emin-128+crow) in fp32; epilogues as the bf16 GEMMs. */
size_t xtu_i8_weight_bytes(int N, int K);
hipError_t xtu_i8_prepare(const void* w, const void* s, int E, int N, int K, void* w8, void* emin,
                          int32_t* dmax, hipStream_t stream);
hipError_t xtu_i8_quant_rows(const void* rows_bf16, int M, int K, int8_t* a8, int32_t* crow,
                             hipStream_t stream);
hipError_t xtu_i8_gemm_gate_up(const int8_t* a8, const int32_t* crow, const int32_t* sorted_tok,
                               int H, int I, const void* w8, const void* emin,
                               const int32_t* slot_map, const int32_t* seg_start,
                               const int32_t* tile_expert, const int32_t* tile_row0,
                               const int32_t* tile_lo, const int32_t* tile_hi, int max_tiles,
                               void* act, int32_t* acc_out, float limit, float alpha, float beta,
                               hipStream_t stream);
hipError_t xtu_i8_gemm_down(const int8_t* a8, const int32_t* crow, int H, int I, const void* w8,
                            const void* emin, const int32_t* slot_map, const int32_t* seg_start,
                            const int32_t* tile_expert, const int32_t* tile_row0,
                            const int32_t* tile_lo, const int32_t* tile_hi, int max_tiles,
                            float* y, int32_t* acc_out, hipStream_t stream);
/* fp32 path for the marked columns: gate_up = 1 writes act[m][n] =
 * bf16(SwiGLU(x.w_gate_n, x.w_up_n)) for the column pairs n listed per weight
 * slot (CSR col_start [slots + 1] / cols), x rows gathered through
 * sorted_tok; gate_up = 0 writes y[m][h] = act_m . w2_h for the listed rows
 * h.  Operands: bf16 activations (x / act) and the MXFP4 weights (P16 codes
 * and packed e8m0 scales) dequantised exactly; fp32 sums.  Tiles of bm <= 128
 * rows from the same tile list as the integer GEMMs. */
hipError_t xtu_i8_fallback(int gate_up, const void* x, const int32_t* sorted_tok, int H, int I,
                           const void* w, const void* s, const int32_t* slot_map,
                           const int32_t* seg_start, const int32_t* tile_expert,
                           const int32_t* tile_row0, const int32_t* tile_lo,
                           const int32_t* tile_hi, int max_tiles, int bm,
                           const int32_t* col_start, const int32_t* cols, void* out, float limit,
                           float alpha, float beta, hipStream_t stream);
/* The engine's offset guard (moe_v2_packed4_w4a8.inc:436, :1361-1364: a tile
 * with cmin + emin - 128 < -24 takes the fp32 path), restated per sorted row:
 * xtu_i8_emin_min writes eminmin[e] = the smallest e8m0 byte of expert e's
 * [N][K] MXFP4 matrix; xtu_i8_row_fallback then recomputes in fp32 every
 * output column of each row whose activation exponent (crow of its token for
 * gate_up = 1, of its act row for gate_up = 0) plus eminmin of its weight
 * slot, minus 128, is below -24, overwriting what the integer GEMM wrote
 * (same operands and sums as xtu_i8_fallback).  Run after the integer GEMM
 * and xtu_i8_fallback, on the same stream. */
hipError_t xtu_i8_emin_min(const void* s, int E, int N, int K, int32_t* eminmin,
                           hipStream_t stream);
hipError_t xtu_i8_row_fallback(int gate_up, const void* x, const int32_t* sorted_tok,
                               const int32_t* crow, const int32_t* eminmin, int H, int I,
                               const void* w, const void* s, const int32_t* slot_map,
                               const int32_t* seg_start, const int32_t* tile_expert,
                               const int32_t* tile_row0, const int32_t* tile_lo,
                               const int32_t* tile_hi, int max_tiles, int bm, void* out,
                               float limit, float alpha, float beta, hipStream_t stream);

/* ------------------------------------------------ expert staging (ring / pool)
 * dst[i*dst_stride, +bytes) <- src[experts[i]*src_stride, +bytes), i < n, as
 * one hipMemcpyAsync per expert on `stream` (experts: host array; src/dst:
 * pinned host or device memory).  Replaces the engine's per-expert shard DMA
 * the ring and the resident pool consume (copy_hostbuf_to_device /
 * copy_hostbuf_to_device_2d, xiaotu_moe/csrc/binding.cpp:1368-1437;
 * _dma_hostbuf_range, vllm_xiaotu_moe/gpu_prefill.py:1897). */
hipError_t xtu_copy_experts(int n, const int32_t* experts, const void* src, long src_stride,
                            void* dst, long dst_stride, long bytes, hipStream_t stream);
/* Pitched copy: height rows of width bytes, src rows spitch apart, dst rows
 * dpitch apart (hipMemcpy2DAsync, any direction).  Replaces the engine's
 * copy_hostbuf_to_device_2d (xiaotu_moe/csrc/python_binding/binding.cpp:
 * 1404-1435), which DMAs a NUMA node's shard rows straight into their strided
 * place in a device slot. */
hipError_t xtu_copy_2d(void* dst, size_t dpitch, const void* src, size_t spitch, size_t width,
                       size_t height, hipStream_t stream);

/* FP8 prefill on v_mfma_scale_f32_32x32x64_f8f6f4, both operands staged in
 * LDS by direct loads (replaces gate_up_kernel_fp8 / down_kernel_fp8,
 * vllm_xiaotu_moe/gpu_prefill_fp8.py:101-205).  Activation pairs
 * interleaved (xtu_pair_quant_il); weights FP8 P16 with fp32 block scales
 * [N/128][K/128] per expert, every one finite and positive with max/min at
 * most 2^32 (the caller checks; the block scale is applied by rescaling the
 * accumulators by s(kb-1)/s(kb) at each 128-k block and by the last scale
 * at the end).  M tiles of xtu_f8_pair_tile_m()
 * rows; shapes where xtu_f8_pair_fits(H, I). */
int xtu_f8_pair_fits(int H, int I);
int xtu_f8_pair_tile_m(void);
hipError_t xtu_f8_pair_gate_up(const uint8_t* hilo, const uint8_t* shi, const int32_t* sorted_tok,
                               int H, int I, const void* w13, const float* s13, long w_estride,
                               long s_estride, const int32_t* slot_map, const int32_t* seg_start,
                               const int32_t* tile_expert, const int32_t* tile_row0,
                               const int32_t* expert_tile_start, const int32_t* tile_lo,
                               const int32_t* tile_hi, int max_tiles, void* act, float limit,
                               float alpha, float beta, hipStream_t stream);
/* xtu_f8_pair_gate_up with the activation written as the down pass's exact
 * pairs (act_hilo [A][2I], act_shi [A][I/32], the bytes xtu_pair_quant_il
 * would make of the bf16 rows, which are never written). */
hipError_t xtu_f8_pair_gate_up_q(const uint8_t* hilo, const uint8_t* shi,
                                 const int32_t* sorted_tok, int H, int I, const void* w13,
                                 const float* s13, long w_estride, long s_estride,
                                 const int32_t* slot_map, const int32_t* seg_start,
                                 const int32_t* tile_expert, const int32_t* tile_row0,
                                 const int32_t* expert_tile_start, const int32_t* tile_lo,
                                 const int32_t* tile_hi, int max_tiles, uint8_t* act_hilo,
                                 uint8_t* act_shi, float limit, float alpha, float beta,
                                 hipStream_t stream);
hipError_t xtu_f8_pair_down(const uint8_t* hilo, const uint8_t* shi, int H, int I, const void* w2,
                            const float* s2, long w_estride, long s_estride,
                            const int32_t* slot_map, const int32_t* seg_start,
                            const int32_t* tile_expert, const int32_t* tile_row0,
                            const int32_t* expert_tile_start, const int32_t* tile_lo,
                            const int32_t* tile_hi, int max_tiles, void* y, hipStream_t stream);

/* ------------------------------------------------ reference-signature small-M ABI
 * The reference's native moe4_smallm_* entry points (xiaotu_moe/csrc/
 * moe4_smallm.cu:346-430), same names, arguments and meaning, over the
 * pool's K-major MXFP4 planes: W [S][K/2][N] (byte (j, n) = codes of k = 2j,
 * 2j+1, low nibble first), SC [S][K/32][N] e8m0.  Up to 8 rows per expert.
 * They ADD into Y (fp32; the caller zeroes it), with float atomics as the
 * reference kernels.  K % 32 == 0, N % 4 == 0.
 *   gu:  Y[r][n] += sum_k W[row(e)][k][n] X[tok[r]][k], rows r of segment
 *        seg2exp[z] (row(e) = slot_map ? slot_map[e] - slot_base : e); X bf16
 *   dn:  Y[tok[r]][n] += wts[r] sum_k W[row(e)][k][n] X[r][k]; X fp32 act rows
 *   gu2: Y[e*8+c][n] += ..., rows c = the first 8 pairs (t, j) with
 *        ids[t][j] == e, e < nexp; X bf16 [T][K]
 *   dn2: Y[t_c][n] += wts[t_c][j_c] sum_k W[e][k][n] X[e*8+c][k]; X fp32 */
hipError_t moe4_smallm_init(void);
hipError_t moe4_smallm_gu(const void* W, const void* SC, const void* X, void* Y,
                          const int* seg2exp, const int* seg_start, const int* tok,
                          const int* slot_map, int slot_base, int nseg, int K, int N,
                          hipStream_t stream);
hipError_t moe4_smallm_dn(const void* W, const void* SC, const void* X, void* Y,
                          const int* seg2exp, const int* seg_start, const int* tok,
                          const float* wts, const int* slot_map, int slot_base, int nseg, int K,
                          int N, hipStream_t stream);
hipError_t moe4_smallm_gu2(const void* W, const void* SC, const void* X, void* Y, const int* ids,
                           int T, int TOPSEL, int nexp, int K, int N, hipStream_t stream);
hipError_t moe4_smallm_dn2(const void* W, const void* SC, const void* X, void* Y, const int* ids,
                           const float* wts, int T, int TOPSEL, int nexp, int K, int N,
                           hipStream_t stream);

/* ------------------------------------------------ pool-miss split
 * Pairs whose expert is resident in the GPU pool run on the device, the
 * others on a host engine; the results are added
 * (vllm_xiaotu_moe/mixed_experts.py:2956-3186).
 *
 * xtu_pin_split: the pool path's pin mask (vllm_xiaotu_moe/pin_mask_triton.py:
 * 53-85).  For each of n pairs, bad = id < 0 || id >= n_local, sl =
 * slotmap[id], res = !bad && sl >= n_local:
 *   cpu_ids = res||bad ? 0 : id,  cpu_w = res||bad ? 0 : w,
 *   part_ids = res ? sl - n_local : -1,  part_w = res ? w : 0,
 * *hits += resident pairs (hits may be NULL). */
hipError_t xtu_pin_split(const int32_t* ids, const float* wts, int n, const int32_t* slotmap,
                         int n_local, int32_t* cpu_ids, float* cpu_w, int32_t* part_ids,
                         float* part_w, unsigned long long* hits, hipStream_t stream);
/* Host engine over the pinned host copy of a layer (the reference engine's
 * CPU MoE behind cpu_decode, xiaotu_moe/csrc/python_binding/binding.cpp:
 * 859-1296).  w13_nodes / w2_nodes: ns NUMA-node buffers of P16 rows
 * ([expert][gate rows | up rows] and [expert][rows] of the node; strides in
 * bytes per expert); s13 / s2: packed scale groups (fp4), fp32 block
 * scales (fp8), or fp32 [N][K/group_k] row scales (fmt 4, INT4/WNA16:
 * value = code - 8, the engine's MOE_WNA16, moe_v2_packed4_base.inc:1-20,
 * :1594); gs13 [E][2] / gs2 [E]: NVFP4 second-level scales.  isa: -1 best available, 0
 * portable, 2 AVX-512.  max_tokens > 0 allocates the pinned staging of
 * xtu_cpu_decode (max_tokens rows of max_topk pairs); 0 = host-only engine.
 * The weights are read in place and must outlive the engine. */
hipError_t xtu_cpu_engine_create(int fmt, int H, int I, int n_experts, int ns,
                                 const void* const* w13_nodes, long w13_estride,
                                 const void* const* w2_nodes, long w2_estride, const void* s13,
                                 long s13_estride, const void* s2, long s2_estride,
                                 const float* gs13, const float* gs2, int group_k, float limit,
                                 float alpha, float beta, int n_threads, int isa, int max_tokens,
                                 int max_topk, void** engine);
hipError_t xtu_cpu_engine_info(const void* engine, int* isa, int* threads);
/* Synchronous, host memory: out [T][H] fp32 = sum over pairs with
 * 0 <= id < n_experts and w != 0 of w * expert(x); x bf16 [T][H]. */
hipError_t xtu_cpu_forward(void* engine, int T, int K, const void* x, const int32_t* ids,
                           const float* wts, float* out);
/* cpu_decode (binding.cpp:859): on `stream`, device x/ids/wts -> pinned
 * staging, a host-function node runs the engine, pinned fp32 result -> out
 * [T][H] on the device.  Allocates nothing: may be captured into a HIP graph
 * (the captured call lives until the engine is destroyed).  T <= max_tokens,
 * K <= max_topk; calls on one engine share its staging (one stream). */
hipError_t xtu_cpu_decode(void* engine, int T, int K, const void* x, const int32_t* ids,
                          const float* wts, float* out, hipStream_t stream);
/* After every stream that ran its calls is synchronised and the graphs that
 * captured them are destroyed. */
hipError_t xtu_cpu_engine_destroy(void* engine);

#ifdef __cplusplus
}
#endif

#endif /* XTU_MOE_AMD_H */
