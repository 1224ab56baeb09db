"""The benchmark configurations at their full shapes on the GPU, against the
oracle (where the whole batch would take the CPU too long, a set of tokens
that covers every routed expert, chosen greedily)
plus properties that hold at any size:

* tiny Mixtral-style bf16 layer: H=1024, 8 experts, I=2048, softmax top-2
  renormalised, T=128 -- routing bit-exact and every token against the oracle;
* Qwen3-Next shape: H=2048, I=512, 512 routed + 1 shared experts, softmax
  top-10, SwiGLU clamp 7 -- INT8-activation x MXFP4 at T=8192 (sampled
  tokens covering every routed expert, the token-permutation bitwise
  property, the int32 accumulators of sampled tiles bit-exact), INT8 forced
  at T=1 and 4, NVFP4 at T=1, 4 and 8192, MXFP4 decode at T=1, 4;
* DeepSeek-V3 FP8 streamed prefill: 64 resident experts (+ the shared one)
  in the pool, the other 192 streamed from pinned host memory through a
  ring of 4 slots of 16 experts, Zipf(1.1)-skewed routing, T=8192 -- bitwise
  equal to the all-resident layer, and tokens covering every routed expert
  (the last rows of eight experts' buckets among them) against the oracle.
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import (MAX_ABS, REL_L2, bf16_tensor_to_bits, check_close, cover_tokens,
                     dense_to_numpy, make_dense_layer, oracle_layer, rel_l2, sampled_oracle)
from xtu_moe_amd import _lib
from xtu_moe_amd import formats as F
from xtu_moe_amd import layer as L
from xtu_moe_amd.expert_pool import LayerPool
from xtu_moe_amd.host_store import HostExpertStore
from xtu_moe_amd.layer import ExpertWeights, _p, _stream, moe_forward, route, segmentation
from xtu_moe_amd.ring import RingStats, gpu_moe_layer_from_engine_tiled
from xtu_moe_amd.synthetic import dense_experts, synth_layer

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _sampled_oracle(fmt, W, x, ids, wts, toks, limit=0.0, int8=False):
    return sampled_oracle(fmt, W, x, ids, wts, toks, limit=limit, int8=int8)


def _cover(ids, E, NS, seed):
    """Tokens covering every routed expert of the batch (and the shared ones,
    which every token uses), with the last token of 8 experts' buckets."""
    toks, covered = cover_tokens(ids.cpu().numpy(), E, seed=seed)
    routed = int(torch.unique(ids[(ids >= 0) & (ids < E)]).numel())
    # every routed expert, plus the NS shared ones that each sampled token runs
    assert len(covered) + NS == routed + NS and len(toks) > 0
    return toks


# ------------------------------------------------------------- tiny Mixtral
def test_mixtral_tiny_whole_batch_matches_oracle():
    H, E, I, K, T = 1024, 8, 2048, 2, 128
    fmt = F.FMT_BF16
    d = make_dense_layer(fmt, E, H, I, seed=0)
    W = ExpertWeights.from_dense(fmt, d["w13"], d["s13"], d["w2"], d["s2"], device=DEV)
    g = torch.Generator().manual_seed(0)
    x = torch.randn((T, H), generator=g).to(torch.bfloat16)
    wr = torch.randn((E, H), generator=g) * 0.02
    logits = (x.float() @ wr.T).contiguous()
    rids, rwts = oracle.route_softmax_topk(logits.numpy(), K)
    ids = torch.empty((T, K), dtype=torch.int32, device=DEV)
    wts = torch.empty((T, K), dtype=torch.float32, device=DEV)
    out = moe_forward(x.to(DEV), ids, wts, W, out_dtype=torch.bfloat16,
                      router=dict(logits=logits.to(DEV), scoring="softmax"))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    np.testing.assert_array_equal(wts.cpu().numpy().view(np.uint32), rwts.view(np.uint32))
    ref = oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x), rids, rwts, E, 0, H, I)
    check_close(out.float().cpu().numpy(), ref, bf16_out=True, what="mixtral T=128 (all tokens)")


# -------------------------------------------------------------- Qwen3-Next
QH, QI, QE, QNS, QK, QLIM = 2048, 512, 512, 1, 10, 7.0


@pytest.fixture(scope="module")
def qwen_mxfp4():
    W = synth_layer(F.FMT_MXFP4, QE, QNS, QH, QI, seed=4, device=DEV)
    yield W
    del W
    torch.cuda.empty_cache()


def _qwen_batch(T, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn((T, QH), generator=g, device=DEV).to(torch.bfloat16)
    logits = torch.randn((T, QE), generator=g, device=DEV)
    wts, ids = route(logits, top_k=QK, scoring="softmax")
    return x, logits, ids, wts


def test_qwen3_next_int8_t8192(qwen_mxfp4):
    W = qwen_mxfp4
    T = 8192
    x, logits, ids, wts = _qwen_batch(T, seed=5)
    toks = _cover(ids, QE, QNS, seed=6)
    rids, rwts = oracle.route_softmax_topk(logits[toks].cpu().numpy(), QK)
    np.testing.assert_array_equal(ids[toks].cpu().numpy(), rids)
    np.testing.assert_array_equal(wts[toks].cpu().numpy().view(np.uint32), rwts.view(np.uint32))
    out = moe_forward(x, ids, wts, W, int8=True, swiglu_limit=QLIM, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = _sampled_oracle(F.FMT_MXFP4, W, x, ids, wts, toks, limit=QLIM, int8=True)
    check_close(out[toks].cpu().numpy(), ref, bf16_out=False, what="qwen3-next int8 T=8192")
    # permuting the batch permutes the output bit for bit
    perm = torch.randperm(T, generator=torch.Generator().manual_seed(7)).to(DEV)
    out_p = moe_forward(x[perm].contiguous(), ids[perm].contiguous(), wts[perm].contiguous(), W,
                        int8=True, swiglu_limit=QLIM, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(out_p, out[perm])


def test_qwen3_next_int8_accumulators_bit_exact(qwen_mxfp4):
    """The int32 accumulators of the gate/up GEMM for three m tiles of a
    T=8192 batch equal the oracle's integer closed form."""
    W = qwen_mxfp4
    T = 8192
    x, _, ids, wts = _qwen_batch(T, seed=8)
    NS, E, H, I = W.n_shared, W.E, W.H, W.I
    w13_8, emin13, _, _ = W.int8_planes()
    seg = segmentation(T, QK, E, NS, 128, DEV).run(ids, wts)
    A = seg.A
    st = _stream()
    a8x = torch.empty((T, H), dtype=torch.int8, device=DEV)
    crx = torch.empty(T, dtype=torch.int32, device=DEV)
    _lib.call("xtu_i8_quant_rows", _p(x), T, H, _p(a8x), _p(crx), st)
    act = torch.empty((A, I), dtype=torch.bfloat16, device=DEV)
    acc = torch.zeros((A, 2 * I), dtype=torch.int32, device=DEV)
    lo, hi = seg.tile_range_ptrs(0, E + NS)
    _lib.call("xtu_i8_gemm_gate_up", _p(a8x), _p(crx), _p(seg.sorted_tok), H, I, _p(w13_8),
              _p(emin13), 0, _p(seg.seg_start), _p(seg.tile_expert), _p(seg.tile_row0), lo, hi,
              seg.max_tiles, _p(act), _p(acc), QLIM, 1.0, 0.0, st)
    torch.cuda.synchronize()
    n_tiles = int(seg.n_tiles.item())
    te, tr = seg.tile_expert.cpu().numpy(), seg.tile_row0.cpu().numpy()
    ss, stok = seg.seg_start.cpu().numpy(), seg.sorted_tok.cpu().numpy()
    for t in (0, n_tiles // 2, n_tiles - 1):   # the last tile is a shared-expert tile
        e, r0 = int(te[t]), int(tr[t])
        r1 = min(r0 + 128, int(ss[e + 1]))
        rows = stok[r0:r1]
        dn = dense_experts(W, [e])
        xf = oracle.bf16_bits_to_f32(bf16_tensor_to_bits(x[torch.from_numpy(rows).long().to(DEV)]))
        ref_acc, _, dmax = oracle.i8_gemm(xf, dn["w13"][0], dn["s13"][0])
        assert dmax <= 3
        np.testing.assert_array_equal(acc[r0:r1].cpu().numpy(), ref_acc,
                                      err_msg=f"tile {t} expert {e}")


@pytest.mark.parametrize("T", [1, 4, 8192])
def test_qwen3_next_nvfp4(T):
    W = synth_layer(F.FMT_NVFP4, QE, QNS, QH, QI, seed=9, device=DEV)
    x, _, ids, wts = _qwen_batch(T, seed=10 + T)
    out = moe_forward(x, ids, wts, W, swiglu_limit=QLIM, out_dtype=torch.float32)
    torch.cuda.synchronize()
    toks = _cover(ids, QE, QNS, seed=11)
    ref = _sampled_oracle(F.FMT_NVFP4, W, x, ids, wts, toks, limit=QLIM)
    check_close(out[toks].cpu().numpy(), ref, bf16_out=False, what=f"qwen3-next nvfp4 T={T}")
    del W
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T", [1, 4])
def test_qwen3_next_mxfp4_decode(qwen_mxfp4, T):
    W = qwen_mxfp4
    x, logits, ids, wts = _qwen_batch(T, seed=12 + T)
    ids_o = torch.empty((T, QK), dtype=torch.int32, device=DEV)
    wts_o = torch.empty((T, QK), dtype=torch.float32, device=DEV)
    out = moe_forward(x, ids_o, wts_o, W, swiglu_limit=QLIM, out_dtype=torch.bfloat16,
                      router=dict(logits=logits, scoring="softmax"))
    torch.cuda.synchronize()
    assert torch.equal(ids_o, ids) and torch.equal(wts_o, wts)
    ref = _sampled_oracle(F.FMT_MXFP4, W, x, ids, wts, list(range(T)), limit=QLIM)
    check_close(out.float().cpu().numpy(), ref, bf16_out=True, what=f"qwen3-next mxfp4 T={T}")


@pytest.mark.parametrize("T", [1, 4])
def test_qwen3_next_nvfp4_decode_routed(T):
    """NVFP4 decode routed from logits, as the layer serves it (at T = 1 the
    whole layer in one launch, the fused down included), against the oracle
    and the router's ids and weights."""
    W = synth_layer(F.FMT_NVFP4, QE, QNS, QH, QI, seed=21, device=DEV)
    x, logits, ids, wts = _qwen_batch(T, seed=22 + T)
    ids_o = torch.empty((T, QK), dtype=torch.int32, device=DEV)
    wts_o = torch.empty((T, QK), dtype=torch.float32, device=DEV)
    out = moe_forward(x, ids_o, wts_o, W, swiglu_limit=QLIM, out_dtype=torch.bfloat16,
                      router=dict(logits=logits, scoring="softmax"))
    torch.cuda.synchronize()
    assert torch.equal(ids_o, ids) and torch.equal(wts_o, wts)
    ref = _sampled_oracle(F.FMT_NVFP4, W, x, ids, wts, list(range(T)), limit=QLIM)
    check_close(out.float().cpu().numpy(), ref, bf16_out=True, what=f"qwen3-next nvfp4 routed T={T}")
    del W
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T", [1, 4])
def test_qwen3_next_int8_forced_at_decode_sizes(qwen_mxfp4, T, monkeypatch):
    """XIAOTU_MOE_INT8_ALIGN=1 takes the INT8 ALIGN path below the 160-token
    gate as well (the reference engine's override): T = 1 and 4 on the
    grouped integer GEMMs, every token against the INT8 oracle."""
    monkeypatch.setenv(L.INT8_FORCE_ENV, "1")
    assert L.int8_align_on(T)
    W = qwen_mxfp4
    x, logits, ids, wts = _qwen_batch(T, seed=30 + T)
    out, seg = moe_forward(x, ids, wts, W, int8="auto", swiglu_limit=QLIM,
                           out_dtype=torch.float32, return_seg=True)
    torch.cuda.synchronize()
    assert seg.bm == 128   # the integer GEMMs' tiles, not the decode kernels'
    ref = _sampled_oracle(F.FMT_MXFP4, W, x, ids, wts, list(range(T)), limit=QLIM, int8=True)
    check_close(out.cpu().numpy(), ref, bf16_out=False, what=f"qwen3-next forced int8 T={T}")


# ---------------------------------------------------- DeepSeek-V3 streamed
def test_ds_v3_fp8_streamed_prefill():
    H, I, E, NS, K, T = 7168, 2048, 256, 1, 8, 8192
    W = synth_layer(F.FMT_FP8, E, NS, H, I, seed=13, device=DEV)
    store = HostExpertStore.from_weights(W)
    gen = torch.Generator(device=DEV).manual_seed(14)
    rank = torch.randperm(E, generator=torch.Generator().manual_seed(15)) + 1
    skew = (-1.1 * torch.log(rank.double())).float().to(DEV)    # Zipf(1.1) popularity
    u = torch.rand((T, E), generator=gen, device=DEV).clamp_(1e-12, 1.0 - 1e-7)
    logits = skew - torch.log(-torch.log(u))
    x = torch.randn((T, H), generator=gen, device=DEV).to(torch.bfloat16)
    wts, ids = route(logits, top_k=K, scoring="sigmoid", n_group=8, topk_group=4,
                     routed_scaling_factor=2.5)
    counts = torch.bincount(ids.flatten().long(), minlength=E)
    pinned = torch.argsort(counts, descending=True, stable=True)[:64].tolist()
    pool = LayerPool(store, DEV, H, I, 128, E, pinned, 0, layout="fp8", topk=K)
    stats = RingStats()
    out = gpu_moe_layer_from_engine_tiled(store, x, ids, wts, H, I, E, K, device=DEV, nslots=4,
                                          pool=pool, tile_e=16, out_dtype=torch.float32,
                                          stats=stats)
    torch.cuda.synchronize()
    stats.finish()
    routed = set(ids.flatten().tolist())
    assert stats.tiles == (len(routed - set(pinned)) + 15) // 16
    ref = moe_forward(x, ids, wts, W, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    toks = _cover(ids, E, NS, seed=16)
    want = _sampled_oracle(F.FMT_FP8, W, x, ids, wts, toks)
    check_close(out[toks].cpu().numpy(), want, bf16_out=False, what="ds-v3 fp8 streamed")
    del W, store, pool
    torch.cuda.empty_cache()


# ------------------------------------------------------ DeepSeek-V3 MXFP4 prefill
_ORACLE_CACHE: dict = {}


@pytest.mark.parametrize("mode", ["tri", "pair", "bf16"])
def test_ds_v3_mxfp4_prefill_t8192(mode, monkeypatch):
    """DeepSeek-V3 shape with MXFP4 experts at T=8192, on the double-rate fp6
    / fp4 MFMA (activation triples), the scaled fp8 x fp4 MFMA (exact
    activation pairs) and the bf16-operand GEMM: sampled tokens against the
    oracle, and the token-permutation bitwise property."""
    monkeypatch.setenv(L.MXFP4_PREFILL_ENV, mode)
    assert L.mx_tri(F.FMT_MXFP4, 7168, 2048) == (mode == "tri")
    assert mode == "bf16" or L.mx_act_mode(F.FMT_MXFP4, 7168, 2048) == mode
    H, I, E, NS, K, T = 7168, 2048, 256, 1, 8, 8192
    W = synth_layer(F.FMT_MXFP4, E, NS, H, I, seed=17, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(18)
    x = torch.randn((T, H), generator=g, device=DEV).to(torch.bfloat16)
    logits = torch.randn((T, E), generator=g, device=DEV)
    wts, ids = route(logits, top_k=K, scoring="sigmoid", n_group=8, topk_group=4,
                     routed_scaling_factor=2.5)
    out = moe_forward(x, ids, wts, W, out_dtype=torch.float32)
    torch.cuda.synchronize()
    toks = _cover(ids, E, NS, seed=19)
    key = ("ds-v3-mxfp4", tuple(toks))
    if key not in _ORACLE_CACHE:   # the three modes share weights, tokens and routing
        _ORACLE_CACHE.clear()
        _ORACLE_CACHE[key] = _sampled_oracle(F.FMT_MXFP4, W, x, ids, wts, toks)
    ref = _ORACLE_CACHE[key]
    check_close(out[toks].cpu().numpy(), ref, bf16_out=False, what="ds-v3 mxfp4 T=8192")
    perm = torch.randperm(T, generator=torch.Generator().manual_seed(20)).to(DEV)
    out_p = moe_forward(x[perm].contiguous(), ids[perm].contiguous(), wts[perm].contiguous(), W,
                        out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(out_p, out[perm])
    del W
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T", [40, 700])
def test_mxfp4_prefill_pair_and_bf16_paths(T, monkeypatch):
    """MXFP4 prefill at a shape the 32x32x64 kernel does not take (I = 384):
    "pair" runs the 16x16x128 exact-pair kernel, "bf16" the bf16-operand
    GEMM, and "tri" (the default's mode) falls back to the bf16-operand GEMM;
    each against the oracle, with a SwiGLU clamp and a shared expert."""
    E, NS, H, I, K = 24, 1, 768, 384, 4
    d = make_dense_layer(F.FMT_MXFP4, E + NS, H, I, seed=21)
    W = ExpertWeights.from_dense(F.FMT_MXFP4, d["w13"], d["s13"], d["w2"], d["s2"], n_shared=NS,
                                 device=DEV)
    rng = np.random.default_rng(22)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    wts = (rng.random((T, K)) + 0.05).astype(np.float32)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(23)).to(torch.bfloat16)
    ref = oracle_layer(F.FMT_MXFP4, dense_to_numpy(F.FMT_MXFP4, d), bf16_tensor_to_bits(x), ids,
                       wts, E, NS, H, I, limit=4.0)
    for mode in ("pair", "bf16", "tri"):
        monkeypatch.setenv(L.MXFP4_PREFILL_ENV, mode)
        assert L.pair_gemm(F.FMT_MXFP4, H, I) == (mode == "pair")
        out = moe_forward(x.to(DEV), torch.from_numpy(ids).to(DEV), torch.from_numpy(wts).to(DEV),
                          W, path="gemm", swiglu_limit=4.0, out_dtype=torch.float32)
        torch.cuda.synchronize()
        check_close(out.cpu().numpy(), ref, bf16_out=False, what=f"mxfp4 {mode} T={T}")
