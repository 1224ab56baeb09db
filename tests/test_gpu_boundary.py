"""The drop-in boundary called the way the reference's callers call it, each
result checked against the oracle:

* FP8 layer entries with the pool's / ring's scale planes (uint8 planes of
  fp32 bytes, gpu_prefill_fp8.py:489-496), and gpu_moe_decode_fp8 above 16
  tokens (the caller uses it up to 32, mixed_experts.py:2133-2141);
* a pool's planes star-unpacked into gpu_moe_layer with its slot;
* the device pack cache: planes rewritten in place, or a new tensor at the
  same address, are packed again; host planes are not kept on the device;
* scratch buffers bounded over many batch sizes;
* the hook writes `output` directly and takes the fused router path;
* decode batches where an expert holds more than 16 rows (a token listing an
  expert twice, zero-weight pairs kept);
* the engine's host-buffer ABI: shard_geometry keys, per-node shard copies
  and pitched copies reassemble the device layout byte for byte.
"""
import types

import numpy as np
import pytest
import torch

import oracle
from helpers import (bf16_tensor_to_bits, check_close, dense_to_numpy, make_dense_layer,
                     oracle_layer, random_routing)
from xtu_moe_amd import formats as F
from xtu_moe_amd import gpu_prefill as GP
from xtu_moe_amd import layer as L
from xtu_moe_amd.engine import MOE_FP8, MOE_MXFP4, MOEConfigV2
from xtu_moe_amd.expert_pool import LayerPool
from xtu_moe_amd.layer import ExpertWeights, moe_forward
from xtu_moe_amd.mixed_experts import XiaotuExpertsMxfp4

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _x(T, H, seed):
    return torch.randn((T, H), generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)


def _u8_scale_plane(s_kmajor):
    """fp32 [S, a, b] -> the reference pool's uint8 plane [S, a, b*4] (same bytes)."""
    return s_kmajor.contiguous().view(torch.uint8)


@pytest.mark.parametrize("T", [3, 24])
def test_fp8_entries_take_u8_scale_planes(T):
    E, H, I, K = 8, 512, 256, 4
    d = make_dense_layer(F.FMT_FP8, E, H, I, seed=40)
    ids, wts = random_routing(T, K, E, seed=41)
    x = _x(T, H, 42)
    km = lambda t: t.transpose(1, 2).contiguous().to(DEV)
    w13t, w2t = km(d["w13"]), km(d["w2"])
    s13u, s2u = _u8_scale_plane(km(d["s13"])), _u8_scale_plane(km(d["s2"]))
    assert s13u.dtype == torch.uint8 and s13u.shape == (E, H // 128, 2 * I // 128 * 4)
    ref = oracle_layer(F.FMT_FP8, dense_to_numpy(F.FMT_FP8, d), bf16_tensor_to_bits(x), ids, wts,
                       E, 0, H, I, limit=7.0)
    ti, tw = torch.from_numpy(ids).to(DEV), torch.from_numpy(wts).to(DEV)
    for fn in (GP.gpu_moe_layer_fp8, GP.gpu_moe_decode_fp8):
        out = fn(x.to(DEV), ti, tw, w13t, s13u, w2t, s2u, H, I, K, device=DEV, swiglu_limit=7.0)
        torch.cuda.synchronize()
        assert out.dtype == torch.float32
        check_close(out.cpu().numpy(), ref, bf16_out=False, what=f"{fn.__name__} T={T}")
    # a plane of the wrong shape is refused, not misread
    with pytest.raises(ValueError):
        GP.gpu_moe_layer_fp8(x.to(DEV), ti, tw, w13t, s13u[:, :, :-4], w2t, s2u, H, I, K,
                             device=DEV)


def test_pool_planes_star_unpacked_with_slot():
    E, H, I, T, K = 16, 512, 256, 10, 2
    fmt = F.FMT_MXFP4
    d = make_dense_layer(fmt, E, H, I, seed=43)
    W = ExpertWeights.from_dense(fmt, d["w13"], d["s13"], d["w2"], d["s2"], device=DEV)
    cfg = MOEConfigV2(expert_num=E, top_k=K, hidden_size=H, intermediate_size=I)
    eng = MOE_MXFP4(cfg, d["w13"], d["w2"], d["s13"], d["s2"], device=DEV)
    pinned = [2, 5, 11, 14]
    pool = LayerPool(eng, DEV, H, I, 32, E, pinned, 0, layout="mxfp4")
    ids, wts = random_routing(T, K, E, seed=44)
    x = _x(T, H, 45)
    # the reference's call: ids are pool slot rows, non-resident pairs -1
    sm = pool.slotmap.cpu().numpy()
    res = sm[np.clip(ids, 0, E - 1)] >= E
    part = np.where(res, sm[np.clip(ids, 0, E - 1)] - E, -1).astype(np.int32)
    out = GP.gpu_moe_layer(x.to(DEV), torch.from_numpy(part).to(DEV),
                           torch.from_numpy(np.where(res, wts, 0).astype(np.float32)).to(DEV),
                           *pool.planes, H, I, K, device=DEV, slot=pool.as_slot(),
                           out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x),
                       np.where(res, ids, -1).astype(np.int32), wts, E, 0, H, I)
    check_close(out.cpu().numpy(), ref, bf16_out=False, what="pool planes + slot")


def test_pack_cache_sees_rewrites_and_reused_addresses():
    E, H, I, T, K = 8, 512, 256, 12, 2
    fmt = F.FMT_MXFP4
    da = make_dense_layer(fmt, E, H, I, seed=46)
    db = make_dense_layer(fmt, E, H, I, seed=47)
    ids, wts = random_routing(T, K, E, seed=48)
    x = _x(T, H, 49)
    ti, tw = torch.from_numpy(ids).to(DEV), torch.from_numpy(wts).to(DEV)
    planes = [da[k].to(DEV) for k in ("w13", "s13", "w2", "s2")]

    def run(ps):
        o = GP.gpu_moe_layer(x.to(DEV), ti, tw, *ps, H, I, K, device=DEV, out_dtype=torch.float32)
        torch.cuda.synchronize()
        return o.cpu().numpy()

    ref_a = oracle_layer(fmt, dense_to_numpy(fmt, da), bf16_tensor_to_bits(x), ids, wts, E, 0, H, I)
    ref_b = oracle_layer(fmt, dense_to_numpy(fmt, db), bf16_tensor_to_bits(x), ids, wts, E, 0, H, I)
    check_close(run(planes), ref_a, bf16_out=False, what="first contents")
    for p, k in zip(planes, ("w13", "s13", "w2", "s2")):   # rewritten in place
        p.copy_(db[k].to(DEV))
    check_close(run(planes), ref_b, bf16_out=False, what="rewritten in place")
    # same address, new tensor objects (views of the same storage)
    views = [p.view(p.shape) for p in planes]
    check_close(run(views), ref_b, bf16_out=False, what="views")
    n_before = len(GP._PACKED)
    # host planes: packed per call, nothing kept
    host = [da[k] for k in ("w13", "s13", "w2", "s2")]
    check_close(run(host), ref_a, bf16_out=False, what="host planes")
    assert len(GP._PACKED) == n_before
    assert len(GP._PACKED) <= GP.PACK_CACHE_MAX


def test_scratch_stays_bounded_over_many_batch_sizes():
    fmt, E, NS, H, I, K = F.FMT_MXFP4, 16, 1, 256, 256, 4
    d = make_dense_layer(fmt, E + NS, H, I, seed=50)
    W = ExpertWeights.from_dense(fmt, d["w13"], d["s13"], d["w2"], d["s2"], n_shared=NS,
                                 device=DEV)
    sizes = list(range(17, 300, 7))
    for T in sizes:
        ids, wts = random_routing(T, K, E, seed=T)
        moe_forward(_x(T, H, T).to(DEV), torch.from_numpy(ids).to(DEV),
                    torch.from_numpy(wts).to(DEV), W, out_dtype=torch.float32)
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    n_seg, n_buf = len(L._SEG_CACHE), len(L._BUF_CACHE)
    for T in sizes:   # a second pass allocates nothing new
        ids, wts = random_routing(T, K, E, seed=T + 1)
        out = moe_forward(_x(T, H, T).to(DEV), torch.from_numpy(ids).to(DEV),
                          torch.from_numpy(wts).to(DEV), W, out_dtype=torch.float32)
        del out
    torch.cuda.synchronize()
    assert len(L._SEG_CACHE) == n_seg and len(L._BUF_CACHE) == n_buf
    assert torch.cuda.memory_allocated() <= base + (1 << 20)
    # retired buffers: geometric growth, so fewer than log2(T_max) generations each
    assert len(L._RETIRED) <= 8 * (n_seg + n_buf)
    T = sizes[-1]
    ids, wts = random_routing(T, K, E, seed=51)
    x = _x(T, H, 52)
    out = moe_forward(x.to(DEV), torch.from_numpy(ids).to(DEV), torch.from_numpy(wts).to(DEV),
                      W, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x), ids, wts, E, NS, H, I)
    check_close(out.cpu().numpy(), ref, bf16_out=False, what="after the size sweep")


def _hook(E, H, I, seed):
    d = make_dense_layer(F.FMT_MXFP4, E, H, I, seed=seed)
    bias = torch.randn(E, generator=torch.Generator().manual_seed(seed)) * 0.05
    lay = types.SimpleNamespace(w13_weight=d["w13"], w2_weight=d["w2"], top_k=8,
                                use_grouped_topk=True, renormalize=True, scoring_func="sigmoid",
                                num_expert_group=8, topk_group=4, routed_scaling_factor=2.5,
                                e_score_correction_bias=bias, swiglu_limit=7.0,
                                w13_weight_scale=d["s13"], w2_weight_scale=d["s2"])
    hook = XiaotuExpertsMxfp4()
    hook.process_weights_after_loading(lay)
    return d, bias, hook


@pytest.mark.parametrize("T", [1, 4, 40])
def test_hook_writes_output_directly_and_matches_oracle(T):
    E, H, I = 64, 512, 256
    d, bias, hook = _hook(E, H, I, seed=53)
    x = _x(T, H, 54).to(DEV)
    logits = torch.randn((T, E), generator=torch.Generator().manual_seed(55)).to(DEV)
    buf = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device=DEV)
    res = hook.apply(x, None, None, router_logits=logits, output=buf)
    torch.cuda.synchronize()
    assert res is buf
    rids, rwts = oracle.route_grouped_sigmoid(logits.cpu().numpy(), bias.numpy(), 8, 4, 8, 2.5)
    ref = oracle_layer(F.FMT_MXFP4, dense_to_numpy(F.FMT_MXFP4, d), bf16_tensor_to_bits(x),
                       rids, rwts, E, 0, H, I, limit=7.0)
    check_close(buf.float().cpu().numpy(), ref, bf16_out=True, what=f"hook T={T}")
    # fp32 hidden states: an fp32 output buffer is written directly as well
    buf32 = torch.empty((T, H), dtype=torch.float32, device=DEV)
    assert hook.apply(x.float(), None, None, router_logits=logits, output=buf32) is buf32
    torch.cuda.synchronize()
    check_close(buf32.cpu().numpy(), ref, bf16_out=False, what=f"hook fp32 T={T}")


@pytest.mark.parametrize("fused", ["1", "0"])
@pytest.mark.parametrize("fmt", [F.FMT_MXFP4, F.FMT_FP8])
def test_decode_expert_with_more_than_16_rows(fmt, fused, monkeypatch):
    monkeypatch.setenv(L.FUSED_DOWN_ENV, fused)
    E, NS, H, I, T, K = 16, 1, 512, 256, 16, 4
    d = make_dense_layer(fmt, E + NS, H, I, seed=56)
    W = ExpertWeights.from_dense(fmt, d["w13"], d["s13"], d["w2"], d["s2"], n_shared=NS,
                                 device=DEV)
    ids, wts = random_routing(T, K, E, seed=57)
    ids[:, 1] = ids[:, 0] = 3          # every token lists expert 3 twice: 32 rows
    x = _x(T, H, 58)
    dn = dense_to_numpy(fmt, d)
    for t in L._BUF_CACHE.values():    # rows the kernels fail to write show up as NaN
        if t.is_floating_point():
            t.fill_(float("nan"))
    out = moe_forward(x.to(DEV), torch.from_numpy(ids).to(DEV), torch.from_numpy(wts).to(DEV), W,
                      path="decode", out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = oracle_layer(fmt, dn, bf16_tensor_to_bits(x), ids, wts, E, NS, H, I)
    check_close(out.cpu().numpy(), ref, bf16_out=False, what="duplicated expert, 32 rows")
    # expert-parallel masking: remote pairs mapped to local expert 0 with
    # weight 0 and kept (drop_zero=False) -- 40 rows in expert 0's bucket
    ids2, wts2 = random_routing(T, K, E, seed=59)
    remote = np.random.default_rng(60).random((T, K)) < 0.6
    ids2[remote], wts2[remote] = 0, 0.0
    out2 = moe_forward(x.to(DEV), torch.from_numpy(ids2).to(DEV), torch.from_numpy(wts2).to(DEV),
                       W, path="decode", drop_zero=False, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref2 = oracle_layer(fmt, dn, bf16_tensor_to_bits(x), ids2, wts2, E, NS, H, I)
    check_close(out2.cpu().numpy(), ref2, bf16_out=False, what="masked pairs kept")


def test_engine_shard_abi_reassembles_device_layout(monkeypatch):
    monkeypatch.setenv("XIAOTU_MOE_NSHARD", "2")
    E, H, I, K = 6, 512, 256, 2
    d = make_dense_layer(F.FMT_FP8, E, H, I, seed=61)
    cfg = MOEConfigV2(expert_num=E, top_k=K, hidden_size=H, intermediate_size=I, groupN=128,
                      groupK=128)
    eng = MOE_FP8(cfg, d["w13"], d["w2"], d["s13"], d["s2"], device=DEV)
    g = eng.shard_geometry()
    assert set(g) == {"ns", "w13_node_bytes", "w2_node_bytes", "w13_scale_bytes",
                      "w2_scale_bytes", "w13_crows", "w13_cbytes", "w2_crows", "w2_cbytes"}
    assert g["ns"] == 2 and g["w13_crows"] == I // 2 and g["w2_crows"] == H // 2
    assert g["w13_cbytes"] == g["w13_crows"] * H and g["w2_cbytes"] == g["w2_crows"] * I
    assert g["w13_node_bytes"] == E * 2 * g["w13_cbytes"] and g["w2_node_bytes"] == E * g["w2_cbytes"]
    assert eng.pin_hostbufs() == 2 + 2 + 2
    W = eng.weights
    st = torch.cuda.current_stream().cuda_stream
    # whole node shards, then the pitched copies that place them
    w13 = torch.zeros_like(W.w13)
    w2 = torch.zeros_like(W.w2)
    c13, c2 = g["w13_cbytes"], g["w2_cbytes"]
    e13, e2 = W.w13.shape[1], W.w2.shape[1]
    for n in range(2):
        shard = torch.empty(g["w13_node_bytes"], dtype=torch.uint8, device=DEV)
        assert eng.copy_hostbuf_to_device(0, n, shard.data_ptr(), st) == g["w13_node_bytes"]
        torch.cuda.synchronize()
        s = shard.view(E, 2 * c13)
        w13[:, n * c13:(n + 1) * c13] = s[:, :c13]
        w13[:, I * H + n * c13:I * H + (n + 1) * c13] = s[:, c13:]
        # gate half of node n straight into place with one pitched copy
        assert eng.copy_hostbuf_to_device_2d(0, n, 0, w13.data_ptr() + n * c13, e13, 2 * c13,
                                             c13, E, st) == c13 * E
        assert eng.copy_hostbuf_to_device_2d(1, n, 0, w2.data_ptr() + n * c2, e2, c2, c2, E,
                                             st) == c2 * E
    torch.cuda.synchronize()
    assert torch.equal(w13, W.w13) and torch.equal(w2, W.w2)
    s13 = torch.empty_like(W.s13)
    assert eng.copy_hostbuf_to_device(2, 0, s13.data_ptr(), st) == g["w13_scale_bytes"]
    torch.cuda.synchronize()
    assert torch.equal(s13, W.s13)
    # bad requests return 0, as the reference's do
    assert eng.copy_hostbuf_to_device(0, 5, w13.data_ptr(), st) == 0
    assert eng.copy_hostbuf_to_device_2d(0, 0, 0, w13.data_ptr(), e13, 2 * c13, c13, E + 1, st) == 0
    # negative or zero sizes and pitches are refused before any copy is queued
    for bad in ((-1, c13, e13, 2 * c13), (E, -c13, e13, 2 * c13), (E, c13, -e13, 2 * c13),
                (E, c13, e13, -2 * c13), (0, c13, e13, 2 * c13)):
        h, wdt, dp, sp = bad
        assert eng.copy_hostbuf_to_device_2d(0, 0, 0, w13.data_ptr(), dp, sp, wdt, h, st) == 0
