"""Ring stage, resident pool, engine and hook surfaces on the GPU.

The ring-streamed layer (experts copied tile by tile from pinned host memory,
pool-resident experts read in place) equals the all-resident layer bit for
bit and the oracle within tolerance; the pool's resident part equals the
layer restricted to the resident experts and the oracle restricted the same
way, before and after swaps; the engine, the quant-method hook and the
reference-signature layer entries agree with the oracle / the direct call."""
import os
import types

import numpy as np
import pytest
import torch

import oracle
from helpers import (bf16_tensor_to_bits, check_close, dense_to_numpy, make_dense_layer,
                     oracle_layer, random_routing)
from xtu_moe_amd import formats as F
from xtu_moe_amd import gpu_prefill as GP
from xtu_moe_amd.engine import MOE_FP8, MOE_MXFP4, MOEConfigV2
from xtu_moe_amd.expert_pool import LayerPool
from xtu_moe_amd.host_store import HostExpertStore
from xtu_moe_amd.layer import ExpertWeights, moe_forward, route
from xtu_moe_amd.mixed_experts import XiaotuExpertsFp8, XiaotuExpertsMxfp4
from xtu_moe_amd.ring import RingStats, gpu_moe_layer_from_engine_tiled

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _layer(fmt, E, NS, H, I, seed):
    d = make_dense_layer(fmt, E + NS, H, I, seed=seed)
    W = ExpertWeights.from_dense(fmt, d["w13"], d["s13"], d["w2"], d["s2"], d["gs13"], d["gs2"],
                                 n_shared=NS, device=DEV)
    return d, W


def _oracle(fmt, d, x, ids, wts, E, NS, H, I, keep=None):
    """The oracle layer; with `keep`, only those routed experts' pairs."""
    ids = ids.cpu().numpy().copy() if torch.is_tensor(ids) else ids.copy()
    wts = wts.cpu().numpy() if torch.is_tensor(wts) else wts
    if keep is not None:
        ids[~np.isin(ids, list(keep))] = -1
    return oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x), ids, wts, E, NS,
                        H, I)


def _inputs(T, K, E, H, seed, invalid=0.0):
    ids, wts = random_routing(T, K, E, seed=seed, invalid_frac=invalid)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((T, H), generator=g).to(torch.bfloat16)
    return x.to(DEV), torch.from_numpy(ids).to(DEV), torch.from_numpy(wts).to(DEV)


@pytest.mark.parametrize("fmt", [F.FMT_FP8, F.FMT_MXFP4, F.FMT_NVFP4])
@pytest.mark.parametrize("nslots", [2, 3])
def test_ring_equals_resident_layer_bitwise(fmt, nslots):
    E, NS, H, I, T, K = 32, 1, 512, 256, 300, 4
    d, W = _layer(fmt, E, NS, H, I, seed=fmt + 30)
    x, ids, wts = _inputs(T, K, E, H, seed=7, invalid=0.05)
    ref = moe_forward(x, ids, wts, W, path="gemm", out_dtype=torch.float32)
    store = HostExpertStore.from_weights(W)
    pool = LayerPool(store, DEV, H, I, 32, E, [3, 0, 17, 9], 0, layout=F.FMT_NAMES[fmt])
    st = RingStats()
    out = gpu_moe_layer_from_engine_tiled(store, x, ids, wts, H, I, E, K, device=DEV,
                                          nslots=nslots, pool=pool, tile_e=5,
                                          out_dtype=torch.float32, stats=st)
    torch.cuda.synchronize()
    st.finish()
    routed = set(ids[(ids >= 0) & (ids < E)].tolist())
    streamed = routed - {3, 0, 17, 9}
    assert st.tiles == (len(streamed) + 4) // 5
    assert st.bytes == len(streamed) * store.expert_bytes()
    np.testing.assert_array_equal(out.cpu().numpy(), ref.cpu().numpy())
    check_close(out.cpu().numpy(), _oracle(fmt, d, x, ids, wts, E, NS, H, I), bf16_out=False,
                what=f"ring fmt={fmt}")


def test_ring_takes_the_engine_object_and_accumulates_into_out():
    """The reference calls the ring with its engine object and E, and adds
    the layer into a given `out` (gpu_prefill.py:2984-3095)."""
    E, H, I, T, K = 24, 512, 256, 200, 4
    fmt = F.FMT_FP8
    d = make_dense_layer(fmt, E, H, I, seed=34)
    cfg = MOEConfigV2(expert_num=E, top_k=K, hidden_size=H, intermediate_size=I, groupN=128,
                      groupK=128)
    eng = MOE_FP8(cfg, d["w13"], d["w2"], d["s13"], d["s2"], device=DEV)
    x, ids, wts = _inputs(T, K, E, H, seed=35, invalid=0.05)
    wts[::7, 0] = 0.0     # zero-weight pairs: skipped, their experts need not stream
    base = torch.randn((T, H), generator=torch.Generator().manual_seed(36)).to(DEV)
    out = base.clone()
    st = RingStats()
    got = gpu_moe_layer_from_engine_tiled(eng, x, ids, wts, H, I, E, K, device=DEV,
                                          group_k=128, nslots=2, out=out, tile_e=4, stats=st)
    torch.cuda.synchronize()
    assert got is out
    ref = _oracle(fmt, d, x, ids, wts, E, 0, H, I)
    check_close((out - base).cpu().numpy(), ref, bf16_out=False, what="ring via engine")
    live = ((ids >= 0) & (ids < E) & (wts != 0))
    assert st.bytes == len(set(ids[live].tolist())) * eng.host_store().expert_bytes()


def test_ring_streams_shared_experts_without_a_pool():
    """Without a pool the shared experts are streamed as one more tile (the
    layer equals the all-resident one bit for bit); a layer that cannot be
    streamed (more shared experts than a tile holds and no pool, a shape
    mismatch) returns None before any copy is queued or any slot written."""
    from xtu_moe_amd import ring as R
    E, NS, H, I, T, K = 16, 1, 512, 256, 40, 2
    d, W = _layer(F.FMT_MXFP4, E, NS, H, I, seed=3)
    x, ids, wts = _inputs(T, K, E, H, seed=4)
    store = HostExpertStore.from_weights(W)
    ref = moe_forward(x, ids, wts, W, path="gemm", out_dtype=torch.float32)
    st = RingStats()
    out = gpu_moe_layer_from_engine_tiled(store, x, ids, wts, H, I, E, K, device=DEV, tile_e=4,
                                          out_dtype=torch.float32, stats=st)
    torch.cuda.synchronize()
    st.finish()
    routed = set(ids[(ids >= 0) & (ids < E)].tolist())
    assert st.tiles == (len(routed) + 3) // 4 + 1
    assert st.bytes == (len(routed) + NS) * store.expert_bytes()
    np.testing.assert_array_equal(out.cpu().numpy(), ref.cpu().numpy())
    # three shared experts do not fit a tile of two: refused, nothing queued
    _, W3 = _layer(F.FMT_MXFP4, E, 3, H, I, seed=5)
    store3 = HostExpertStore.from_weights(W3)
    n_rings = len(R._RINGS)
    assert gpu_moe_layer_from_engine_tiled(store3, x, ids, wts, H, I, E, K, device=DEV,
                                           tile_e=2) is None
    assert gpu_moe_layer_from_engine_tiled(store, x, ids, wts, H + 256, I, E, K, device=DEV) is None
    assert len(R._RINGS) == n_rings   # no ring was even allocated for them


def _restricted(W, x, ids, wts, resident):
    """The layer with only `resident` routed experts (others' pairs dropped)."""
    keep = torch.zeros(W.E, dtype=torch.bool, device=DEV)
    keep[list(resident)] = True
    ok = (ids >= 0) & (ids < W.E)
    m = ok & keep[ids.clamp(0, W.E - 1).long()]
    ids2 = torch.where(m, ids, torch.full_like(ids, -1))
    return moe_forward(x, ids2, wts, W, path="gemm", out_dtype=torch.float32)


def test_pool_resident_part_and_swaps():
    E, NS, H, I, T, K = 24, 1, 512, 256, 64, 3
    d, W = _layer(F.FMT_FP8, E, NS, H, I, seed=5)
    x, ids, wts = _inputs(T, K, E, H, seed=6)
    store = HostExpertStore.from_weights(W)
    pool = LayerPool(store, DEV, H, I, 128, E, [1, 4, 7, 10, 13, 16], 0, layout="fp8")
    got = pool.forward(x, ids, wts, path="gemm", out_dtype=torch.float32)
    ref = _restricted(W, x, ids, wts, {1, 4, 7, 10, 13, 16})
    np.testing.assert_array_equal(got.cpu().numpy(), ref.cpu().numpy())
    check_close(got.cpu().numpy(), _oracle(F.FMT_FP8, d, x, ids, wts, E, NS, H, I,
                                           keep={1, 4, 7, 10, 13, 16}),
                bf16_out=False, what="pool before swaps")
    # swap expert 7 out and 20 in (slot 2), then 11 into the freed slot of 16;
    # `gp` first, as the reference's adapter calls it
    assert pool.swap_out(2) == 7 and int(pool.slotmap[7]) == 7
    assert pool.swap_in(GP, 20, 2) == 2 and int(pool.slotmap[20]) == E + 2
    assert pool.swap_in(GP, 20, 3) is None   # already resident
    pool.swap_out(5)
    pool.swap_in(GP, 11, 5)
    got = pool.forward(x, ids, wts, path="gemm", out_dtype=torch.float32)
    ref = _restricted(W, x, ids, wts, {1, 4, 20, 10, 13, 11})
    np.testing.assert_array_equal(got.cpu().numpy(), ref.cpu().numpy())
    check_close(got.cpu().numpy(), _oracle(F.FMT_FP8, d, x, ids, wts, E, NS, H, I,
                                           keep={1, 4, 20, 10, 13, 11}),
                bf16_out=False, what="pool after swaps")
    assert pool.swaps_in == 2 and pool.swaps_out == 2


def test_pool_routing_counts_and_adaptation(monkeypatch):
    E, NS, H, I, K = 16, 0, 256, 128, 2
    d, W = _layer(F.FMT_MXFP4, E, NS, H, I, seed=8)
    store = HostExpertStore.from_weights(W)
    pool = LayerPool(store, DEV, H, I, 32, E, [0, 1, 2, 3], 0)
    hot = torch.tensor([[9, 12]] * 30 + [[0, 9]] * 5, dtype=torch.int32, device=DEV)
    pool.note_routing(hot)
    pool.note_routing(torch.tensor([[-1, 99]], dtype=torch.int32, device=DEV))   # ignored ids
    counts = pool._hits.cpu().tolist()
    assert counts[9] == 35 and counts[12] == 30 and counts[0] == 5 and sum(counts) == 70
    monkeypatch.setenv("XTU_PIN_WINDOW", "2")
    monkeypatch.setenv("XTU_PIN_MAXSWAP", "2")
    assert pool.maybe_adapt(GP) == 0                  # staging may be active: no-op
    n = pool.maybe_adapt(GP, staging_active=False)    # the reference's call form
    assert n == 2 and pool.expert_of == [0, 9, 12, 3]
    x, ids, wts = _inputs(20, K, E, H, seed=9)
    got = pool.forward(x, ids, wts, path="gemm", out_dtype=torch.float32)
    res = set(e for e in pool.expert_of if e >= 0)
    ref = _restricted(W, x, ids, wts, res)
    np.testing.assert_array_equal(got.cpu().numpy(), ref.cpu().numpy())
    check_close(got.cpu().numpy(), _oracle(F.FMT_MXFP4, d, x, ids, wts, E, NS, H, I, keep=res),
                bf16_out=False, what="pool after adaptation")


def test_engine_forward_many_matches_oracle():
    E, H, I, T, K = 8, 512, 256, 37, 2
    fmt = F.FMT_FP8
    d = make_dense_layer(fmt, E, H, I, seed=12)
    cfg = MOEConfigV2(expert_num=E, top_k=K, hidden_size=H, intermediate_size=I, groupN=128,
                      groupK=128, activation_type=1, swiglu_limit=7.0)
    eng = MOE_FP8(cfg, d["w13"], d["w2"], d["s13"], d["s2"], device=DEV)
    ids, wts = random_routing(T, K, E, seed=13)
    ids[0, 0] = E + 3   # out of range: ignored, as the engine does
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    out = torch.zeros((T, H), dtype=torch.float32, device=DEV)
    eng.cpu_prefill(T, K, torch.from_numpy(ids.astype(np.int32)).to(DEV),
                    torch.from_numpy(wts).to(DEV), x.to(DEV), out)
    torch.cuda.synchronize()
    ref = oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x), ids, wts, E, 0, H, I,
                       limit=7.0)
    check_close(out.cpu().numpy(), ref, bf16_out=False, what="engine fp8")
    g = eng.shard_geometry()
    assert g["w13_node_bytes"] == g["ns"] * 0 + E * 2 * g["w13_cbytes"]
    assert g["w13_cbytes"] * g["ns"] == I * H and eng.pin_hostbufs() == 2 * g["ns"] + 2
    with pytest.raises(ValueError):
        MOE_MXFP4(MOEConfigV2(expert_num=E, top_k=K, hidden_size=H, intermediate_size=I,
                              groupN=128, groupK=128), d["w13"], d["w2"], device=DEV)


def _hook_layer(fmt, E, H, I, seed):
    d = make_dense_layer(fmt, E, H, I, seed=seed)
    lay = types.SimpleNamespace(w13_weight=d["w13"], w2_weight=d["w2"], top_k=8,
                                use_grouped_topk=True, renormalize=True, scoring_func="sigmoid",
                                num_expert_group=8, topk_group=4, routed_scaling_factor=2.5,
                                e_score_correction_bias=torch.randn(E, generator=torch.Generator().manual_seed(1)) * 0.05,
                                swiglu_limit=None)
    if fmt == F.FMT_MXFP4:
        lay.w13_weight_scale, lay.w2_weight_scale = d["s13"], d["s2"]
    else:
        lay.w13_weight_scale_inv, lay.w2_weight_scale_inv = d["s13"], d["s2"]
    return d, lay


@pytest.mark.parametrize("cls,fmt", [(XiaotuExpertsMxfp4, F.FMT_MXFP4), (XiaotuExpertsFp8, F.FMT_FP8)])
def test_hook_monolithic_and_modular_paths(cls, fmt):
    E, H, I, T = 64, 512, 256, 12
    d, lay = _hook_layer(fmt, E, H, I, seed=21)
    hook = cls()
    hook.process_weights_after_loading(lay)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(DEV)
    logits = torch.randn((T, E), generator=torch.Generator().manual_seed(4)).to(DEV)
    out = hook.apply(x, None, None, router_logits=logits)
    w, i = route(logits, top_k=8, scoring="sigmoid", n_group=8, topk_group=4,
                 routed_scaling_factor=2.5, bias=lay.e_score_correction_bias.to(DEV))
    W = ExpertWeights.from_dense(fmt, d["w13"], d["s13"], d["w2"], d["s2"], device=DEV)
    ref = moe_forward(x, i, w, W, out_dtype=torch.float32).to(torch.bfloat16)
    np.testing.assert_array_equal(out.view(torch.int16).cpu().numpy(), ref.view(torch.int16).cpu().numpy())
    # modular path with an output buffer
    buf = torch.empty_like(x)
    res = hook.apply(x, None, None, topk_weights=w, topk_ids=i, output=buf)
    assert res is buf
    np.testing.assert_array_equal(buf.view(torch.int16).cpu().numpy(), ref.view(torch.int16).cpu().numpy())
    with pytest.raises(NotImplementedError):
        hook.apply(x, None, None, router_logits=logits, apply_router_weight_on_input=True)
    assert hook._supports_activation("silu") and not hook._supports_activation("gelu")


def test_hook_expert_map_zeroes_remote_experts():
    E, H, I, T = 64, 512, 256, 6
    d, lay = _hook_layer(F.FMT_MXFP4, E, H, I, seed=22)
    hook = XiaotuExpertsMxfp4()
    hook.process_weights_after_loading(lay)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(DEV)
    logits = torch.randn((T, E), generator=torch.Generator().manual_seed(6)).to(DEV)
    em = torch.arange(E, dtype=torch.int32)
    em[::2] = -1   # even experts live on another rank
    out = hook.apply(x, None, None, router_logits=logits, expert_map=em.to(DEV))
    w, i = route(logits, top_k=8, scoring="sigmoid", n_group=8, topk_group=4,
                 routed_scaling_factor=2.5, bias=lay.e_score_correction_bias.to(DEV))
    w = torch.where(i % 2 == 0, torch.zeros_like(w), w)
    W = ExpertWeights.from_dense(F.FMT_MXFP4, d["w13"], d["s13"], d["w2"], d["s2"], device=DEV)
    ref = moe_forward(x, i, w, W, out_dtype=torch.float32).to(torch.bfloat16)
    np.testing.assert_array_equal(out.view(torch.int16).cpu().numpy(), ref.view(torch.int16).cpu().numpy())


def test_layer_entries_match_oracle():
    E, H, I, T, K = 8, 512, 256, 20, 2
    ids, wts = random_routing(T, K, E, seed=31)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(8)).to(torch.bfloat16)
    xb = bf16_tensor_to_bits(x)
    ti, tw = torch.from_numpy(ids).to(DEV), torch.from_numpy(wts).to(DEV)
    # fp4 checkpoint planes on the host (MXFP4) -> gpu_moe_layer
    d = make_dense_layer(F.FMT_MXFP4, E, H, I, seed=32)
    out = GP.gpu_moe_layer(x.to(DEV), ti, tw, d["w13"], d["s13"], d["w2"], d["s2"], H, I, K,
                           device=DEV, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = oracle_layer(F.FMT_MXFP4, dense_to_numpy(F.FMT_MXFP4, d), xb, ids, wts, E, 0, H, I)
    check_close(out.cpu().numpy(), ref, bf16_out=False, what="gpu_moe_layer")
    # FP8 K-major planes -> gpu_moe_layer_fp8 / gpu_moe_decode_fp8
    d8 = make_dense_layer(F.FMT_FP8, E, H, I, seed=33)
    km = lambda t: t.transpose(1, 2).contiguous().to(DEV)
    ref8 = oracle_layer(F.FMT_FP8, dense_to_numpy(F.FMT_FP8, d8), xb, ids, wts, E, 0, H, I)
    o8 = GP.gpu_moe_layer_fp8(x.to(DEV), ti, tw, km(d8["w13"]), km(d8["s13"]), km(d8["w2"]),
                              km(d8["s2"]), H, I, K, device=DEV)
    check_close(o8.cpu().numpy(), ref8, bf16_out=False, what="gpu_moe_layer_fp8")
    o8d = GP.gpu_moe_decode_fp8(x[:4].to(DEV), ti[:4], tw[:4], km(d8["w13"]), km(d8["s13"]),
                                km(d8["w2"]), km(d8["s2"]), H, I, K, device=DEV)
    check_close(o8d.cpu().numpy(), ref8[:4], bf16_out=False, what="gpu_moe_decode_fp8")
    # small-M fp4 entry: within its envelope it matches, outside it declines
    bufs = tuple(km(t) for t in (d["w13"], d["s13"], d["w2"], d["s2"]))
    o4 = GP.moe_layer(bufs, x[:3].to(DEV), ti[:3], tw[:3], H, I, out_dtype=torch.float32)
    check_close(o4.cpu().numpy(), ref[:3], bf16_out=False, what="moe4 moe_layer")
    assert GP.moe_layer(bufs, x.to(DEV), ti, tw, H, I) is None
