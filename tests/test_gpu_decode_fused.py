"""Decode down projection with the weighted combine fused (xtu_decode_down_combine)
against the dequantized-fp32 oracle and against the separate down + combine
kernels, all four weight formats, plus the cases the fused form treats on its
own: a token listing an expert twice, zero weights kept or dropped, invalid
ids, every pair dropped, a weight-slot map, bf16 output, and token order."""
import numpy as np
import pytest
import torch

from helpers import (bf16_tensor_to_bits, check_close, dense_to_numpy, make_dense_layer,
                     oracle_layer, random_routing)
from xtu_moe_amd import formats as F
from xtu_moe_amd import layer as L
from xtu_moe_amd.layer import ExpertWeights, moe_forward

pytestmark = pytest.mark.gpu

FMTS = [F.FMT_MXFP4, F.FMT_NVFP4, F.FMT_FP8, F.FMT_BF16]


def _layer(fmt, E, NS, H, I, seed):
    d = make_dense_layer(fmt, E + NS, H, I, seed=seed)
    W = ExpertWeights.from_dense(fmt, d["w13"], d["s13"], d["w2"], d["s2"], d["gs13"], d["gs2"],
                                 n_shared=NS, device="cuda")
    return d, W


def _run(x, ids, wts, W, monkeypatch, fused, **kw):
    monkeypatch.setenv(L.FUSED_DOWN_ENV, "1" if fused else "0")
    out = moe_forward(x.cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(wts).cuda(), W,
                      path="decode", **kw)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("T,H,I", [(1, 512, 512), (2, 256, 1024), (4, 512, 256), (16, 512, 256)])
def test_fused_vs_oracle_and_unfused(fmt, T, H, I, monkeypatch):
    E, NS, K = 16, 1, 4
    d, W = _layer(fmt, E, NS, H, I, seed=T + I)
    ids, wts = random_routing(T, K, E, seed=T)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(T)).to(torch.bfloat16)
    A = T * (K + NS)
    assert L.decode_fused_down_ok(fmt, T, A, H, I, min(E, T * K) + NS, E + NS)
    fused = _run(x, ids, wts, W, monkeypatch, True, out_dtype=torch.float32)
    split = _run(x, ids, wts, W, monkeypatch, False, out_dtype=torch.float32)
    ref = oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x), ids, wts, E, NS, H, I)
    check_close(fused.cpu().numpy(), ref, bf16_out=False, what=f"fused fmt={fmt} T={T}")
    check_close(split.cpu().numpy(), ref, bf16_out=False, what=f"split fmt={fmt} T={T}")
    # same products, summed in another order (the fused down, in its own
    # launch or after the one-launch layer's barrier, splits K differently):
    # fp32 rounding, within 1e-4 of the output's scale
    scale = float(np.abs(ref).max()) + 1e-6
    assert float((fused - split).abs().max()) <= 1e-4 * scale


@pytest.mark.parametrize("drop_zero", [True, False])
def test_fused_duplicates_zero_weights_invalid_ids(drop_zero, monkeypatch):
    fmt, E, NS, H, I, T, K = F.FMT_MXFP4, 12, 1, 256, 512, 6, 4
    d, W = _layer(fmt, E, NS, H, I, seed=21)
    ids, wts = random_routing(T, K, E, seed=22)
    ids[0, 1] = ids[0, 0]            # token 0 lists one expert twice
    ids[1, 2] = ids[1, 3] = ids[1, 0]
    wts[2, 1] = 0.0                  # zero weights, kept or dropped
    wts[3, :] = 0.0
    ids[4, 0], ids[4, 2] = -1, E + 2  # invalid ids go to the trash bucket
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(23)).to(torch.bfloat16)
    out = _run(x, ids, wts, W, monkeypatch, True, out_dtype=torch.float32, drop_zero=drop_zero)
    split = _run(x, ids, wts, W, monkeypatch, False, out_dtype=torch.float32,
                 drop_zero=drop_zero)
    ref = oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x), ids, wts, E, NS, H, I)
    check_close(out.cpu().numpy(), ref, bf16_out=False, what=f"dup/zero drop_zero={drop_zero}")
    scale = float(np.abs(ref).max()) + 1e-6
    assert float((out - split).abs().max()) <= 1e-4 * scale


def test_fused_every_pair_dropped_writes_zero_rows(monkeypatch):
    fmt, E, NS, H, I, T, K = F.FMT_NVFP4, 8, 0, 256, 256, 3, 2
    _, W = _layer(fmt, E, NS, H, I, seed=31)
    ids = np.full((T, K), -1, np.int32)
    wts = np.ones((T, K), np.float32)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(32)).to(torch.bfloat16)
    for dt in (torch.float32, torch.bfloat16):
        out = torch.full((T, H), float("nan"), dtype=dt, device="cuda")
        _run(x, ids, wts, W, monkeypatch, True, out=out)
        assert torch.equal(out.float(), torch.zeros((T, H), device="cuda"))


def test_fused_slot_map_and_bf16_out(monkeypatch):
    fmt, E, NS, H, I, T, K = F.FMT_FP8, 16, 1, 512, 512, 3, 4
    d, _ = _layer(fmt, E, NS, H, I, seed=41)
    # store the experts in reverse order; slot_map[b] = where bucket b's weights live
    order = np.arange(E + NS)[::-1].copy()
    idx = torch.from_numpy(order)
    rev = {k: (v[idx].contiguous() if v is not None else None) for k, v in d.items()}
    W = ExpertWeights.from_dense(fmt, rev["w13"], rev["s13"], rev["w2"], rev["s2"], rev["gs13"],
                                 rev["gs2"], n_shared=NS, device="cuda")
    slot_map = torch.from_numpy(np.argsort(order).astype(np.int32)).cuda()
    ids, wts = random_routing(T, K, E, seed=42)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(43)).to(torch.bfloat16)
    out = _run(x, ids, wts, W, monkeypatch, True, out_dtype=torch.bfloat16, slot_map=slot_map)
    ref = oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x), ids, wts, E, NS, H, I)
    check_close(out.float().cpu().numpy(), ref, bf16_out=True, what="slot map, bf16 out")


def test_fused_token_permutation_is_bitwise(monkeypatch):
    fmt, E, NS, H, I, T, K = F.FMT_MXFP4, 32, 1, 512, 1024, 8, 4
    _, W = _layer(fmt, E, NS, H, I, seed=51)
    ids, wts = random_routing(T, K, E, seed=52)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(53)).to(torch.bfloat16)
    out = _run(x, ids, wts, W, monkeypatch, True, out_dtype=torch.float32)
    perm = np.random.default_rng(54).permutation(T)
    out_p = _run(x[perm], ids[perm].copy(), wts[perm].copy(), W, monkeypatch, True,
                 out_dtype=torch.float32)
    assert torch.equal(out_p, out[torch.from_numpy(perm).cuda()])


def test_fused_ds_v3_mxfp4_t2(monkeypatch):
    """DeepSeek-V3 shape (H=7168, I=2048, top-8 + 1 shared) at T=2, where the
    18 act rows still fit the stage; experts compacted to those routed."""
    H, I, E, K, T = 7168, 2048, 256, 8, 2
    rng = np.random.default_rng(61)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    wts = (rng.random((T, K)) * 0.3 + 0.05).astype(np.float32)
    used = np.unique(ids)
    cids = np.vectorize({int(e): i for i, e in enumerate(used)}.get)(ids).astype(np.int32)
    U = len(used)
    d, W = _layer(F.FMT_MXFP4, U, 1, H, I, seed=62)
    assert L.decode_fused_down_ok(F.FMT_MXFP4, T, T * (K + 1), H, I, min(E, T * K) + 1, U + 1)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(63)).to(torch.bfloat16)
    # the shared expert beside the router: its act rows staged from act_sh,
    # only the 16 routed sorted rows from act (the stage then fits)
    assert L.decode_fused_down_ok(F.FMT_MXFP4, T, T * (K + 1), H, I, min(E, T * K) + 1, U + 1,
                                  T)
    assert L._route_shared_ok(F.FMT_MXFP4, 2, T, U, K, None, H, I, 1)
    out = _run(x, cids, wts, W, monkeypatch, True, out_dtype=torch.float32)
    ref = oracle_layer(F.FMT_MXFP4, dense_to_numpy(F.FMT_MXFP4, d), bf16_tensor_to_bits(x), cids,
                       wts, U, 1, H, I)
    check_close(out.cpu().numpy(), ref, bf16_out=False, what="ds-v3 fused T=2")
    monkeypatch.setenv(L.SHARED_SPLIT_ENV, "0")
    out0 = _run(x, cids, wts, W, monkeypatch, True, out_dtype=torch.float32)
    assert torch.equal(out, out0), "shared expert beside the router vs with the routed ones"



@pytest.mark.parametrize("fmt", [F.FMT_MXFP4, F.FMT_NVFP4])
@pytest.mark.parametrize("T,H", [(1, 2048), (3, 2048), (5, 4096), (2, 7168)])
def test_decode_hidden_sizes_and_single_expert(fmt, T, H, monkeypatch):
    """Decode layers at hidden sizes 2048 / 4096 / 7168 (16, 32 and 56 units
    of 128 k per gate/up row) against the oracle, and a batch whose tokens all
    route to one expert with no shared expert (most work items idle)."""
    E, NS, I, K = 24, 1, 256, 4
    d, W = _layer(fmt, E, NS, H, I, seed=T + H)
    ids, wts = random_routing(T, K, E, seed=T + 1)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(T + 2)).to(torch.bfloat16)
    out = _run(x, ids, wts, W, monkeypatch, True, out_dtype=torch.float32)
    ref = oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x), ids, wts, E, NS, H, I)
    check_close(out.cpu().numpy(), ref, bf16_out=False, what=f"decode fmt={fmt} T={T} H={H}")
    # a single routed expert for every token and no shared expert
    _, W1 = _layer(fmt, E, 0, H, I, seed=T + H + 1)
    ids1 = np.full((T, 1), 5, np.int32)
    wts1 = np.ones((T, 1), np.float32)
    out1 = _run(x, ids1, wts1, W1, monkeypatch, True, out_dtype=torch.float32)
    d1 = make_dense_layer(fmt, E, H, I, seed=T + H + 1)
    ref1 = oracle_layer(fmt, dense_to_numpy(fmt, d1), bf16_tensor_to_bits(x), ids1, wts1, E, 0, H,
                        I)
    check_close(out1.cpu().numpy(), ref1, bf16_out=False, what=f"single expert T={T}")


# ---------------------------------------------------------------------------
# shared experts' gate/up inside the routing launch (xtu_decode_route_shared)

_SEG_FIELDS = ("sorted_pair", "sorted_tok", "sorted_wts", "inv", "seg_start", "active",
               "n_active", "tile_expert", "tile_row0", "n_tiles", "expert_tile_start")


def _seg_state(seg):
    n_act = int(seg.n_active.item())
    n_til = int(seg.n_tiles.item())
    out = {}
    for f in _SEG_FIELDS:
        t = getattr(seg, f)
        if f in ("sorted_pair", "sorted_tok", "sorted_wts", "inv"):
            t = t[:seg.A]
        elif f == "active":
            t = t[:n_act]
        elif f in ("tile_expert", "tile_row0"):
            t = t[:n_til]
        out[f] = t.clone()
    return out


def _split_run(monkeypatch, split, x, W, K, router=None, ids=None, wts=None, **kw):
    monkeypatch.setenv(L.SHARED_SPLIT_ENV, "1" if split else "0")
    monkeypatch.setenv(L.FUSED_DOWN_ENV, "1")
    T = x.shape[0]
    if router is not None:
        ids = torch.full((T, K), -7, dtype=torch.int32, device="cuda")
        wts = torch.full((T, K), float("nan"), dtype=torch.float32, device="cuda")
    for t in L._BUF_CACHE.values():   # unwritten rows would show up as NaN
        if t.is_floating_point():
            t.fill_(float("nan"))
    out, seg = moe_forward(x, ids, wts, W, path="decode", router=router, return_seg=True,
                           out_dtype=torch.float32, **kw)
    torch.cuda.synchronize()
    return out, ids.clone(), wts.clone(), _seg_state(seg)


def _same(a, b, what):
    oa, ia, wa, sa = a
    ob, ib, wb, sb = b
    assert torch.equal(ia, ib), f"{what}: ids"
    assert torch.equal(wa.view(torch.int32), wb.view(torch.int32)), f"{what}: weights"
    for f in _SEG_FIELDS:
        ta, tb = sa[f], sb[f]
        if ta.dtype == torch.float32:
            ta, tb = ta.view(torch.int32), tb.view(torch.int32)
        assert torch.equal(ta, tb), f"{what}: {f}"
    assert torch.equal(oa, ob), f"{what}: output"


@pytest.mark.parametrize("T,H", [(1, 512), (2, 512), (4, 4096)])
def test_shared_split_grouped_sigmoid(T, H, monkeypatch):
    # one routing wave per token: H = 512 gives 2-wave workgroups, 4096 four
    fmt, E, NS, I, K = F.FMT_MXFP4, 256, 1, 256, 8
    d, W = _layer(fmt, E, NS, H, I, seed=70 + T)
    g = torch.Generator(device="cuda").manual_seed(71 + T)
    logits = torch.randn((T, E), generator=g, device="cuda")
    bias = torch.randn((E,), generator=g, device="cuda") * 0.1
    x = torch.randn((T, H), generator=g, device="cuda").to(torch.bfloat16)
    router = dict(logits=logits, scoring="sigmoid", bias=bias, n_group=8, topk_group=4,
                  routed_scaling_factor=2.5, renormalize=True)
    assert L._route_shared_ok(fmt, 1, T, E, K, router, H, I, NS)
    a = _split_run(monkeypatch, True, x, W, K, router=router)
    b = _split_run(monkeypatch, False, x, W, K, router=router)
    _same(a, b, f"grouped sigmoid T={T}")
    out, ids, wts, _ = a
    ref = oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x), ids.cpu().numpy(),
                       wts.cpu().numpy(), E, NS, H, I)
    check_close(out.cpu().numpy(), ref, bf16_out=False, what=f"split T={T} vs oracle")


@pytest.mark.parametrize("T", [1, 2])
def test_shared_split_softmax_512(T, monkeypatch):
    fmt, E, NS, H, I, K = F.FMT_NVFP4, 512, 1, 512, 256, 10
    _, W = _layer(fmt, E, NS, H, I, seed=80 + T)
    g = torch.Generator(device="cuda").manual_seed(81 + T)
    logits = torch.randn((T, E), generator=g, device="cuda")
    x = torch.randn((T, H), generator=g, device="cuda").to(torch.bfloat16)
    router = dict(logits=logits, scoring="softmax", renormalize=True)
    assert L._route_shared_ok(fmt, 0, T, E, K, router, H, I, NS)
    _same(_split_run(monkeypatch, True, x, W, K, router=router),
          _split_run(monkeypatch, False, x, W, K, router=router), f"softmax T={T}")


@pytest.mark.parametrize("drop_zero", [True, False])
def test_shared_split_given_ids_two_shared(drop_zero, monkeypatch):
    fmt, E, NS, H, I, T, K = F.FMT_FP8, 16, 2, 512, 256, 2, 4
    d, _ = _layer(fmt, E, NS, H, I, seed=91)
    # experts stored in reverse order behind a slot map, ids through an id map
    order = np.arange(E + NS)[::-1].copy()
    idx = torch.from_numpy(order)
    rev = {k: (v[idx].contiguous() if v is not None else None) for k, v in d.items()}
    W = ExpertWeights.from_dense(fmt, rev["w13"], rev["s13"], rev["w2"], rev["s2"], rev["gs13"],
                                 rev["gs2"], n_shared=NS, device="cuda")
    slot_map = torch.from_numpy(np.argsort(order).astype(np.int32)).cuda()
    ids_np, wts_np = random_routing(T, K, E, seed=92)
    ids_np[0, 1] = -1
    ids_np[1, 2] = ids_np[1, 0]
    wts_np[1, 3] = 0.0
    ids = torch.from_numpy(ids_np).cuda()
    wts = torch.from_numpy(wts_np).cuda()
    id_map = torch.from_numpy(np.roll(np.arange(E), 3).astype(np.int32)).cuda()
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(93)).to(torch.bfloat16).cuda()
    assert L._route_shared_ok(fmt, 2, T, E, K, None, H, I, NS)
    kw = dict(ids=ids, wts=wts, drop_zero=drop_zero, id_map=id_map, slot_map=slot_map)
    a = _split_run(monkeypatch, True, x, W, K, **kw)
    _same(a, _split_run(monkeypatch, False, x, W, K, **kw), f"given ids drop_zero={drop_zero}")
    mapped = np.where((ids_np >= 0) & (ids_np < E), np.roll(np.arange(E), 3)[ids_np % E], -1)
    ref = oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x.cpu()),
                       mapped.astype(np.int32), wts_np, E, NS, H, I)
    check_close(a[0].cpu().numpy(), ref, bf16_out=False, what="split given ids vs oracle")


def test_shared_split_misaligned_logits_fall_back(monkeypatch):
    fmt, E, NS, H, I, T, K = F.FMT_MXFP4, 256, 1, 512, 256, 1, 8
    _, W = _layer(fmt, E, NS, H, I, seed=95)
    base = torch.randn((T * E + 1,), device="cuda")
    logits = base[1:].view(T, E)          # 4-byte offset: not 16-byte aligned
    router = dict(logits=logits, scoring="sigmoid", n_group=8, topk_group=4,
                  routed_scaling_factor=2.5)
    assert not L._route_shared_ok(fmt, 1, T, E, K, router, H, I, NS)
    x = torch.randn((T, H), device="cuda").to(torch.bfloat16)
    _same(_split_run(monkeypatch, True, x, W, K, router=router),
          _split_run(monkeypatch, False, x, W, K, router=router), "misaligned logits")


# ---------------------------------------------------------------------------
# routing, segmentation and gate/up in one launch (xtu_decode_route_gate_up)

def _fr_run(monkeypatch, fused_route, split, x, W, K, one=False, **kw):
    monkeypatch.setenv(L.FUSED_ROUTE_ENV, "1" if fused_route else "0")
    monkeypatch.setenv(L.ONE_LAUNCH_ENV, "1" if one else "0")
    return _split_run(monkeypatch, split, x, W, K, **kw)


@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("fmt,T,H", [(F.FMT_MXFP4, 1, 512), (F.FMT_MXFP4, 2, 512),
                                     (F.FMT_MXFP4, 4, 512), (F.FMT_MXFP4, 4, 4096),
                                     (F.FMT_FP8, 7, 4096)])
def test_fused_route_grouped_sigmoid(fmt, T, H, split, monkeypatch):
    """Every gate/up workgroup routes the batch itself: routing outputs,
    segmentation and the layer output are bitwise those of the separate
    routing launch, with the shared expert split off or as a sorted bucket;
    at H = 512 two waves route four tokens."""
    E, NS, I, K = 256, 1, 256, 8
    d, W = _layer(fmt, E, NS, H, I, seed=170 + T)
    g = torch.Generator(device="cuda").manual_seed(171 + T)
    logits = torch.randn((T, E), generator=g, device="cuda")
    bias = torch.randn((E,), generator=g, device="cuda") * 0.1
    x = torch.randn((T, H), generator=g, device="cuda").to(torch.bfloat16)
    router = dict(logits=logits, scoring="sigmoid", bias=bias, n_group=8, topk_group=4,
                  routed_scaling_factor=2.5, renormalize=True)
    assert L._route_gate_up_ok(fmt, 1, T, E, K, router, H, I, NS)
    a = _fr_run(monkeypatch, True, split, x, W, K, router=router)
    b = _fr_run(monkeypatch, False, split, x, W, K, router=router)
    _same(a, b, f"fused route T={T} split={split}")
    out, ids, wts, _ = a
    ref = oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x), ids.cpu().numpy(),
                       wts.cpu().numpy(), E, NS, H, I)
    check_close(out.cpu().numpy(), ref, bf16_out=False, what=f"fused route T={T} vs oracle")


@pytest.mark.parametrize("T", [1, 2])
def test_fused_route_softmax_512_no_shared(T, monkeypatch):
    fmt, E, NS, H, I, K = F.FMT_NVFP4, 512, 0, 512, 256, 10
    _, W = _layer(fmt, E, NS, H, I, seed=180 + T)
    g = torch.Generator(device="cuda").manual_seed(181 + T)
    logits = torch.randn((T, E), generator=g, device="cuda")
    x = torch.randn((T, H), generator=g, device="cuda").to(torch.bfloat16)
    router = dict(logits=logits, scoring="softmax", renormalize=True)
    assert L._route_gate_up_ok(fmt, 0, T, E, K, router, H, I, NS)
    _same(_fr_run(monkeypatch, True, False, x, W, K, router=router),
          _fr_run(monkeypatch, False, False, x, W, K, router=router), f"softmax 512 T={T}")


@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("drop_zero", [True, False])
def test_fused_route_given_ids_maps_two_shared(drop_zero, split, monkeypatch):
    """Given ids (no router) through an id map, experts behind a slot map,
    two shared experts, an invalid id, an expert listed twice, a zero
    weight: bitwise the separate launches, and the oracle."""
    fmt, E, NS, H, I, T, K = F.FMT_FP8, 16, 2, 2048, 256, 3, 4
    d, _ = _layer(fmt, E, NS, H, I, seed=191)
    order = np.arange(E + NS)[::-1].copy()
    idx = torch.from_numpy(order)
    rev = {k: (v[idx].contiguous() if v is not None else None) for k, v in d.items()}
    W = ExpertWeights.from_dense(fmt, rev["w13"], rev["s13"], rev["w2"], rev["s2"], rev["gs13"],
                                 rev["gs2"], n_shared=NS, device="cuda")
    slot_map = torch.from_numpy(np.argsort(order).astype(np.int32)).cuda()
    ids_np, wts_np = random_routing(T, K, E, seed=192)
    ids_np[0, 1] = -1
    ids_np[1, 2] = ids_np[1, 0]
    wts_np[2, 3] = 0.0
    ids = torch.from_numpy(ids_np).cuda()
    wts = torch.from_numpy(wts_np).cuda()
    id_map = torch.from_numpy(np.roll(np.arange(E), 5).astype(np.int32)).cuda()
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(193)).to(torch.bfloat16).cuda()
    assert L._route_gate_up_ok(fmt, 2, T, E, K, None, H, I, NS)
    kw = dict(ids=ids, wts=wts, drop_zero=drop_zero, id_map=id_map, slot_map=slot_map)
    a = _fr_run(monkeypatch, True, split, x, W, K, **kw)
    _same(a, _fr_run(monkeypatch, False, split, x, W, K, **kw),
          f"given ids drop_zero={drop_zero} split={split}")
    mapped = np.where((ids_np >= 0) & (ids_np < E), np.roll(np.arange(E), 5)[ids_np % E], -1)
    ref = oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x.cpu()),
                       mapped.astype(np.int32), wts_np, E, NS, H, I)
    check_close(a[0].cpu().numpy(), ref, bf16_out=False, what="fused route given ids vs oracle")


def test_fused_route_every_pair_invalid(monkeypatch):
    """No live pair: the routed workgroups find no tile and exit; the shared
    expert alone makes the output."""
    fmt, E, NS, H, I, T, K = F.FMT_MXFP4, 16, 1, 512, 256, 2, 4
    d, W = _layer(fmt, E, NS, H, I, seed=195)
    ids = torch.full((T, K), -1, dtype=torch.int32, device="cuda")
    wts = torch.ones((T, K), dtype=torch.float32, device="cuda")
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(196)).to(torch.bfloat16).cuda()
    for split in (True, False):
        a = _fr_run(monkeypatch, True, split, x, W, K, ids=ids, wts=wts)
        _same(a, _fr_run(monkeypatch, False, split, x, W, K, ids=ids, wts=wts),
              f"all invalid split={split}")
        ref = oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x.cpu()),
                           ids.cpu().numpy(), wts.cpu().numpy(), E, NS, H, I)
        check_close(a[0].cpu().numpy(), ref, bf16_out=False, what="all invalid vs oracle")


def test_fused_route_rejects_a_short_tile_grid():
    """xtu_decode_route_gate_up refuses a max_tiles below the batch's tile
    bound (a tile left without a work item would leave act rows unwritten),
    and an act_shared without shared experts, before launching anything."""
    from xtu_moe_amd import _lib
    from xtu_moe_amd.layer import _p, _stream
    fmt, E, NS, H, I, T, K = F.FMT_MXFP4, 16, 1, 512, 256, 2, 4
    _, W = _layer(fmt, E, NS, H, I, seed=197)
    dev = torch.device("cuda")
    seg = L.segmentation(T, K, E, NS, L.DECODE_TILE, dev)
    ids = torch.zeros((T, K), dtype=torch.int32, device=dev)
    wts = torch.ones((T, K), dtype=torch.float32, device=dev)
    x = torch.zeros((T, H), dtype=torch.bfloat16, device=dev)
    act = torch.empty((seg.A, I), dtype=torch.bfloat16, device=dev)
    act_sh = torch.empty((NS * T, I), dtype=torch.bfloat16, device=dev)

    def call(max_tiles, ns=NS, sh=act_sh):
        return _lib.load().xtu_decode_route_gate_up(
            2, None, None, _p(ids), _p(wts), T, E, K, 1, 1, 1.0, 1, None, ns, 1, seg.bm,
            _p(seg.sorted_pair), _p(seg.sorted_tok), _p(seg.sorted_wts), _p(seg.inv),
            _p(seg.seg_start), _p(seg.active), _p(seg.n_active), _p(seg.tile_expert),
            _p(seg.tile_row0), _p(seg.n_tiles), _p(seg.expert_tile_start), fmt, _p(x), H, I,
            _p(W.w13), _p(W.s13), _p(W.gs13), 0, 0, None, max_tiles, _p(act),
            _p(sh) if sh is not None else None, 0.0, 1.0, 0.0, _stream())

    # T (K + NS) = 10 pairs in at most min(E, 8) + 1 = 9 buckets: at least 9 tiles
    assert call(8) == 1                     # hipErrorInvalidValue
    assert call(0) == 1
    assert call(65) == 1
    assert call(9, ns=0) == 1               # act_shared with no shared experts
    assert call(9) == 0
    torch.cuda.synchronize()


# ---------------------------------------------------------------------------
# the whole decode layer in one launch (xtu_decode_layer): routing, gate/up,
# a barrier across the launch's workgroups, the down with the combine

def _barrier_clean():
    """Every counter back at zero, no wait ran out (the generations move)."""
    for t in L._BAR_CACHE.values():
        w = t.cpu().view(-1, 64)[:, 0].tolist()
        assert w[:9] == [0] * 9 and w[17] == 0, f"barrier words {w}"


def _near(a, b, what):
    """Routing and segmentation bitwise; the output the same products summed
    over another K split of the down (fp32 rounding: within 1e-4 of the
    output's scale, far inside the oracle bar each side is checked against)."""
    oa, ia, wa, sa = a
    ob, ib, wb, sb = b
    assert torch.equal(ia, ib), f"{what}: ids"
    assert torch.equal(wa.view(torch.int32), wb.view(torch.int32)), f"{what}: weights"
    for f in _SEG_FIELDS:
        ta, tb = sa[f], sb[f]
        if ta.dtype == torch.float32:
            ta, tb = ta.view(torch.int32), tb.view(torch.int32)
        assert torch.equal(ta, tb), f"{what}: {f}"
    scale = float(ob.abs().max()) + 1e-6
    assert float((oa - ob).abs().max()) <= 1e-4 * scale, f"{what}: output"


@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("fmt,T,H,I", [(F.FMT_MXFP4, 1, 512, 256), (F.FMT_MXFP4, 4, 4096, 256),
                                       (F.FMT_NVFP4, 2, 2048, 512), (F.FMT_FP8, 3, 1024, 256),
                                       (F.FMT_BF16, 2, 512, 512)])
def test_one_launch_layer_grouped_sigmoid(fmt, T, H, I, split, monkeypatch):
    E, NS, K = 256, 1, 8
    d, W = _layer(fmt, E, NS, H, I, seed=210 + T + H)
    g = torch.Generator(device="cuda").manual_seed(211 + T)
    logits = torch.randn((T, E), generator=g, device="cuda")
    bias = torch.randn((E,), generator=g, device="cuda") * 0.1
    x = torch.randn((T, H), generator=g, device="cuda").to(torch.bfloat16)
    router = dict(logits=logits, scoring="sigmoid", bias=bias, n_group=8, topk_group=4,
                  routed_scaling_factor=2.5, renormalize=True)
    assert L._layer_ok(fmt, 1, T, E, K, router, H, I, NS)
    a = _fr_run(monkeypatch, True, split, x, W, K, one=True, router=router)
    b = _fr_run(monkeypatch, True, split, x, W, K, one=False, router=router)
    _near(a, b, f"one launch fmt={fmt} T={T} split={split}")
    out, ids, wts, _ = a
    ref = oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x), ids.cpu().numpy(),
                       wts.cpu().numpy(), E, NS, H, I)
    check_close(out.cpu().numpy(), ref, bf16_out=False, what=f"one launch T={T} vs oracle")
    _barrier_clean()


@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("drop_zero", [True, False])
def test_one_launch_given_ids_maps_two_shared(drop_zero, split, monkeypatch):
    """Given ids through an id map, experts behind a slot map, two shared
    experts, an invalid id, an expert listed twice, a zero weight."""
    fmt, E, NS, H, I, T, K = F.FMT_FP8, 16, 2, 2048, 256, 3, 4
    d, _ = _layer(fmt, E, NS, H, I, seed=221)
    order = np.arange(E + NS)[::-1].copy()
    idx = torch.from_numpy(order)
    rev = {k: (v[idx].contiguous() if v is not None else None) for k, v in d.items()}
    W = ExpertWeights.from_dense(fmt, rev["w13"], rev["s13"], rev["w2"], rev["s2"], rev["gs13"],
                                 rev["gs2"], n_shared=NS, device="cuda")
    slot_map = torch.from_numpy(np.argsort(order).astype(np.int32)).cuda()
    ids_np, wts_np = random_routing(T, K, E, seed=222)
    ids_np[0, 1] = -1
    ids_np[1, 2] = ids_np[1, 0]
    wts_np[2, 3] = 0.0
    ids = torch.from_numpy(ids_np).cuda()
    wts = torch.from_numpy(wts_np).cuda()
    id_map = torch.from_numpy(np.roll(np.arange(E), 5).astype(np.int32)).cuda()
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(223)).to(torch.bfloat16).cuda()
    assert L._layer_ok(fmt, 2, T, E, K, None, H, I, NS)
    kw = dict(ids=ids, wts=wts, drop_zero=drop_zero, id_map=id_map, slot_map=slot_map)
    a = _fr_run(monkeypatch, True, split, x, W, K, one=True, **kw)
    _near(a, _fr_run(monkeypatch, True, split, x, W, K, one=False, **kw),
          f"given ids drop_zero={drop_zero} split={split}")
    mapped = np.where((ids_np >= 0) & (ids_np < E), np.roll(np.arange(E), 5)[ids_np % E], -1)
    ref = oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x.cpu()),
                       mapped.astype(np.int32), wts_np, E, NS, H, I)
    check_close(a[0].cpu().numpy(), ref, bf16_out=False, what="one launch given ids vs oracle")
    _barrier_clean()


def test_one_launch_every_pair_invalid(monkeypatch):
    """No live routed pair: the shared expert alone makes the output (split or
    as a sorted bucket); with no shared expert either, every row is zero."""
    fmt, E, NS, H, I, T, K = F.FMT_MXFP4, 16, 1, 512, 256, 2, 4
    d, W = _layer(fmt, E, NS, H, I, seed=225)
    ids = torch.full((T, K), -1, dtype=torch.int32, device="cuda")
    wts = torch.ones((T, K), dtype=torch.float32, device="cuda")
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(226)).to(torch.bfloat16).cuda()
    assert L._layer_ok(fmt, 2, T, E, K, None, H, I, NS)
    for split in (True, False):
        a = _fr_run(monkeypatch, True, split, x, W, K, one=True, ids=ids, wts=wts)
        _near(a, _fr_run(monkeypatch, True, split, x, W, K, one=False, ids=ids, wts=wts),
              f"all invalid split={split}")
        ref = oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x.cpu()),
                           ids.cpu().numpy(), wts.cpu().numpy(), E, NS, H, I)
        check_close(a[0].cpu().numpy(), ref, bf16_out=False, what="all invalid vs oracle")
    _, W0 = _layer(fmt, E, 0, H, I, seed=227)
    monkeypatch.setenv(L.FUSED_ROUTE_ENV, "1")
    monkeypatch.setenv(L.ONE_LAUNCH_ENV, "1")
    monkeypatch.setenv(L.FUSED_DOWN_ENV, "1")
    for dt in (torch.float32, torch.bfloat16):
        out = torch.full((T, H), float("nan"), dtype=dt, device="cuda")
        moe_forward(x, ids, wts, W0, path="decode", out=out)
        torch.cuda.synchronize()
        assert torch.equal(out.float(), torch.zeros((T, H), device="cuda"))
    _barrier_clean()


def test_one_launch_ds_v3_shape(monkeypatch):
    """DeepSeek-V3 widths (H = 7168, I = 2048: eight-wave workgroups, the down
    split eight ways) at T = 1 and 2, experts compacted to those routed."""
    H, I, E, K = 7168, 2048, 256, 8
    rng = np.random.default_rng(231)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(2)]).astype(np.int32)
    wts = (rng.random((2, K)) * 0.3 + 0.05).astype(np.float32)
    used = np.unique(ids)
    cids = np.vectorize({int(e): i for i, e in enumerate(used)}.get)(ids).astype(np.int32)
    U = len(used)
    d, W = _layer(F.FMT_MXFP4, U, 1, H, I, seed=232)
    x = torch.randn((2, H), generator=torch.Generator().manual_seed(233)).to(torch.bfloat16).cuda()
    for T in (1, 2):
        monkeypatch.setenv(L.ONE_LAUNCH_ENV, "1")
        assert L._layer_ok(F.FMT_MXFP4, 2, T, U, K, None, H, I, 1)
        xi = x[:T].contiguous()
        it = torch.from_numpy(cids[:T].copy()).cuda()
        wt = torch.from_numpy(wts[:T].copy()).cuda()
        a = _fr_run(monkeypatch, True, True, xi, W, K, one=True, ids=it, wts=wt)
        _near(a, _fr_run(monkeypatch, True, True, xi, W, K, one=False, ids=it, wts=wt),
              f"ds-v3 one launch T={T}")
        ref = oracle_layer(F.FMT_MXFP4, dense_to_numpy(F.FMT_MXFP4, d),
                           bf16_tensor_to_bits(xi.cpu()), cids[:T], wts[:T], U, 1, H, I)
        check_close(a[0].cpu().numpy(), ref, bf16_out=False, what=f"ds-v3 one launch T={T}")
    _barrier_clean()


def test_one_launch_back_to_back_and_graph(monkeypatch):
    """Many launches in a row on one stream share the barrier words (each
    leaves them reset), across batch sizes, and inside a HIP graph replayed
    with eager calls between the replays: every result equals the first."""
    fmt, E, NS, H, I, K = F.FMT_MXFP4, 256, 1, 2048, 512, 8
    _, W = _layer(fmt, E, NS, H, I, seed=241)
    g = torch.Generator(device="cuda").manual_seed(242)
    monkeypatch.setenv(L.FUSED_ROUTE_ENV, "1")
    monkeypatch.setenv(L.ONE_LAUNCH_ENV, "1")
    monkeypatch.setenv(L.FUSED_DOWN_ENV, "1")
    outs = {}
    inputs = {}
    for T in (1, 4, 2):
        logits = torch.randn((T, E), generator=g, device="cuda")
        x = torch.randn((T, H), generator=g, device="cuda").to(torch.bfloat16)
        router = dict(logits=logits, scoring="sigmoid", n_group=8, topk_group=4,
                      routed_scaling_factor=2.5, renormalize=True)
        assert L._layer_ok(fmt, 1, T, E, K, router, H, I, NS)
        inputs[T] = (x, router)
    def run(T, out=None):
        x, router = inputs[T]
        ids = torch.empty((T, K), dtype=torch.int32, device="cuda")
        wts = torch.empty((T, K), dtype=torch.float32, device="cuda")
        return moe_forward(x, ids, wts, W, path="decode", router=router, out=out,
                           out_dtype=torch.float32)
    for T in inputs:
        outs[T] = run(T).clone()
    for _ in range(20):
        for T in (4, 1, 2):
            assert torch.equal(run(T), outs[T]), f"back-to-back T={T}"
    torch.cuda.synchronize()
    _barrier_clean()
    # graph: the layer at T = 4, replayed three times with eager calls between
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        gout = torch.empty((4, H), dtype=torch.float32, device="cuda")
        run(4, out=gout)                     # warm the stream's buffers
        s.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            run(4, out=gout)
    torch.cuda.current_stream().wait_stream(s)
    for i in range(3):
        gout.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout, outs[4]), f"graph replay {i}"
        assert torch.equal(run(1), outs[1]), f"eager between replays {i}"
        torch.cuda.synchronize()
    _barrier_clean()
    assert L.barrier_timeouts() == 0


def test_one_launch_layer_random_shapes(monkeypatch):
    """Seeded shapes across the one-launch layer's envelope (formats, T = 1..16,
    top-k, zero to two shared experts, hidden and intermediate sizes, split
    shared experts or not): routing and segmentation bitwise those of the
    separate launches, the output within their fp32 rounding and within the
    oracle's tolerance."""
    rng = np.random.default_rng(301)
    ran = 0
    for case in range(40):
        fmt = int(rng.choice([F.FMT_MXFP4, F.FMT_FP8, F.FMT_BF16, F.FMT_NVFP4]))
        T = int(rng.integers(1, 17))
        K = int(rng.integers(1, 9))
        NS = int(rng.integers(0, 3))
        if T * (K + NS) > 64:
            continue
        E = int(rng.choice([16, 24, 32]))
        H = int(rng.choice([512, 1024, 2048]))
        I = int(rng.choice([256, 512, 1024]))
        split = bool(rng.integers(0, 2)) and NS > 0
        monkeypatch.setenv(L.ONE_LAUNCH_ENV, "1")
        if not L._layer_ok(fmt, 2, T, E, K, None, H, I, NS):
            continue
        d, W = _layer(fmt, E, NS, H, I, seed=310 + case)
        ids_np, wts_np = random_routing(T, K, E, seed=320 + case)
        ids = torch.from_numpy(ids_np).cuda()
        wts = torch.from_numpy(wts_np).cuda()
        x = torch.randn((T, H), generator=torch.Generator().manual_seed(330 + case)).to(
            torch.bfloat16).cuda()
        what = f"case {case}: fmt={fmt} T={T} K={K} NS={NS} E={E} H={H} I={I} split={split}"
        a = _fr_run(monkeypatch, True, split, x, W, K, one=True, ids=ids, wts=wts)
        _near(a, _fr_run(monkeypatch, True, split, x, W, K, one=False, ids=ids, wts=wts), what)
        ref = oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x.cpu()), ids_np,
                           wts_np, E, NS, H, I)
        check_close(a[0].cpu().numpy(), ref, bf16_out=False, what=what)
        ran += 1
        if ran == 12:
            break
    assert ran >= 8, f"only {ran} shapes inside the envelope"
    _barrier_clean()
