"""Routing and segmentation on the GPU: bit-exact against the oracle.

Routing: ids, weights and their order.  Segmentation: sorted_pair / sorted_tok /
sorted_wts / inv / seg_start / active / tile lists, including invalid ids
(-1, >= E -> trash bucket), zero weights (kept, or dropped with drop_zero),
shared-expert pairs and an id translation map."""
import numpy as np
import pytest
import torch

import oracle
from helpers import random_routing
from xtu_moe_amd import layer as L

pytestmark = pytest.mark.gpu


def _gpu_route(logits, **kw):
    w, i = L.route(torch.from_numpy(logits).cuda(), **kw)
    torch.cuda.synchronize()
    return i.cpu().numpy(), w.cpu().numpy()


@pytest.mark.parametrize("T,E,K", [(1, 8, 2), (128, 8, 2), (4, 512, 10), (8192, 512, 10),
                                   (33, 256, 8), (3, 64, 1)])
def test_softmax_topk_bit_exact(T, E, K):
    rng = np.random.default_rng(T * 7 + E)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    if T > 4:   # plant exact ties so the tie-break is exercised
        logits[::3, 1] = logits[::3, 5]
        logits[1::5, : E // 2] = np.round(logits[1::5, : E // 2] * 2) / 2
    ids, wts = _gpu_route(logits, top_k=K, scoring="softmax")
    rids, rwts = oracle.route_softmax_topk(logits, K)
    np.testing.assert_array_equal(ids, rids)
    np.testing.assert_array_equal(wts.view(np.uint32), rwts.view(np.uint32))


def test_softmax_not_renormalized_bit_exact():
    rng = np.random.default_rng(5)
    logits = rng.standard_normal((17, 64)).astype(np.float32)
    ids, wts = _gpu_route(logits, top_k=4, scoring="softmax", renormalize=False)
    rids, rwts = oracle.route_softmax_topk(logits, 4, renormalize=False)
    np.testing.assert_array_equal(ids, rids)
    np.testing.assert_array_equal(wts.view(np.uint32), rwts.view(np.uint32))


@pytest.mark.parametrize("T", [1, 2, 4, 61, 8192])
@pytest.mark.parametrize("with_bias", [False, True])
def test_grouped_sigmoid_bit_exact(T, with_bias):
    rng = np.random.default_rng(T + 11 * with_bias)
    E, G, TG, K = 256, 8, 4, 8
    logits = rng.standard_normal((T, E)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32) if with_bias else None
    ids, wts = _gpu_route(logits, top_k=K, scoring="sigmoid", n_group=G, topk_group=TG,
                          routed_scaling_factor=2.5,
                          bias=None if bias is None else torch.from_numpy(bias).cuda())
    rids, rwts = oracle.route_grouped_sigmoid(logits, bias, G, TG, K, 2.5)
    np.testing.assert_array_equal(ids, rids)
    np.testing.assert_array_equal(wts.view(np.uint32), rwts.view(np.uint32))


def _gpu_segment(ids, wts, E, NS, drop_zero, id_map=None, bm=128):
    T, K = ids.shape
    seg = L.segmentation(T, K, E, NS, bm, torch.device("cuda"))
    idm = None if id_map is None else torch.from_numpy(id_map).cuda()
    seg.run(torch.from_numpy(ids).cuda(), torch.from_numpy(wts).cuda(), idm, drop_zero)
    torch.cuda.synchronize()
    return seg


@pytest.mark.parametrize("T,K,E,NS", [(1, 8, 256, 1), (4, 8, 256, 1), (128, 2, 8, 0),
                                      (8192, 8, 256, 1), (8192, 10, 512, 1), (5000, 3, 40, 2),
                                      (0, 4, 16, 1), (3000, 6, 1024, 3), (4096, 4, 5, 0)])
@pytest.mark.parametrize("drop_zero", [False, True])
def test_segmentation_bit_exact(T, K, E, NS, drop_zero):
    ids, wts = random_routing(T, K, E, seed=T + K, invalid_frac=0.05, zero_frac=0.05)
    seg = _gpu_segment(ids, wts, E, NS, drop_zero)
    ref = oracle.segment(ids, wts, E, NS, drop_zero)
    A = seg.A
    np.testing.assert_array_equal(seg.seg_start.cpu().numpy(), ref["seg_start"])
    for k in ("sorted_pair", "sorted_tok", "inv"):
        np.testing.assert_array_equal(getattr(seg, k).cpu().numpy()[:A], ref[k])
    np.testing.assert_array_equal(seg.sorted_wts.cpu().numpy()[:A].view(np.uint32),
                                  ref["sorted_wts"].view(np.uint32))
    counts = np.diff(ref["seg_start"])[: E + NS]
    nz = np.nonzero(counts)[0]
    assert int(seg.n_active.item()) == len(nz)
    np.testing.assert_array_equal(seg.active.cpu().numpy()[: len(nz)], nz)
    # tile list: bm-row tiles of every non-trash bucket, in bucket order
    tiles = [(e, ref["seg_start"][e] + j * 128) for e in range(E + NS)
             for j in range((counts[e] + 127) // 128)]
    assert int(seg.n_tiles.item()) == len(tiles)
    if tiles:
        np.testing.assert_array_equal(seg.tile_expert.cpu().numpy()[: len(tiles)], [t[0] for t in tiles])
        np.testing.assert_array_equal(seg.tile_row0.cpu().numpy()[: len(tiles)], [t[1] for t in tiles])
    ets = np.concatenate([[0], np.cumsum((counts + 127) // 128)])
    np.testing.assert_array_equal(seg.expert_tile_start.cpu().numpy()[: E + NS + 1], ets)


def test_segmentation_id_map():
    T, K, E = 300, 4, 32
    ids, wts = random_routing(T, K, E, seed=9, invalid_frac=0.02)
    rng = np.random.default_rng(1)
    id_map = rng.permutation(E).astype(np.int32)
    id_map[3] = -1     # an expert mapped away -> trash
    seg = _gpu_segment(ids, wts, E, 0, True, id_map=id_map)
    mapped = np.where((ids >= 0) & (ids < E), id_map[np.clip(ids, 0, E - 1)], ids).astype(np.int32)
    ref = oracle.segment(mapped, wts, E, 0, True)
    np.testing.assert_array_equal(seg.seg_start.cpu().numpy(), ref["seg_start"])
    np.testing.assert_array_equal(seg.sorted_pair.cpu().numpy()[: seg.A], ref["sorted_pair"])


@pytest.mark.parametrize("T,E,K,NS,mode", [(1, 256, 8, 1, 1), (4, 256, 8, 1, 1), (16, 256, 8, 1, 1),
                                           (1, 512, 10, 1, 0), (4, 512, 10, 1, 0), (13, 8, 2, 0, 0),
                                           (16, 64, 4, 2, 2), (64, 128, 8, 0, 2)])
def test_fused_small_route_segment_bit_exact(T, E, K, NS, mode):
    """One-launch routing + segmentation for small batches == router + segmentation."""
    rng = np.random.default_rng(T * 13 + E)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    dev = torch.device("cuda")
    seg = L.segmentation(T, K, E, NS, 128, dev)
    assert seg.small
    if mode == 2:
        ids_np, wts_np = random_routing(T, K, E, seed=T, invalid_frac=0.1, zero_frac=0.1)
        ids = torch.from_numpy(ids_np).to(dev)
        wts = torch.from_numpy(wts_np).to(dev)
        seg.run_small(2, ids, wts, drop_zero=True)
    else:
        ids = torch.empty((T, K), dtype=torch.int32, device=dev)
        wts = torch.empty((T, K), dtype=torch.float32, device=dev)
        kw = dict(n_group=8, topk_group=4, routed_scaling=2.5) if mode == 1 else {}
        seg.run_small(mode, ids, wts, logits=torch.from_numpy(logits).to(dev), **kw)
        if mode == 1:
            ids_np, wts_np = oracle.route_grouped_sigmoid(logits, None, 8, 4, K, 2.5)
        else:
            ids_np, wts_np = oracle.route_softmax_topk(logits, K)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_np)
    np.testing.assert_array_equal(wts.cpu().numpy().view(np.uint32), wts_np.view(np.uint32))
    ref = oracle.segment(ids_np, wts_np, E, NS, True)
    A = seg.A
    np.testing.assert_array_equal(seg.seg_start.cpu().numpy(), ref["seg_start"])
    for k in ("sorted_pair", "sorted_tok", "inv"):
        np.testing.assert_array_equal(getattr(seg, k).cpu().numpy()[:A], ref[k])
    np.testing.assert_array_equal(seg.sorted_wts.cpu().numpy()[:A].view(np.uint32),
                                  ref["sorted_wts"].view(np.uint32))
    counts = np.diff(ref["seg_start"])[: E + NS]
    nz = np.nonzero(counts)[0]
    assert int(seg.n_active.item()) == len(nz)
    np.testing.assert_array_equal(seg.active.cpu().numpy()[: len(nz)], nz)
    ets = np.concatenate([[0], np.cumsum((counts + 127) // 128)])
    np.testing.assert_array_equal(seg.expert_tile_start.cpu().numpy()[: E + NS + 1], ets)
    assert int(seg.n_tiles.item()) == ets[-1]


@pytest.mark.parametrize("T,E,K,renorm", [(128, 8, 2, True), (500, 8, 2, True),
                                           (40, 32, 8, True), (300, 16, 3, False),
                                           (7, 8, 2, False)])
def test_lane_softmax_route_segment_bit_exact(T, E, K, renorm):
    """Softmax over at most 32 experts, one thread per token, fused with the
    segmentation (any batch of at most 1024 pairs): ids, weights and the
    segmentation bit-exact, with exact ties and equal logits planted."""
    rng = np.random.default_rng(T + 3 * E + K)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    logits[::4, 1] = logits[::4, 0]
    logits[2::7] = np.round(logits[2::7] * 2) / 2
    logits[5::11, :] = 0.25                       # every expert tied
    dev = torch.device("cuda")
    seg = L.segmentation(T, K, E, 0, 128, dev)
    assert seg.small
    ids = torch.empty((T, K), dtype=torch.int32, device=dev)
    wts = torch.empty((T, K), dtype=torch.float32, device=dev)
    seg.run_small(0, ids, wts, logits=torch.from_numpy(logits).to(dev), renormalize=renorm)
    torch.cuda.synchronize()
    rids, rwts = oracle.route_softmax_topk(logits, K, renormalize=renorm)
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    np.testing.assert_array_equal(wts.cpu().numpy().view(np.uint32), rwts.view(np.uint32))
    ref = oracle.segment(rids, rwts, E, 0, True)
    np.testing.assert_array_equal(seg.seg_start.cpu().numpy(), ref["seg_start"])
    for k in ("sorted_pair", "sorted_tok", "inv"):
        np.testing.assert_array_equal(getattr(seg, k).cpu().numpy()[: seg.A], ref[k])


@pytest.mark.parametrize("NS", [55, 56, 60])
def test_lane_softmax_with_many_shared_buckets(NS):
    """Softmax over 8 experts with enough shared experts that the buckets
    (E + NS + 1) pass the ballot segmentation's 64: NS = 55 still fits it,
    56 and 60 take the counting-sort segmentation.  Routing and the whole
    segmentation bit-exact against the oracle."""
    T, E, K = 7, 8, 2
    rng = np.random.default_rng(NS)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    logits[::3, 1] = logits[::3, 4]
    dev = torch.device("cuda")
    seg = L.segmentation(T, K, E, NS, 16, dev)
    assert seg.small
    ids = torch.empty((T, K), dtype=torch.int32, device=dev)
    wts = torch.empty((T, K), dtype=torch.float32, device=dev)
    seg.run_small(0, ids, wts, logits=torch.from_numpy(logits).to(dev))
    torch.cuda.synchronize()
    rids, rwts = oracle.route_softmax_topk(logits, K, renormalize=True)
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    np.testing.assert_array_equal(wts.cpu().numpy().view(np.uint32), rwts.view(np.uint32))
    ref = oracle.segment(rids, rwts, E, NS, True)
    np.testing.assert_array_equal(seg.seg_start.cpu().numpy(), ref["seg_start"])
    for k in ("sorted_pair", "sorted_tok", "inv"):
        np.testing.assert_array_equal(getattr(seg, k).cpu().numpy()[: seg.A], ref[k])
    np.testing.assert_array_equal(seg.sorted_wts.cpu().numpy()[: seg.A].view(np.uint32),
                                  ref["sorted_wts"].view(np.uint32))


@pytest.mark.parametrize("case", ["grouped_ties_bias", "softmax_ties", "given_ids_idmap",
                                  "grouped_bm4", "grouped_e512_ties", "softmax_e256_ties"])
def test_tiny_route_segment_edge_cases(case):
    """The one-wave-per-token path (<= 64 pairs): exact ties, bias, id_map,
    given ids with invalid / zero-weight pairs, several tiles per bucket; both
    routers at both lane widths (4 and 8 experts per lane, so each lane's
    sorted list of tied scores is exercised at either size)."""
    dev = torch.device("cuda")
    rng = np.random.default_rng(len(case))
    T, E, K, NS, bm = 4, 256, 8, 1, 128
    id_map = None
    if case == "softmax_ties":
        E, K = 512, 10
    if case == "grouped_e512_ties":
        E, K = 512, 8
    if case == "softmax_e256_ties":
        E, K = 256, 6
    if case == "grouped_bm4":
        bm = 4
    # few distinct values: many exact ties in scores and group scores
    logits = (rng.integers(-2, 3, size=(T, E)) * 0.5).astype(np.float32)
    bias = (rng.integers(-1, 2, size=E) * 0.125).astype(np.float32) if case == "grouped_ties_bias" else None
    seg = L.segmentation(T, K, E, NS, bm, dev)
    if case == "given_ids_idmap":
        ids_np, wts_np = random_routing(T, K, E, seed=3, invalid_frac=0.15, zero_frac=0.15)
        id_map = rng.permutation(E).astype(np.int32)
        id_map[int(ids_np[0, 0]) % E] = -1
        ids = torch.from_numpy(ids_np).to(dev)
        wts = torch.from_numpy(wts_np).to(dev)
        seg.run_small(2, ids, wts, id_map=torch.from_numpy(id_map).to(dev), drop_zero=True)
        mapped = np.where((ids_np >= 0) & (ids_np < E), id_map[np.clip(ids_np, 0, E - 1)],
                          ids_np).astype(np.int32)
        ref = oracle.segment(mapped, wts_np, E, NS, True)
    else:
        ids = torch.empty((T, K), dtype=torch.int32, device=dev)
        wts = torch.empty((T, K), dtype=torch.float32, device=dev)
        lg = torch.from_numpy(logits).to(dev)
        if case in ("softmax_ties", "softmax_e256_ties"):
            seg.run_small(0, ids, wts, logits=lg)
            ids_np, wts_np = oracle.route_softmax_topk(logits, K)
        else:
            b = None if bias is None else torch.from_numpy(bias).to(dev)
            seg.run_small(1, ids, wts, logits=lg, bias=b, n_group=8, topk_group=4,
                          routed_scaling=2.5)
            ids_np, wts_np = oracle.route_grouped_sigmoid(logits, bias, 8, 4, K, 2.5)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(ids.cpu().numpy(), ids_np)
        np.testing.assert_array_equal(wts.cpu().numpy().view(np.uint32), wts_np.view(np.uint32))
        ref = oracle.segment(ids_np, wts_np, E, NS, True)
    torch.cuda.synchronize()
    A = seg.A
    np.testing.assert_array_equal(seg.seg_start.cpu().numpy(), ref["seg_start"])
    for k in ("sorted_pair", "sorted_tok", "inv"):
        np.testing.assert_array_equal(getattr(seg, k).cpu().numpy()[:A], ref[k])
    np.testing.assert_array_equal(seg.sorted_wts.cpu().numpy()[:A].view(np.uint32),
                                  ref["sorted_wts"].view(np.uint32))
    counts = np.diff(ref["seg_start"])[: E + NS]
    nz = np.nonzero(counts)[0]
    assert int(seg.n_active.item()) == len(nz)
    np.testing.assert_array_equal(seg.active.cpu().numpy()[: len(nz)], nz)
    nt = (counts + bm - 1) // bm
    ets = np.concatenate([[0], np.cumsum(nt)])
    np.testing.assert_array_equal(seg.expert_tile_start.cpu().numpy()[: E + NS + 1], ets)
    assert int(seg.n_tiles.item()) == ets[-1]
    te = np.repeat(np.arange(E + NS), nt)
    tr = np.concatenate([ref["seg_start"][e] + bm * np.arange(nt[e]) for e in range(E + NS)])
    np.testing.assert_array_equal(seg.tile_expert.cpu().numpy()[: ets[-1]], te)
    np.testing.assert_array_equal(seg.tile_row0.cpu().numpy()[: ets[-1]], tr)


@pytest.mark.parametrize("case", ["misaligned", "not-renormalized", "other-E"])
def test_large_batch_router_fallbacks_bit_exact(case):
    """Batches outside the one-wave-per-token router's envelope (logit rows
    not 16-byte aligned, softmax without renormalisation, E other than 256 or
    512) take the 256-thread-team router: same bit-exact results."""
    rng = np.random.default_rng(77)
    T = 300
    if case == "other-E":
        E, G, TG, K = 320, 16, 4, 8
        logits = rng.standard_normal((T, E)).astype(np.float32)
        ids, wts = _gpu_route(logits, top_k=K, scoring="sigmoid", n_group=G, topk_group=TG,
                              routed_scaling_factor=2.5)
        rids, rwts = oracle.route_grouped_sigmoid(logits, None, G, TG, K, 2.5)
    else:
        E, K = 512, 10
        logits = rng.standard_normal((T, E)).astype(np.float32)
        renorm = case != "not-renormalized"
        if case == "misaligned":
            base = torch.from_numpy(np.concatenate([[0.0], logits.ravel()]).astype(np.float32))
            lg = base.cuda()[1:].view(T, E)     # 4-byte offset
            w, i = L.route(lg, top_k=K, scoring="softmax")
            torch.cuda.synchronize()
            ids, wts = i.cpu().numpy(), w.cpu().numpy()
        else:
            ids, wts = _gpu_route(logits, top_k=K, scoring="softmax", renormalize=False)
        rids, rwts = oracle.route_softmax_topk(logits, K, renormalize=renorm)
    np.testing.assert_array_equal(ids, rids)
    np.testing.assert_array_equal(wts.view(np.uint32), rwts.view(np.uint32))
