"""Decode down projection writing y in flat pair order
(xtu_decode_down_by_pair) and the combine that reads it without inv first
(xtu_combine_by_pair), against the sorted-order down + combine (bitwise: the
same rows, the same sums in the same order) and against the dequantized-fp32
oracle, all four weight formats, plus the cases the skip rule covers: a token
listing an expert twice, zero weights kept or dropped, invalid ids (their y
rows are never written), every pair dropped, two shared experts, and a
weight-slot map with bf16 output."""
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


def _run(x, ids, wts, W, monkeypatch, by_pair, **kw):
    monkeypatch.setenv(L.FUSED_DOWN_ENV, "0")
    monkeypatch.setenv(L.DOWN_BY_PAIR_ENV, "1" if by_pair else "0")
    out = moe_forward(x.cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(wts).cuda(), W,
                      path="decode", **kw)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("T,H,I,E,K,NS", [(2, 256, 1024, 16, 4, 1), (4, 512, 256, 16, 8, 0),
                                          (5, 2048, 512, 64, 10, 1), (16, 512, 256, 16, 6, 2)])
def test_by_pair_vs_sorted_and_oracle(fmt, T, H, I, E, K, NS, monkeypatch):
    print(f"down by pair fmt={fmt} T={T} H={H} I={I} E={E} K={K} NS={NS}", flush=True)
    d, W = _layer(fmt, E, NS, H, I, seed=T + I + E)
    ids, wts = random_routing(T, K, E, seed=T + 7)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(T)).to(torch.bfloat16)
    bp = _run(x, ids, wts, W, monkeypatch, True, out_dtype=torch.float32)
    srt = _run(x, ids, wts, W, monkeypatch, False, out_dtype=torch.float32)
    assert torch.equal(bp, srt)
    ref = oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x), ids, wts, E, NS, H, I)
    check_close(bp.cpu().numpy(), ref, bf16_out=False, what=f"by pair fmt={fmt} T={T}")


@pytest.mark.parametrize("drop_zero", [True, False])
def test_by_pair_duplicates_zero_weights_invalid_ids(drop_zero, monkeypatch):
    fmt, E, NS, H, I, T, K = F.FMT_MXFP4, 12, 1, 256, 512, 6, 4
    d, W = _layer(fmt, E, NS, H, I, seed=21)
    ids, wts = random_routing(T, K, E, seed=22)
    ids[0, 1] = ids[0, 0]            # token 0 lists one expert twice
    ids[1, 2] = ids[1, 3] = ids[1, 0]
    wts[2, 1] = 0.0                  # zero weights, kept or dropped
    wts[3, :] = 0.0
    ids[4, 0], ids[4, 2] = -1, E + 2  # invalid ids go to the trash bucket
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(23)).to(torch.bfloat16)
    # y rows of trash pairs are never written: NaN in every cached y row first,
    # so a row added that should have been skipped shows
    _run(x, ids, wts, W, monkeypatch, True, out_dtype=torch.float32, drop_zero=drop_zero)
    for key, buf in L._BUF_CACHE.items():
        if key[0] == "y":
            buf.fill_(float("nan"))
    bp = _run(x, ids, wts, W, monkeypatch, True, out_dtype=torch.float32, drop_zero=drop_zero)
    srt = _run(x, ids, wts, W, monkeypatch, False, out_dtype=torch.float32, drop_zero=drop_zero)
    assert torch.equal(bp, srt)
    ref = oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x), ids, wts, E, NS, H, I)
    check_close(bp.cpu().numpy(), ref, bf16_out=False, what=f"dup/zero drop_zero={drop_zero}")


def test_by_pair_every_pair_dropped_writes_zero_rows(monkeypatch):
    fmt, E, NS, H, I, T, K = F.FMT_NVFP4, 8, 0, 256, 256, 3, 2
    _, W = _layer(fmt, E, NS, H, I, seed=31)
    ids = np.full((T, K), -1, np.int32)
    wts = np.ones((T, K), np.float32)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(32)).to(torch.bfloat16)
    for dt in (torch.float32, torch.bfloat16):
        out = torch.full((T, H), float("nan"), dtype=dt, device="cuda")
        _run(x, ids, wts, W, monkeypatch, True, out=out)
        assert torch.equal(out.float(), torch.zeros((T, H), device="cuda"))


def test_by_pair_slot_map_bf16_out(monkeypatch):
    fmt, E, NS, H, I, K = F.FMT_FP8, 16, 1, 512, 512, 4
    d, _ = _layer(fmt, E, NS, H, I, seed=41)
    order = np.arange(E + NS)[::-1].copy()
    idx = torch.from_numpy(order)
    rev = {k: (v[idx].contiguous() if v is not None else None) for k, v in d.items()}
    W = ExpertWeights.from_dense(fmt, rev["w13"], rev["s13"], rev["w2"], rev["s2"], rev["gs13"],
                                 rev["gs2"], n_shared=NS, device="cuda")
    slot_map = torch.from_numpy(np.argsort(order).astype(np.int32)).cuda()
    for T in (8, 3):
        ids, wts = random_routing(T, K, E, seed=42 + T)
        x = torch.randn((T, H), generator=torch.Generator().manual_seed(43 + T)).to(torch.bfloat16)
        bp = _run(x, ids, wts, W, monkeypatch, True, out_dtype=torch.bfloat16, slot_map=slot_map)
        srt = _run(x, ids, wts, W, monkeypatch, False, out_dtype=torch.bfloat16,
                   slot_map=slot_map)
        assert torch.equal(bp, srt)
        ref = oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x), ids, wts, E, NS,
                           H, I)
        check_close(bp.float().cpu().numpy(), ref, bf16_out=True, what=f"slot map T={T}")
