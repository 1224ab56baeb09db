"""MXFP4 GEMMs on the 32x32x64 scaled MFMA, with exact e4m3 activation pairs
(xtu_mx_pair_*) and with activation triples on the double-rate fp6 / fp4
MFMA (xtu_mx_tri_*) or their first two pieces (xtu_mx_duo_*): the
interleaved activation pairs bit-exact against the
planar quantiser's, the triples bit-exact against their CPU restatement
(tests/tri_ref.py), the step-major scale re-layout bit-exact against the
dense scales, and the layer against the oracle in both modes over tile
shapes (single rows, partial and multi-tile experts, a shared expert, a
SwiGLU clamp) and through a slot map on mutable planes (the ring / pool
layout)."""
import os

import numpy as np
import pytest
import torch

from helpers import bf16_tensor_to_bits, check_close, dense_to_numpy, make_dense_layer, oracle_layer
from tri_ref import tri_split
from xtu_moe_amd import _lib
from xtu_moe_amd import formats as F
from xtu_moe_amd import layer as L
from xtu_moe_amd.layer import ExpertWeights, _p, _stream, moe_forward

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


@pytest.fixture(params=["pair", "tri", "duo"])
def mode(request, monkeypatch):
    monkeypatch.setenv(L.MXFP4_PREFILL_ENV, request.param)
    return request.param


def test_triples_match_restatement():
    """xtu_tri_quant_il bytes and scale bytes equal tri_ref.tri_split's, on
    N(0,1) rows, rows of widely scaled blocks, and blocks at the edges (near
    the bf16 maximum, below the pieces' scale range, zeros, negative zeros,
    values on the e2m3 grid)."""
    x = torch.cat([_tri_rows(), torch.randn((37, 1024), generator=torch.Generator().manual_seed(5))
                   .to(torch.bfloat16)])
    for M, K, xx in ((x.shape[0], 1024, x), (1, 256, x[:1, :256]), (9, 7168, None)):
        if xx is None:
            xx = (torch.randn((M, K), generator=torch.Generator().manual_seed(6)) *
                  torch.exp2(torch.randint(-30, 30, (M, 1), generator=torch.Generator()
                                           .manual_seed(7)).float())).to(torch.bfloat16)
        xx = xx.contiguous()
        q = torch.empty((M, 2 * K), dtype=torch.uint8, device=DEV)
        sq = torch.empty((M, K // 32), dtype=torch.uint8, device=DEV)
        _lib.call("xtu_tri_quant_il", _p(xx.to(DEV)), M, K, _p(q), _p(sq), _stream())
        torch.cuda.synchronize()
        wq, wsq, _ = tri_split(xx)
        assert np.array_equal(sq.cpu().numpy(), wsq), (M, K)
        assert np.array_equal(q.cpu().numpy(), wq), (M, K)


def _tri_rows():
    from test_tri_ref import _rows
    return _rows()


@pytest.mark.parametrize("M,K", [(1, 256), (300, 1024), (37, 7168)])
def test_interleaved_pairs_match_planar(M, K):
    g = torch.Generator(device=DEV).manual_seed(M + K)
    x = (torch.randn((M, K), generator=g, device=DEV) *
         torch.exp2(torch.randint(-20, 12, (M, 1), generator=g, device=DEV).float())).to(torch.bfloat16)
    x[0, :32] = 0        # an all-zero block
    hi = torch.empty((M, K), dtype=torch.uint8, device=DEV)
    lo, shi, slo = torch.empty_like(hi), torch.empty((M, K // 32), dtype=torch.uint8, device=DEV), \
        torch.empty((M, K // 32), dtype=torch.uint8, device=DEV)
    hilo = torch.empty((M, 2 * K), dtype=torch.uint8, device=DEV)
    shi2 = torch.empty_like(shi)
    st = _stream()
    _lib.call("xtu_fp8pair_quant", _p(x), M, K, _p(hi), _p(lo), _p(shi), _p(slo), st)
    _lib.call("xtu_pair_quant_il", _p(x), M, K, _p(hilo), _p(shi2), st)
    torch.cuda.synchronize()
    il = hilo.view(M, K // 64, 2, 64)
    assert torch.equal(il[:, :, 0].reshape(M, K), hi)
    assert torch.equal(il[:, :, 1].reshape(M, K), lo)
    assert torch.equal(shi2, shi)
    # the lo scale the kernel derives is the one the planar quantiser writes
    assert torch.equal(torch.clamp(shi.int() - 4, min=0).to(torch.uint8), slo)


@pytest.mark.parametrize("N,K,pad", [(512, 256, 0), (4096, 7168, 0), (768, 1024, 4096)])
def test_step_major_scales(N, K, pad):
    E = 3
    g = torch.Generator().manual_seed(N + K)
    s = torch.randint(100, 140, (E, N, K // 32), generator=g, dtype=torch.uint8)
    packed = F.pack_scales(F.FMT_MXFP4, s, N, K)
    if pad:   # slots wider than the scale groups (a staging plane's row)
        packed = torch.cat([packed, torch.zeros((E, pad), dtype=torch.uint8)], 1)
    packed = packed.to(DEV)
    out = torch.empty((E, N * K // 32), dtype=torch.uint8, device=DEV)
    _lib.call("xtu_mx_pair_scales", _p(packed), E, N, K, packed.stride(0), _p(out), _stream())
    torch.cuda.synchronize()
    # [e][step][p][r][c] = s[e][16 p + r][2 step + c]
    want = s.view(E, N // 16, 16, K // 64, 2).permute(0, 3, 1, 2, 4).reshape(E, -1)
    assert torch.equal(out.cpu(), want)


FMTS = [F.FMT_MXFP4]


def _layer(fmt, E, NS, H, I, seed):
    d = make_dense_layer(fmt, E + NS, H, I, seed=seed)
    return d, ExpertWeights.from_dense(fmt, d["w13"], d["s13"], d["w2"], d["s2"], n_shared=NS,
                                       device=DEV)


def _on_kernel(fmt, H, I):
    mode = L.mx_act_mode(fmt, H, I)
    return (L.mx_pair_kernel(fmt, H, I) and L.gemm_tile_m(fmt, False, H, I) == 128
            and os.environ.get(L.MXFP4_PREFILL_ENV) == mode)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("T,K,skew", [(1, 2, False), (40, 4, False), (700, 4, False), (900, 2, True)])
def test_layer_against_oracle(fmt, T, K, skew, mode):
    E, NS, H, I = 16, 1, 1024, 512
    d, W = _layer(fmt, E, NS, H, I, seed=30 + T)
    assert _on_kernel(fmt, H, I)
    rng = np.random.default_rng(31 + T)
    if skew:   # experts 0 and 1 take most pairs: several full tiles and a partial one
        ids = np.stack([np.array([rng.integers(0, 2), rng.integers(2, E)]) for _ in range(T)])
    else:
        ids = np.stack([rng.permutation(E)[:K] for _ in range(T)])
    ids = ids.astype(np.int32)
    wts = (rng.random((T, K)) + 0.05).astype(np.float32)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(32 + T)).to(torch.bfloat16)
    out = moe_forward(x.to(DEV), torch.from_numpy(ids).to(DEV), torch.from_numpy(wts).to(DEV), W,
                      path="gemm", swiglu_limit=5.0, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x), ids, wts, E, NS, H, I,
                       limit=5.0)
    check_close(out.cpu().numpy(), ref, bf16_out=False, what=f"{mode} fmt={fmt} T={T}")


@pytest.mark.parametrize("fmt", FMTS)
def test_slot_map_on_mutable_planes(fmt, mode):
    """Experts at permuted slots of planes flagged mutable (restaged in
    place): the step-major scales are rebuilt per call, so restaging the
    slots between two calls gives the new experts' results."""
    E, NS, H, I, K, T = 8, 0, 1024, 256, 2, 300
    d, W = _layer(fmt, E, NS, H, I, seed=40)
    assert _on_kernel(fmt, H, I)
    perm = torch.tensor([5, 2, 7, 0, 3, 6, 1, 4], dtype=torch.int64)
    slots = ExpertWeights(fmt, H, I, E, 0, torch.empty_like(W.w13), torch.empty_like(W.s13),
                          torch.empty_like(W.w2), torch.empty_like(W.s2), mutable=True)
    rng = np.random.default_rng(41)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    wts = (rng.random((T, K)) + 0.05).astype(np.float32)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(42)).to(torch.bfloat16)
    ref = oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x), ids, wts, E, NS, H, I)
    xd, idd, wd = x.to(DEV), torch.from_numpy(ids).to(DEV), torch.from_numpy(wts).to(DEV)
    for round_ in range(2):
        p = perm if round_ == 0 else torch.roll(perm, 3)
        for e in range(E):   # expert e at slot p[e]
            for name in ("w13", "s13", "w2", "s2"):
                getattr(slots, name)[p[e]].copy_(getattr(W, name)[e])
        smap = p.to(torch.int32).to(DEV)
        out = moe_forward(xd, idd, wd, slots, path="gemm", slot_map=smap, out_dtype=torch.float32)
        torch.cuda.synchronize()
        check_close(out.cpu().numpy(), ref, bf16_out=False, what=f"slot map round {round_}")


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("T,K,skew", [(1, 2, False), (700, 4, False), (900, 2, True)])
def test_fused_act_quant_is_bitwise(fmt, T, K, skew, mode, monkeypatch):
    """The gate/up epilogue writing the down pass's pairs / triples
    (xtu_mx_gate_up_q) gives the layer output bitwise equal to the bf16 rows
    quantised by the separate kernel, over single rows, partial and
    multi-tile experts and a shared expert."""
    E, NS, H, I = 16, 1, 1024, 512
    d, W = _layer(fmt, E, NS, H, I, seed=130 + T)
    assert _on_kernel(fmt, H, I)
    rng = np.random.default_rng(131 + T)
    if skew:
        ids = np.stack([np.array([rng.integers(0, 2), rng.integers(2, E)]) for _ in range(T)])
    else:
        ids = np.stack([rng.permutation(E)[:K] for _ in range(T)])
    ids = torch.from_numpy(ids.astype(np.int32)).to(DEV)
    wts = torch.from_numpy((rng.random((T, K)) + 0.05).astype(np.float32)).to(DEV)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(132 + T)).to(torch.bfloat16)
    outs = []
    for fused in ("1", "0"):
        monkeypatch.setenv(L.ACT_QUANT_ENV, fused)
        outs.append(moe_forward(x.to(DEV), ids, wts, W, path="gemm", swiglu_limit=5.0,
                                out_dtype=torch.float32))
    torch.cuda.synchronize()
    assert torch.equal(outs[0].view(torch.int32), outs[1].view(torch.int32)), mode
