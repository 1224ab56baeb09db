"""Full expert layer on the GPU (decode kernels and grouped GEMMs) against the
dequantized-fp32 oracle, all four weight formats, plus the INT8 ALIGN path's
int32 accumulators bit-exact."""
import numpy as np
import pytest
import torch

import oracle
from helpers import (bf16_tensor_to_bits, check_close, dense_to_numpy, make_dense_layer,
                     oracle_layer, random_routing)
from xtu_moe_amd import _lib
from xtu_moe_amd import formats as F
from xtu_moe_amd import layer as L
from xtu_moe_amd.layer import ExpertWeights, _p, _stream, moe_forward

pytestmark = pytest.mark.gpu

FMTS = [F.FMT_MXFP4, F.FMT_NVFP4, F.FMT_FP8, F.FMT_BF16]


def _poison_scratch():
    """Fill the layer's cached intermediate buffers with NaN so a row the
    kernels fail to write shows up in the output."""
    for t in L._BUF_CACHE.values():
        if t.is_floating_point():
            t.fill_(float("nan"))


def _case(fmt, E, NS, H, I, T, K, seed=0, invalid=0.0, zero=0.0, limit=0.0, path="auto",
          out_dtype=torch.float32):
    d = make_dense_layer(fmt, E + NS, H, I, seed=seed)
    W = ExpertWeights.from_dense(fmt, d["w13"], d["s13"], d["w2"], d["s2"], d["gs13"], d["gs2"],
                                 n_shared=NS, device="cuda")
    ids, wts = random_routing(T, K, E, seed=seed + 1, invalid_frac=invalid, zero_frac=zero)
    g = torch.Generator().manual_seed(seed + 2)
    x = torch.randn((T, H), generator=g).to(torch.bfloat16)
    _poison_scratch()
    out = moe_forward(x.cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(wts).cuda(), W,
                      swiglu_limit=limit, path=path, out_dtype=out_dtype)
    torch.cuda.synchronize()
    ref = oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x), ids, wts, E, NS, H, I,
                       limit=limit)
    return out.float().cpu().numpy(), ref


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("T", [1, 3, 16])
def test_decode_small(fmt, T):
    out, ref = _case(fmt, E=8, NS=1, H=256, I=256, T=T, K=2, seed=T, path="decode")
    check_close(out, ref, bf16_out=False, what=f"decode fmt={fmt} T={T}")


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("T", [5, 70, 300])
def test_gemm_small(fmt, T):
    out, ref = _case(fmt, E=8, NS=1, H=256, I=256, T=T, K=3, seed=T + 1, path="gemm")
    check_close(out, ref, bf16_out=False, what=f"gemm fmt={fmt} T={T}")


@pytest.mark.parametrize("path", ["decode", "gemm"])
def test_edge_invalid_ids_zero_weights_clamp(path):
    out, ref = _case(F.FMT_MXFP4, E=16, NS=0, H=512, I=256, T=12, K=4, seed=3, invalid=0.2,
                     zero=0.2, limit=1.0, path=path)
    check_close(out, ref, bf16_out=False, what=f"edge {path}")


def test_bf16_output_and_default_path():
    out, ref = _case(F.FMT_FP8, E=8, NS=1, H=512, I=256, T=40, K=2, seed=4,
                     out_dtype=torch.bfloat16)
    check_close(out, ref, bf16_out=True, what="bf16 out")


def test_ds_v3_mxfp4_decode_full_shape():
    """DeepSeek-V3 shape (H=7168, I=2048, 256 routed + 1 shared), T=1..4, routed
    with the GPU grouped-sigmoid router; a sample of experts kept small by
    building only the experts the routing touches."""
    H, I, E, K = 7168, 2048, 256, 8
    rng = np.random.default_rng(0)
    for T in (1, 4):
        logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).cuda()
        from xtu_moe_amd.layer import route
        wts, ids = route(logits, top_k=K, scoring="sigmoid", n_group=8, topk_group=4,
                         routed_scaling_factor=2.5)
        ids_np = ids.cpu().numpy()
        used = np.unique(ids_np)
        # compact the used experts to 0..U-1 (+ shared at U) so the test builds U+1 experts
        remap = {int(e): i for i, e in enumerate(used)}
        cids = np.vectorize(remap.get)(ids_np).astype(np.int32)
        U = len(used)
        d = make_dense_layer(F.FMT_MXFP4, U + 1, H, I, seed=10 + T)
        W = ExpertWeights.from_dense(F.FMT_MXFP4, d["w13"], d["s13"], d["w2"], d["s2"],
                                     n_shared=1, device="cuda")
        x = torch.randn((T, H), generator=torch.Generator().manual_seed(T)).to(torch.bfloat16)
        out = moe_forward(x.cuda(), torch.from_numpy(cids).cuda(), wts, W, out_dtype=torch.float32)
        torch.cuda.synchronize()
        ref = oracle_layer(F.FMT_MXFP4, dense_to_numpy(F.FMT_MXFP4, d), bf16_tensor_to_bits(x),
                           cids, wts.cpu().numpy(), U, 1, H, I)
        check_close(out.cpu().numpy(), ref, bf16_out=False, what=f"ds-v3 T={T}")


def test_int8_accumulators_bit_exact():
    """INT8 ALIGN GEMMs: the raw int32 accumulators equal the oracle's exactly."""
    H, I, E = 512, 256, 4
    d = make_dense_layer(F.FMT_MXFP4, E, H, I, seed=21)
    W = ExpertWeights.from_dense(F.FMT_MXFP4, d["w13"], d["s13"], d["w2"], d["s2"], device="cuda")
    w13_8, emin13, w2_8, emin2 = W.int8_planes()
    T = 37
    ids, wts = random_routing(T, 2, E, seed=5)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).cuda()
    from xtu_moe_amd.layer import segmentation
    seg = segmentation(T, 2, E, 0, 128, torch.device("cuda")).run(
        torch.from_numpy(ids).cuda(), torch.from_numpy(wts).cuda())
    A = seg.A
    st = _stream()
    a8x = torch.empty((T, H), dtype=torch.int8, device="cuda")
    crx = torch.empty(T, dtype=torch.int32, device="cuda")
    _lib.call("xtu_i8_quant_rows", _p(x), T, H, _p(a8x), _p(crx), st)
    act = torch.empty((A, I), dtype=torch.bfloat16, device="cuda")
    acc13 = torch.zeros((A, 2 * I), dtype=torch.int32, device="cuda")
    lo, hi = seg.tile_range_ptrs(0, E)
    _lib.call("xtu_i8_gemm_gate_up", _p(a8x), _p(crx), _p(seg.sorted_tok), H, I, _p(w13_8),
              _p(emin13), 0, _p(seg.seg_start), _p(seg.tile_expert), _p(seg.tile_row0), lo, hi,
              seg.max_tiles, _p(act), _p(acc13), 0.0, 1.0, 0.0, st)
    a8a = torch.empty((A, I), dtype=torch.int8, device="cuda")
    cra = torch.empty(A, dtype=torch.int32, device="cuda")
    _lib.call("xtu_i8_quant_rows", _p(act), A, I, _p(a8a), _p(cra), st)
    y = torch.empty((A, H), dtype=torch.float32, device="cuda")
    acc2 = torch.zeros((A, H), dtype=torch.int32, device="cuda")
    _lib.call("xtu_i8_gemm_down", _p(a8a), _p(cra), H, I, _p(w2_8), _p(emin2), 0,
              _p(seg.seg_start), _p(seg.tile_expert), _p(seg.tile_row0), lo, hi, seg.max_tiles,
              _p(y), _p(acc2), st)
    torch.cuda.synchronize()
    dn = dense_to_numpy(F.FMT_MXFP4, d)
    xf = oracle.bf16_bits_to_f32(bf16_tensor_to_bits(x.cpu()))
    tok = seg.sorted_tok.cpu().numpy()[:A]
    seg_start = seg.seg_start.cpu().numpy()
    act_f = oracle.bf16_bits_to_f32(bf16_tensor_to_bits(act.cpu()))
    g_acc13, g_acc2, g_y = acc13.cpu().numpy(), acc2.cpu().numpy(), y.cpu().numpy()
    for e in range(E):
        r0, r1 = seg_start[e], seg_start[e + 1]
        if r1 == r0:
            continue
        acc, c, dmax = oracle.i8_gemm(xf[tok[r0:r1]], dn["w13"][e], dn["s13"][e])
        assert dmax <= 3
        np.testing.assert_array_equal(g_acc13[r0:r1], acc)
        acc, c, _ = oracle.i8_gemm(act_f[r0:r1], dn["w2"][e], dn["s2"][e])
        np.testing.assert_array_equal(g_acc2[r0:r1], acc)
        np.testing.assert_array_equal(g_y[r0:r1].view(np.uint32), c.view(np.uint32))


def test_int8_layer_vs_oracle():
    H, I, E, NS = 512, 256, 8, 1
    d = make_dense_layer(F.FMT_MXFP4, E + NS, H, I, seed=8)
    W = ExpertWeights.from_dense(F.FMT_MXFP4, d["w13"], d["s13"], d["w2"], d["s2"], n_shared=NS,
                                 device="cuda")
    T, K = 200, 3
    ids, wts = random_routing(T, K, E, seed=6)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    out = moe_forward(x.cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(wts).cuda(), W,
                      int8=True, out_dtype=torch.float32)
    torch.cuda.synchronize()
    dn = dense_to_numpy(F.FMT_MXFP4, d)
    ref = oracle.moe_layer_i8(bf16_tensor_to_bits(x), ids, wts, E, NS, H, I, dn["w13"], dn["s13"],
                              dn["w2"], dn["s2"])
    check_close(out.cpu().numpy(), ref, bf16_out=False, what="int8 layer")


@pytest.mark.parametrize("path", ["decode", "gemm"])
def test_two_streams_do_not_share_scratch(path):
    """Layers issued on two streams back to back, without waiting for each
    other: each stream's scratch buffers and segmentation are its own, so both
    outputs equal those of the same layers run one after the other."""
    fmt, E, NS, H, I, K = F.FMT_MXFP4, 32, 1, 512, 256, 4
    T = 4 if path == "decode" else 96
    d = make_dense_layer(fmt, E + NS, H, I, seed=41)
    W = ExpertWeights.from_dense(fmt, d["w13"], d["s13"], d["w2"], d["s2"], d["gs13"], d["gs2"],
                                 n_shared=NS, device="cuda")
    ins = []
    for seed in (42, 43):
        ids, wts = random_routing(T, K, E, seed=seed)
        x = torch.randn((T, H), generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)
        ins.append((x.cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(wts).cuda()))
    ref = [moe_forward(x, i, w, W, path=path, out_dtype=torch.float32) for x, i, w in ins]
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())
    outs = []
    for s, (x, i, w) in zip((s1, s2), ins):
        with torch.cuda.stream(s):
            outs.append(moe_forward(x, i, w, W, path=path, out_dtype=torch.float32, stream=s))
    torch.cuda.synchronize()
    for a, b in zip(outs, ref):
        assert torch.equal(a, b)
