"""INT8 ALIGN with weight rows whose e8m0 spread exceeds 3 (the integer path
cannot hold them): those rows' output columns come from the fp32 fallback,
the rest from the integer GEMMs.  The layer against the oracle's restatement
of the same rule, the unmarked columns' int32 accumulators bit-exact against
the oracle's integer closed form, and the marked rows' accumulators zero
(their int8 weights are cleared, their columns are the fallback's)."""
import numpy as np
import pytest
import torch

import oracle
from helpers import bf16_tensor_to_bits, check_close, dense_to_numpy, make_dense_layer
from xtu_moe_amd import _lib
from xtu_moe_amd import formats as F
from xtu_moe_amd.layer import ExpertWeights, _p, _stream, moe_forward, segmentation

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _marked(E, NS, H, I, seed):
    d = make_dense_layer(F.FMT_MXFP4, E + NS, H, I, seed=seed)
    s13, s2 = d["s13"].clone(), d["s2"].clone()
    # gate row 5 of expert 1 (spread 5), up row 9 of expert 2 (4), down row 7
    # of expert 3 (6) and of the shared expert (5)
    for plane, e, row, spread in ((s13, 1, 5, 5), (s13, 2, I + 9, 4), (s2, 3, 7, 6),
                                  (s2, E, 300, 5)):
        m = int(plane[e, row].min())
        plane[e, row, 0], plane[e, row, 1] = m + spread, m
    d["s13"], d["s2"] = s13, s2
    return d


@pytest.mark.parametrize("T", [200, 1000])
def test_int8_marked_rows_layer_matches_oracle(T):
    E, NS, H, I, K = 8, 1, 512, 512, 2
    d = _marked(E, NS, H, I, seed=80)
    W = ExpertWeights.from_dense(F.FMT_MXFP4, d["w13"], d["s13"], d["w2"], d["s2"], n_shared=NS,
                                 device=DEV)
    fb = W.int8_fallback_cols()
    assert fb is not None
    assert fb[0].cpu().tolist()[:5] == [0, 0, 1, 2, 2]     # gate/up column pairs per slot
    rng = np.random.default_rng(81)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    wts = (rng.random((T, K)) + 0.05).astype(np.float32)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(82)).to(torch.bfloat16)
    out = moe_forward(x.to(DEV), torch.from_numpy(ids).to(DEV), torch.from_numpy(wts).to(DEV), W,
                      int8=True, swiglu_limit=7.0, out_dtype=torch.float32)
    torch.cuda.synchronize()
    dn = dense_to_numpy(F.FMT_MXFP4, d)
    ref = oracle.moe_layer_i8(bf16_tensor_to_bits(x), ids, wts, E, NS, H, I, dn["w13"], dn["s13"],
                              dn["w2"], dn["s2"], limit=7.0)
    check_close(out.cpu().numpy(), ref, bf16_out=False, what=f"int8 marked rows T={T}")


def test_int8_marked_rows_accumulators():
    E, NS, H, I, K, T = 8, 1, 512, 512, 2, 300
    d = _marked(E, NS, H, I, seed=83)
    W = ExpertWeights.from_dense(F.FMT_MXFP4, d["w13"], d["s13"], d["w2"], d["s2"], n_shared=NS,
                                 device=DEV)
    rng = np.random.default_rng(84)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    wts = np.ones((T, K), np.float32)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(85)).to(torch.bfloat16).to(DEV)
    ti, tw = torch.from_numpy(ids).to(DEV), torch.from_numpy(wts).to(DEV)
    w13_8, emin13, _, _ = W.int8_planes()
    seg = segmentation(T, K, E, NS, 128, DEV).run(ti, tw)
    st = _stream()
    a8x = torch.empty((T, H), dtype=torch.int8, device=DEV)
    crx = torch.empty(T, dtype=torch.int32, device=DEV)
    _lib.call("xtu_i8_quant_rows", _p(x), T, H, _p(a8x), _p(crx), st)
    act = torch.empty((seg.A, I), dtype=torch.bfloat16, device=DEV)
    acc = torch.full((seg.A, 2 * I), -1, dtype=torch.int32, device=DEV)
    lo, hi = seg.tile_range_ptrs(0, E + NS)
    _lib.call("xtu_i8_gemm_gate_up", _p(a8x), _p(crx), _p(seg.sorted_tok), H, I, _p(w13_8),
              _p(emin13), 0, _p(seg.seg_start), _p(seg.tile_expert), _p(seg.tile_row0), lo, hi,
              seg.max_tiles, _p(act), _p(acc), 7.0, 1.0, 0.0, st)
    torch.cuda.synchronize()
    ss, stok = seg.seg_start.cpu().numpy(), seg.sorted_tok.cpu().numpy()
    dn = dense_to_numpy(F.FMT_MXFP4, d)
    xf = oracle.bf16_bits_to_f32(bf16_tensor_to_bits(x))
    for e in (1, 2, 4):
        r0, r1 = int(ss[e]), int(ss[e + 1])
        ref_acc, _, _ = oracle.i8_gemm(xf[stok[r0:r1]], dn["w13"][e], dn["s13"][e])
        got = acc[r0:r1].cpu().numpy()
        spread = np.ptp(dn["s13"][e].astype(np.int32), axis=1)
        ok = spread <= 3
        np.testing.assert_array_equal(got[:, ok], ref_acc[:, ok], err_msg=f"expert {e}")
        assert (got[:, ~ok] == 0).all()
        assert (~ok).sum() == (1 if e in (1, 2) else 0)


def test_int8_offset_guard_rows_take_fp32():
    """Tokens scaled by 2^-20 fall past the engine's offset guard (crow + the
    expert's smallest e8m0 byte - 128 < -24) for gate/up and, through their
    tiny act rows, for down: their rows are recomputed whole in fp32 (they
    match the fp32 oracle far inside the ~2e-2 the INT8 rounding would
    leave), the other tokens stay on the integer path (the INT8 oracle)."""
    E, NS, H, I, K, T = 8, 1, 512, 512, 2, 300
    d = make_dense_layer(F.FMT_MXFP4, E + NS, H, I, seed=84)
    W = ExpertWeights.from_dense(F.FMT_MXFP4, d["w13"], d["s13"], d["w2"], d["s2"], n_shared=NS,
                                 device=DEV)
    rng = np.random.default_rng(85)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    wts = (rng.random((T, K)) + 0.05).astype(np.float32)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(86))
    tiny = np.zeros(T, bool)
    tiny[rng.choice(T, size=40, replace=False)] = True
    x[torch.from_numpy(tiny)] *= 2.0 ** -20
    x = x.to(torch.bfloat16)
    out = moe_forward(x.to(DEV), torch.from_numpy(ids).to(DEV), torch.from_numpy(wts).to(DEV), W,
                      int8=True, swiglu_limit=7.0, out_dtype=torch.float32)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    dn = dense_to_numpy(F.FMT_MXFP4, d)
    xb = bf16_tensor_to_bits(x)
    ref8 = oracle.moe_layer_i8(xb, ids, wts, E, NS, H, I, dn["w13"], dn["s13"], dn["w2"],
                               dn["s2"], limit=7.0)
    check_close(o[~tiny], ref8[~tiny], bf16_out=False, what="int8 rows")
    ref32 = oracle.moe_layer(F.FMT_MXFP4, xb[tiny], ids[tiny], wts[tiny], E, NS, H, I, dn["w13"],
                             dn["s13"], dn["w2"], dn["s2"], limit=7.0)
    from helpers import rel_l2
    assert rel_l2(o[tiny], ref32) < 1e-4
    assert rel_l2(ref8[tiny], ref32) < 1e-4      # the oracle restates the same guard
