"""The reference-signature small-M ABI (moe4_smallm_init / gu / dn / gu2 / dn2
over K-major MXFP4 planes), called through the C ABI the way the reference's
Python caller drives it (vllm_xiaotu_moe/moe4_smallm.py:151-341: the fast
in-kernel-dispatch pair gu2 -> SwiGLU in torch -> dn2, and the segment-table
pair gu -> SwiGLU -> dn, with a slot map), against the oracle's layer.

The reference path keeps act in fp32 (no bf16 rounding before down), so its
outputs differ from the oracle's bf16-act layer by act rounding only: well
inside the layer tolerance.  A column count that is a multiple of 4 but not
8 (the narrow-column kernel) is checked against the dequantised product."""
import numpy as np
import pytest
import torch

import oracle
from helpers import bf16_tensor_to_bits, check_close, dense_to_numpy, make_dense_layer
from helpers import random_routing
from xtu_moe_amd import _lib
from xtu_moe_amd import formats as F

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
FMT = F.FMT_MXFP4


def _kmajor(d):
    """Pool K-major planes (w13 [S, H/2, 2I], s13 [S, H/32, 2I], w2 [S, I/2, H],
    s2 [S, I/32, H]) from checkpoint tensors [S, N, K/2] / [S, N, K/32]."""
    km = lambda t: t.view(torch.uint8).permute(0, 2, 1).contiguous().to(DEV)
    return km(d["w13"]), km(d["s13"]), km(d["w2"]), km(d["s2"])


def _p(t):
    return 0 if t is None else t.data_ptr()


def _swiglu(inter, I, limit):
    g, u = inter[:, :I], inter[:, I:]
    if limit > 0:
        g, u = g.clamp(max=limit), u.clamp(-limit, limit)
    return (torch.nn.functional.silu(g) * u).contiguous()


def _fast(planes, x, ids, wts, E, H, I, limit=0.0):
    w13, s13, w2, s2 = planes
    T, K = ids.shape
    st = torch.cuda.current_stream().cuda_stream
    inter = torch.zeros((E * 8, 2 * I), device=DEV)
    _lib.call("moe4_smallm_gu2", _p(w13), _p(s13), _p(x), _p(inter), _p(ids), T, K, E, H, 2 * I,
              st)
    act = _swiglu(inter, I, limit)
    res = torch.zeros((T, H), device=DEV)
    _lib.call("moe4_smallm_dn2", _p(w2), _p(s2), _p(act), _p(res), _p(ids), _p(wts), T, K, E, I,
              H, st)
    return res


def _segments(ids, wts, E):
    """The reference's own segmentation (moe4_smallm.py:97-129): pairs stably
    sorted by expert."""
    fi = ids.reshape(-1).cpu().numpy()
    fw = wts.reshape(-1).cpu().numpy()
    K = ids.shape[1]
    order = np.argsort(fi, kind="stable")
    tok = (order // K).astype(np.int32)
    seg = np.zeros(E + 1, np.int32)
    np.add.at(seg, fi + 1, 1)
    seg = np.cumsum(seg).astype(np.int32)
    return (torch.from_numpy(tok).to(DEV), torch.from_numpy(fw[order].copy()).to(DEV),
            torch.from_numpy(seg).to(DEV), len(fi))


def _segmented(planes, x, ids, wts, E, H, I, slot_map=None, slot_base=0, limit=0.0):
    w13, s13, w2, s2 = planes
    T = ids.shape[0]
    tok, sw, seg, A = _segments(ids, wts, E)
    seg2exp = torch.arange(E, dtype=torch.int32, device=DEV)
    st = torch.cuda.current_stream().cuda_stream
    inter = torch.zeros((A, 2 * I), device=DEV)
    _lib.call("moe4_smallm_gu", _p(w13), _p(s13), _p(x), _p(inter), _p(seg2exp), _p(seg),
              _p(tok), _p(slot_map), slot_base, E, H, 2 * I, st)
    act = _swiglu(inter, I, limit)
    res = torch.zeros((T, H), device=DEV)
    _lib.call("moe4_smallm_dn", _p(w2), _p(s2), _p(act), _p(res), _p(seg2exp), _p(seg), _p(tok),
              _p(sw), _p(slot_map), slot_base, E, I, H, st)
    return res


def _ref(d, x, ids, wts, E, H, I, limit=0.0):
    return oracle.moe_layer(FMT, bf16_tensor_to_bits(x), ids.cpu().numpy(), wts.cpu().numpy(),
                            E, 0, H, I, *[dense_to_numpy(FMT, d)[k] for k in
                                          ("w13", "s13", "w2", "s2", "gs13", "gs2")],
                            limit=limit)


@pytest.mark.parametrize("T,K", [(1, 8), (4, 6), (8, 8)])
def test_fast_pair_matches_oracle(T, K):
    E, H, I = 16, 512, 256
    assert _lib.call("moe4_smallm_init") == 0
    d = make_dense_layer(FMT, E, H, I, seed=T)
    planes = _kmajor(d)
    ids, wts = random_routing(T, K, E, seed=T)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(T)).to(torch.bfloat16)
    idd, wd = torch.from_numpy(ids).to(DEV), torch.from_numpy(wts).to(DEV)
    out = _fast(planes, x.to(DEV), idd, wd, E, H, I, limit=7.0)
    torch.cuda.synchronize()
    check_close(out.cpu().numpy(), _ref(d, x, idd, wd, E, H, I, limit=7.0), bf16_out=False,
                what=f"gu2/dn2 T={T}")


def test_segment_pair_with_slot_map_matches_oracle():
    E, H, I, T, K = 16, 1024, 512, 5, 4
    d = make_dense_layer(FMT, E, H, I, seed=7)
    w13, s13, w2, s2 = _kmajor(d)
    # planes hold the experts in reverse order; slot_map[e] - slot_base = its row
    rev = torch.arange(E - 1, -1, -1, device=DEV)
    planes = tuple(t[rev].contiguous() for t in (w13, s13, w2, s2))
    base = 100
    slot_map = (base + torch.arange(E - 1, -1, -1, dtype=torch.int32)).to(DEV)
    ids, wts = random_routing(T, K, E, seed=8)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    idd, wd = torch.from_numpy(ids).to(DEV), torch.from_numpy(wts).to(DEV)
    out = _segmented(planes, x.to(DEV), idd, wd, E, H, I, slot_map=slot_map, slot_base=base)
    torch.cuda.synchronize()
    check_close(out.cpu().numpy(), _ref(d, x, idd, wd, E, H, I), bf16_out=False,
                what="gu/dn with slot map")
    # identity weight rows: the same result without the map
    out2 = _segmented((w13, s13, w2, s2), x.to(DEV), idd, wd, E, H, I)
    torch.cuda.synchronize()
    check_close(out2.cpu().numpy(), _ref(d, x, idd, wd, E, H, I), bf16_out=False,
                what="gu/dn")


def test_narrow_columns_and_rejected_shapes():
    # N = 36 columns (a multiple of 4, not of 8), K = 64: one expert, 3 tokens
    E, K, N, T = 2, 64, 36, 3
    rng = np.random.default_rng(5)
    w = rng.integers(0, 256, (E, K // 2, N), dtype=np.uint8)
    sc = rng.integers(118, 130, (E, K // 32, N), dtype=np.uint8)
    x = torch.randn((T, K), generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    ids = torch.tensor([[1], [0], [1]], dtype=torch.int32, device=DEV)
    y = torch.zeros((E * 8, N), device=DEV)
    wt, st = torch.from_numpy(w).to(DEV), torch.from_numpy(sc).to(DEV)
    _lib.call("moe4_smallm_gu2", wt.data_ptr(), st.data_ptr(), x.to(DEV).data_ptr(), y.data_ptr(),
              ids.data_ptr(), T, 1, E, K, N, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    e2m1, e8m0 = oracle.e2m1_table(), oracle.e8m0_table()
    deq = np.empty((E, K, N), np.float64)
    deq[:, 0::2, :] = e2m1[w & 15]
    deq[:, 1::2, :] = e2m1[w >> 4]
    deq *= np.repeat(e8m0[sc], 32, axis=1)
    xf = oracle.bf16_bits_to_f32(bf16_tensor_to_bits(x)).astype(np.float64)
    want = np.zeros((E * 8, N))
    want[8 * 1 + 0] = xf[0] @ deq[1]
    want[8 * 1 + 1] = xf[2] @ deq[1]
    want[8 * 0 + 0] = xf[1] @ deq[0]
    np.testing.assert_allclose(y.cpu().numpy(), want, rtol=1e-5, atol=1e-5)
    lib = _lib.load()
    assert lib.moe4_smallm_gu2(None, None, None, None, None, T, 1, E, 48, N, None) == 1   # K % 32
    assert lib.moe4_smallm_dn2(None, None, None, None, None, None, T, 1, E, K, 34, None) == 1
