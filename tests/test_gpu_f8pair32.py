"""FP8 exact-pair GEMMs on the 32x32x64 scaled MFMA (xtu_f8_pair_*), block
scales applied by accumulator rescaling: the layer against the oracle over
tile shapes (single rows, partial and multi-tile experts, a shared expert, a
SwiGLU clamp, several 128-k scale blocks with scales spread over 2^8), the
same layer on the 16x16x128 kernel ("v1") within the layer tolerance of it,
slot planes through a slot map (the ring / pool layout, kernel chosen by the
caller's scale statement), and the scale-bound check (a zero or a spread
beyond 2^32 sends the layer to the 16x16x128 kernel, which still matches the
oracle)."""
import numpy as np
import pytest
import torch

from helpers import bf16_tensor_to_bits, check_close, dense_to_numpy, make_dense_layer, oracle_layer
from xtu_moe_amd import formats as F
from xtu_moe_amd import layer as L
from xtu_moe_amd.layer import ExpertWeights, moe_forward

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
FMT = F.FMT_FP8


def _layer(E, NS, H, I, seed, spread=0):
    d = make_dense_layer(FMT, E + NS, H, I, seed=seed)
    if spread:   # block scales times 2^-u, u uniform in [0, spread]
        g = torch.Generator().manual_seed(seed + 1)
        for k in ("s13", "s2"):
            d[k] = d[k] * torch.exp2(-torch.randint(0, spread + 1, d[k].shape, generator=g)
                                     .float())
    W = ExpertWeights.from_dense(FMT, d["w13"], d["s13"], d["w2"], d["s2"], n_shared=NS,
                                 device=DEV)
    return d, W


def _routing(T, K, E, seed, skew=False):
    rng = np.random.default_rng(seed)
    if skew:   # experts 0 and 1 take most pairs: several full tiles and a partial one
        ids = np.stack([np.array([rng.integers(0, 2), rng.integers(2, E)]) for _ in range(T)])
    else:
        ids = np.stack([rng.permutation(E)[:K] for _ in range(T)])
    return ids.astype(np.int32), (rng.random((T, K)) + 0.05).astype(np.float32)


def _run(x, ids, wts, W, **kw):
    out = moe_forward(x.to(DEV), torch.from_numpy(ids).to(DEV), torch.from_numpy(wts).to(DEV), W,
                      path="gemm", out_dtype=torch.float32, **kw)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("T,K,skew,spread", [(1, 2, False, 0), (40, 4, False, 8),
                                             (700, 4, False, 0), (900, 2, True, 8)])
def test_layer_against_oracle(monkeypatch, T, K, skew, spread):
    monkeypatch.setenv(L.FP8_PREFILL_ENV, "auto")
    E, NS, H, I = 16, 1, 1024, 512
    d, W = _layer(E, NS, H, I, seed=50 + T, spread=spread)
    assert L.fp8_pair32_use(W) and L.gemm_tile_m(FMT, False, H, I, W) == 128
    ids, wts = _routing(T, K, E, 51 + T, skew)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(52 + T)).to(torch.bfloat16)
    got = _run(x, ids, wts, W, swiglu_limit=5.0)
    ref = oracle_layer(FMT, dense_to_numpy(FMT, d), bf16_tensor_to_bits(x), ids, wts, E, NS, H, I,
                       limit=5.0)
    check_close(got, ref, bf16_out=False, what=f"f8 pair32 T={T} spread={spread}")
    # the 16x16x128 kernel on the same layer
    monkeypatch.setenv(L.FP8_PREFILL_ENV, "v1")
    assert not L.fp8_pair32_use(W)
    v1 = _run(x, ids, wts, W, swiglu_limit=5.0)
    check_close(v1, ref, bf16_out=False, what=f"f8 v1 T={T}")


def test_deepseek_shape():
    """H 7168, I 2048 (56 and 16 scale blocks along k), a few experts."""
    E, NS, H, I, T, K = 6, 0, 7168, 2048, 160, 2
    d, W = _layer(E, NS, H, I, seed=60, spread=4)
    assert L.fp8_pair32_use(W)
    ids, wts = _routing(T, K, E, 61)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(62)).to(torch.bfloat16)
    ref = oracle_layer(FMT, dense_to_numpy(FMT, d), bf16_tensor_to_bits(x), ids, wts, E, NS, H, I)
    check_close(_run(x, ids, wts, W), ref, bf16_out=False, what="f8 pair32 7168x2048")


def test_slot_planes_follow_the_callers_statement():
    E, NS, H, I, K, T = 8, 0, 1024, 256, 2, 300
    d, W = _layer(E, NS, H, I, seed=70)
    perm = torch.tensor([5, 2, 7, 0, 3, 6, 1, 4], dtype=torch.int64)
    slots = ExpertWeights(FMT, H, I, E, 0, torch.empty_like(W.w13), torch.empty_like(W.s13),
                          torch.empty_like(W.w2), torch.empty_like(W.s2), mutable=True)
    for e in range(E):
        for name in ("w13", "s13", "w2", "s2"):
            getattr(slots, name)[perm[e]].copy_(getattr(W, name)[e])
    smap = perm.to(torch.int32).to(DEV)
    assert not L.fp8_pair32_use(slots) and L.fp8_pair32_use(slots, True)
    ids, wts = _routing(T, K, E, 71)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(72)).to(torch.bfloat16)
    ref = oracle_layer(FMT, dense_to_numpy(FMT, d), bf16_tensor_to_bits(x), ids, wts, E, NS, H, I)
    resident = _run(x, ids, wts, W)
    for ok in (True, False):
        got = _run(x, ids, wts, slots, slot_map=smap, fp8_scales_ok=ok)
        check_close(got, ref, bf16_out=False, what=f"slot planes scales_ok={ok}")
        if ok:   # the resident layer's kernel: the same bits
            assert np.array_equal(got, resident)


@pytest.mark.parametrize("bad", ["zero", "spread"])
def test_unbounded_scales_take_the_v1_kernel(bad):
    E, NS, H, I, T, K = 8, 0, 1024, 256, 64, 2
    d = make_dense_layer(FMT, E, H, I, seed=80)
    if bad == "zero":
        d["s13"][3, 1, 2] = 0.0
    else:
        d["s2"][2, 0, 0] *= 2.0 ** -40
    W = ExpertWeights.from_dense(FMT, d["w13"], d["s13"], d["w2"], d["s2"], device=DEV)
    assert not L.fp8_pair32_use(W)
    assert not L.fp8_block_scales_bounded(d["s13"], d["s2"])
    ids, wts = _routing(T, K, E, 81)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(82)).to(torch.bfloat16)
    ref = oracle_layer(FMT, dense_to_numpy(FMT, d), bf16_tensor_to_bits(x), ids, wts, E, NS, H, I)
    check_close(_run(x, ids, wts, W), ref, bf16_out=False, what=f"unbounded scales ({bad})")


@pytest.mark.parametrize("T,K,skew", [(1, 2, False), (700, 4, False), (900, 2, True)])
def test_fused_act_pairs_are_bitwise(monkeypatch, T, K, skew):
    """The gate/up epilogue writing the down pass's pairs
    (xtu_f8_pair_gate_up_q) gives the layer output bitwise equal to the bf16
    rows quantised by the separate kernel."""
    monkeypatch.setenv(L.FP8_PREFILL_ENV, "auto")
    E, NS, H, I = 16, 1, 1024, 512
    d, W = _layer(E, NS, H, I, seed=150 + T, spread=8)
    assert L.fp8_pair32_use(W)
    ids, wts = _routing(T, K, E, 151 + T, skew)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(152 + T)).to(torch.bfloat16)
    outs = []
    for fused in ("1", "0"):
        monkeypatch.setenv(L.ACT_QUANT_ENV, fused)
        outs.append(_run(x, ids, wts, W, swiglu_limit=5.0))
    assert np.array_equal(outs[0].view(np.int32), outs[1].view(np.int32))
