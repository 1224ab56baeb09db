"""Host expert engine (the CPU half of the pool-miss split) against the
oracle, on the CPU: every format, one and two NUMA-node shards, the AVX-512
and the portable kernels, invalid ids / zero weights / an expert listed
twice by one token, and bit-identical results for any thread count (each
output element is summed in a fixed order)."""
import types

import numpy as np
import pytest
import torch

from helpers import (bf16_tensor_to_bits, check_close, dense_to_numpy, gptq_pack, int4_dense,
                     int4_layer, make_dense_layer, unpack_nibbles)
import oracle
from xtu_moe_amd import formats as F
from xtu_moe_amd.cpu_experts import ISA_AVX512, ISA_PORTABLE, CpuExperts
from xtu_moe_amd.host_store import HostExpertStore
from xtu_moe_amd.layer import ExpertWeights

FMTS = [F.FMT_BF16, F.FMT_FP8, F.FMT_MXFP4, F.FMT_NVFP4, F.FMT_INT4]
E, H, I = 6, 256, 256


def _avx512_ok():
    try:
        flags = open("/proc/cpuinfo").read()
        return all(f in flags for f in ("avx512f", "avx512bw", "avx512dq", "avx512vl"))
    except OSError:
        return False


ISAS = [ISA_PORTABLE] + ([ISA_AVX512] if _avx512_ok() else [])


def _layer(fmt, seed=0, std=0.05):
    d = make_dense_layer(fmt, E, H, I, seed=seed, std=std)
    W = ExpertWeights.from_dense(fmt, d["w13"], d["s13"], d["w2"], d["s2"], d["gs13"], d["gs2"],
                                 E=E, device="cpu")
    return W, dense_to_numpy(fmt, d)


def _batch(T, K, seed):
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    wts = (rng.random((T, K)) + 0.05).astype(np.float32)
    ids[0, -1] = ids[0, 0]                       # one token lists an expert twice
    if T > 2:
        ids[1, 0], ids[2, 1] = -1, E + 2          # invalid ids add nothing
        wts[2, 0] = 0.0                           # nor do zero weights
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn((T, H), generator=g)).to(torch.bfloat16)
    return x, ids, wts


def _oracle(fmt, dn, x, ids, wts, limit=0.0):
    ok = (ids >= 0) & (ids < E)
    return oracle.moe_layer(fmt, bf16_tensor_to_bits(x), np.where(ok, ids, -1).astype(np.int32),
                            np.where(ok, wts, 0).astype(np.float32), E, 0, H, I, dn["w13"],
                            dn["s13"], dn["w2"], dn["s2"], dn["gs13"], dn["gs2"], limit=limit)


@pytest.mark.parametrize("isa", ISAS)
@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("ns", [1, 2])
def test_host_engine_matches_oracle(fmt, ns, isa):
    W, dn = _layer(fmt, seed=fmt)
    store = HostExpertStore.from_weights(W, ns=ns, pin=False)
    limit = 7.0 if fmt == F.FMT_MXFP4 else 0.0
    eng = CpuExperts.from_store(store, isa=isa, n_threads=4, swiglu_limit=limit)
    try:
        assert eng.isa == isa
        for T, K in ((1, 2), (5, 4), (9, 3)):
            x, ids, wts = _batch(T, K, seed=T)
            out = eng.forward(x, torch.from_numpy(ids), torch.from_numpy(wts))
            ref = _oracle(fmt, dn, x, ids, wts, limit=limit)
            check_close(out.numpy(), ref, bf16_out=False,
                        what=f"{F.FMT_NAMES[fmt]} ns={ns} isa={isa} T={T}")
    finally:
        eng.close()


@pytest.mark.parametrize("fmt", [F.FMT_MXFP4, F.FMT_FP8])
def test_thread_count_does_not_change_bits(fmt):
    W, _ = _layer(fmt, seed=3)
    x, ids, wts = _batch(7, 4, seed=11)
    outs = []
    for thr in (1, 3, 8):
        eng = CpuExperts.from_weights(W, n_threads=thr)
        try:
            outs.append(eng.forward(x, torch.from_numpy(ids), torch.from_numpy(wts)))
        finally:
            eng.close()
    assert all(torch.equal(outs[0], o) for o in outs[1:])


def test_no_valid_pairs_gives_zeros_and_bad_layouts_are_refused():
    W, _ = _layer(F.FMT_MXFP4)
    eng = CpuExperts.from_weights(W, n_threads=2)
    try:
        x = torch.ones((3, H), dtype=torch.bfloat16)
        out = torch.full((3, H), 5.0)
        eng.forward(x, torch.full((3, 2), -1, dtype=torch.int32), torch.ones((3, 2)), out=out)
        assert torch.count_nonzero(out) == 0
        with pytest.raises(ValueError):   # out must be fp32 [T, H]
            eng.forward(x, torch.zeros((3, 2), dtype=torch.int32), torch.ones((3, 2)),
                        out=torch.empty((3, H + 16)))
        # a host-only engine has no staging for the stream bridge
        assert eng.cpu_decode(None, 3, 2, 0, 0, 0, 0) == -2
    finally:
        eng.close()
    with pytest.raises(ValueError):       # shards must hold whole 16-row panels
        HostExpertStore.from_weights(W, ns=3, pin=False)
    w13 = W.w13.contiguous()
    with pytest.raises(RuntimeError):     # NVFP4 needs its global scales
        CpuExperts(F.FMT_NVFP4, H, I, E, [w13], [W.w2.contiguous()], W.s13, W.s2, None, None)


# --------------------------------------------------------------- INT4 / WNA16
@pytest.mark.parametrize("group", [32, 64])
def test_int4_groups_host_engine(group):
    d = int4_dense(E, H, I, group, seed=group)
    W = ExpertWeights.from_dense(F.FMT_INT4, d["w13"], d["s13"], d["w2"], d["s2"], E=E,
                                 device="cpu")
    assert W.group_k == group
    dn = dense_to_numpy(F.FMT_INT4, d)
    for isa in ISAS:
        eng = CpuExperts.from_weights(W, isa=isa, n_threads=3)
        try:
            x, ids, wts = _batch(6, 3, seed=group)
            out = eng.forward(x, torch.from_numpy(ids), torch.from_numpy(wts))
            check_close(out.numpy(), _oracle(F.FMT_INT4, dn, x, ids, wts), bf16_out=False,
                        what=f"int4 group {group} isa {isa}")
        finally:
            eng.close()


def test_gptq_repack_and_zero_points():
    from xtu_moe_amd.mixed_experts import repack_gptq_int4, require_symmetric_zero_points
    d = int4_dense(3, 256, 128, 128, seed=2)
    codes = unpack_nibbles(d["w13"])                     # [E, 2I, H]
    qw = gptq_pack(codes)                        # [E, H/8, 2I]
    w, s = repack_gptq_int4(qw, d["s13"].transpose(1, 2).contiguous())
    assert torch.equal(w, d["w13"]) and torch.equal(s, d["s13"])
    ok = types.SimpleNamespace(w13_qzeros=torch.full((3, 2, 32), 0x77777777, dtype=torch.int32))
    require_symmetric_zero_points(ok, ("w13_qzeros",))
    bad = types.SimpleNamespace(w13_qzeros=torch.full((3, 2, 32), 0x77777775, dtype=torch.int32))
    with pytest.raises(NotImplementedError):
        require_symmetric_zero_points(bad, ("w13_qzeros",))


def test_int4_hook_on_host_tensors_matches_oracle():
    from xtu_moe_amd.mixed_experts import XiaotuExpertsInt4
    d, layer = int4_layer(E, H, I, seed=5)
    hook = XiaotuExpertsInt4(quant_config=types.SimpleNamespace(group_size=128, desc_act=False))
    hook.process_weights_after_loading(layer)
    x, ids, wts = _batch(5, 3, seed=8)
    out = hook.apply(x, None, None, topk_ids=torch.from_numpy(ids),
                     topk_weights=torch.from_numpy(wts))
    assert out.dtype == torch.bfloat16 and tuple(out.shape) == (5, H)
    ref = _oracle(F.FMT_INT4, dense_to_numpy(F.FMT_INT4, d), x, ids, wts, limit=7.0)
    check_close(out.float().numpy(), ref, bf16_out=True, what="int4 hook")
    with pytest.raises(NotImplementedError):
        XiaotuExpertsInt4(quant_config=types.SimpleNamespace(group_size=128, desc_act=True)
                          ).process_weights_after_loading(layer)


def test_wna16_engine_forward_many():
    from xtu_moe_amd.engine import MOE_WNA16, MOEConfigV2
    d = int4_dense(E, H, I, 128, seed=9)
    cfg = MOEConfigV2(expert_num=E, top_k=3, hidden_size=H, intermediate_size=I, groupN=1,
                      groupK=128)
    eng = MOE_WNA16(cfg, d["w13"], d["w2"], d["s13"], d["s2"])
    x, ids, wts = _batch(4, 3, seed=10)
    out = torch.empty((4, H))
    eng.forward_many(4, 3, torch.from_numpy(ids), torch.from_numpy(wts), x, out)
    check_close(out.numpy(), _oracle(F.FMT_INT4, dense_to_numpy(F.FMT_INT4, d), x, ids, wts),
                bf16_out=False, what="MOE_WNA16.forward_many")


def test_nvfp4_second_level_scales():
    """w13's scale_2 comes out as [E, 2] (gate, up) whatever the checkpoint
    gives, w1 / w3 scales that differ included; all zero is refused."""
    from xtu_moe_amd.mixed_experts import nvfp4_global_scales
    g2 = torch.tensor([0.5, 2.0])
    a, b = nvfp4_global_scales(torch.tensor([[0.5, 0.5], [1.5, 1.5]]), g2)
    assert torch.equal(a, torch.tensor([[0.5, 0.5], [1.5, 1.5]])) and torch.equal(b, g2)
    a, _ = nvfp4_global_scales(torch.tensor([0.25, 4.0]), g2)
    assert torch.equal(a, torch.tensor([[0.25, 0.25], [4.0, 4.0]]))
    a, _ = nvfp4_global_scales(torch.tensor([[0.5, 0.5], [1.5, 1.0]]), g2)
    assert torch.equal(a, torch.tensor([[0.5, 0.5], [1.5, 1.0]]))
    with pytest.raises(ValueError):            # neither [E] nor [E, 2]
        nvfp4_global_scales(torch.ones(2, 3), g2)
    with pytest.raises(RuntimeError):          # not loaded
        nvfp4_global_scales(torch.zeros(2, 2), g2)


def test_host_engine_nvfp4_unequal_gate_up_scales():
    """The host engine takes the gate panels' scale_2 from column 0 and the
    up panels' from column 1 (the reference folds each into its half's
    group scales, hybrid_model.py:1546-1563), against the oracle and the
    reference engine over the folded scales."""
    d = make_dense_layer(F.FMT_NVFP4, E, H, I, seed=31, split_gate_up=True)
    assert d["gs13"].shape == (E, 2) and bool((d["gs13"][:, 1] > 2 * d["gs13"][:, 0]).all())
    W = ExpertWeights.from_dense(F.FMT_NVFP4, d["w13"], d["s13"], d["w2"], d["s2"], d["gs13"],
                                 d["gs2"], device="cpu")
    eng = CpuExperts.from_weights(W)
    x, ids, wts = _batch(5, 2, seed=32)
    out = eng.forward(x, torch.from_numpy(ids), torch.from_numpy(wts))
    dn = dense_to_numpy(F.FMT_NVFP4, d)
    ref = _oracle(F.FMT_NVFP4, dn, x, ids, wts)
    check_close(out.numpy(), ref, bf16_out=False, what="host engine, unequal scale_2")
    if oracle.ref_available():
        r = oracle.RefEngine(F.FMT_NVFP4, E, 2, H, I, dn["w13"], dn["s13"], dn["w2"], dn["s2"],
                             dn["gs13"], dn["gs2"])
        got = r.forward(bf16_tensor_to_bits(x), ids, wts)
        check_close(got, ref, bf16_out=False, what="reference engine, folded scale_2")
