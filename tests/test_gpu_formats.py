"""Checkpoint formats at the hook boundary, on the GPU.

* INT4 (WNA16): a GPTQ-layout layer (int32 qweight, fp16 scales [E, G, N],
  symmetric qzeros) through XiaotuExpertsInt4.apply with device tensors: the
  host engine behind the cpu_decode bridge for batches inside the pre-sized
  staging, the synchronous host forward beyond it; both against the oracle.
  The bridged apply captured in a HIP graph replays bit-identically.
* NVFP4: weight_scale_2 given as [E, 2] (gate, up) equal gives the same
  layer as [E]; gate and up scales that differ (w1 / w3 quantised apart) are
  applied per half, on the resident decode and prefill paths and on a
  host-resident layer's host engine, against the oracle.
"""
import numpy as np
import pytest
import torch

from helpers import (bf16_tensor_to_bits, check_close, dense_to_numpy, int4_layer,
                     make_dense_layer, oracle_layer, random_routing)
from xtu_moe_amd import formats as F
from xtu_moe_amd.mixed_experts import XiaotuExpertsInt4, XiaotuExpertsNvfp4

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _inputs(T, K, E, H, seed):
    ids, wts = random_routing(T, K, E, seed=seed)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)
    return x, ids, wts


def test_int4_hook_on_device_tensors(monkeypatch):
    monkeypatch.setenv("XTU_CD_PREALLOC_TOKENS", "32")
    E, H, I, K = 12, 512, 256, 3
    d, layer = int4_layer(E, H, I, seed=21)
    hook = XiaotuExpertsInt4(quant_config=type("Q", (), {"group_size": 128, "desc_act": False}))
    hook.process_weights_after_loading(layer)
    dn = dense_to_numpy(F.FMT_INT4, d)
    for T in (1, 24, 80):       # 80 > 32 staged rows: the synchronous host forward
        x, ids, wts = _inputs(T, K, E, H, seed=T)
        out = torch.empty((T, H), dtype=torch.bfloat16, device=DEV)
        got = hook.apply(x.to(DEV), None, None, output=out,
                         topk_ids=torch.from_numpy(ids).to(DEV),
                         topk_weights=torch.from_numpy(wts).to(DEV))
        torch.cuda.synchronize()
        assert got.data_ptr() == out.data_ptr()
        ref = oracle_layer(F.FMT_INT4, dn, bf16_tensor_to_bits(x), ids, wts, E, 0, H, I,
                           limit=7.0)
        check_close(out.float().cpu().numpy(), ref, bf16_out=True, what=f"int4 hook T={T}")


def test_int4_hook_replays_in_a_graph(monkeypatch):
    monkeypatch.setenv("XTU_CD_PREALLOC_TOKENS", "16")
    E, H, I, K, T = 8, 512, 256, 3, 5
    d, layer = int4_layer(E, H, I, seed=22)
    hook = XiaotuExpertsInt4(quant_config=type("Q", (), {"group_size": 128, "desc_act": False}))
    hook.process_weights_after_loading(layer)
    sx = torch.zeros((T, H), dtype=torch.bfloat16, device=DEV)
    sids = torch.zeros((T, K), dtype=torch.int32, device=DEV)
    sw = torch.zeros((T, K), dtype=torch.float32, device=DEV)
    sout = torch.zeros((T, H), dtype=torch.bfloat16, device=DEV)
    batches = [_inputs(T, K, E, H, seed=30 + i) for i in range(3)]
    run = lambda: hook.apply(sx, None, None, output=sout, topk_ids=sids, topk_weights=sw)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    torch.cuda.synchronize()
    for i, (x, ids, wts) in enumerate(batches):
        sx.copy_(x.to(DEV))
        sids.copy_(torch.from_numpy(ids))
        sw.copy_(torch.from_numpy(wts))
        g.replay()
        torch.cuda.synchronize()
        got = sout.clone()
        eager = hook.apply(x.to(DEV), None, None, topk_ids=torch.from_numpy(ids).to(DEV),
                           topk_weights=torch.from_numpy(wts).to(DEV))
        torch.cuda.synchronize()
        assert torch.equal(got, eager), f"replay {i}"
    del g


def _nvfp4_layer(d, K, g13):
    P = lambda t: torch.nn.Parameter(t, requires_grad=False)
    return type("L", (), dict(w13_weight=P(d["w13"]), w2_weight=P(d["w2"]),
                              w13_weight_scale=P(d["s13"]), w2_weight_scale=P(d["s2"]),
                              w13_weight_scale_2=P(g13), w2_weight_scale_2=P(d["gs2"]),
                              top_k=K, renormalize=True))()


def test_nvfp4_second_level_scales_two_columns():
    E, H, I, T, K = 8, 512, 256, 20, 2
    d = make_dense_layer(F.FMT_NVFP4, E, H, I, seed=23)
    x, ids, wts = _inputs(T, K, E, H, seed=24)
    outs = []
    for g13 in (d["gs13"], torch.stack([d["gs13"], d["gs13"]], 1)):
        hook = XiaotuExpertsNvfp4()
        hook.process_weights_after_loading(_nvfp4_layer(d, K, g13))
        outs.append(hook.apply(x.to(DEV), None, None, topk_ids=torch.from_numpy(ids).to(DEV),
                               topk_weights=torch.from_numpy(wts).to(DEV)))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    ref = oracle_layer(F.FMT_NVFP4, dense_to_numpy(F.FMT_NVFP4, d), bf16_tensor_to_bits(x), ids,
                       wts, E, 0, H, I)
    check_close(outs[1].float().cpu().numpy(), ref, bf16_out=True, what="nvfp4 [E,2] scale_2")


@pytest.mark.parametrize("resident", ["1", ""])
@pytest.mark.parametrize("T", [3, 300])
def test_nvfp4_unequal_gate_up_scales(monkeypatch, resident, T):
    """w1 / w3 second-level scales that differ (about 3x here): each half
    takes its own, on the decode (T = 3) and grouped-GEMM (T = 300) paths of
    a resident layer, and through a host-resident layer (host engine at
    T = 3, the tile ring at T = 300)."""
    monkeypatch.setenv("XIAOTU_MOE_GPU_RESIDENT_LAYERS", resident or "99")
    monkeypatch.setenv("VLLM_XIAOTU_GPU_PREFILL_MIN_TOKENS", "256")
    monkeypatch.setenv("XTU_CD_PREALLOC_TOKENS", "16")
    E, H, I, K = 8, 512, 256, 2
    d = make_dense_layer(F.FMT_NVFP4, E, H, I, seed=25, split_gate_up=True)
    g13 = d["gs13"]
    assert g13.shape == (E, 2) and bool((g13[:, 1] > 2 * g13[:, 0]).all())
    layer = _nvfp4_layer(d, K, g13)
    layer.layer_name = "model.layers.1.mlp.experts"
    hook = XiaotuExpertsNvfp4()
    hook.process_weights_after_loading(layer)
    assert (hook._host_layer is None) == bool(resident)
    x, ids, wts = _inputs(T, K, E, H, seed=26)
    out = hook.apply(x.to(DEV), None, None, topk_ids=torch.from_numpy(ids).to(DEV),
                     topk_weights=torch.from_numpy(wts).to(DEV))
    torch.cuda.synchronize()
    if not resident:
        assert hook._host_layer.last_path == ("ring" if T >= 256 else "host")
    dn = dense_to_numpy(F.FMT_NVFP4, d)
    ref = oracle_layer(F.FMT_NVFP4, dn, bf16_tensor_to_bits(x), ids, wts, E, 0, H, I)
    check_close(out.float().cpu().numpy(), ref, bf16_out=True, what=f"nvfp4 unequal T={T}")
    # one scale for both halves would be a wrong answer this test sees
    dn1 = dict(dn, gs13=dn["gs13"][:, 0].copy())
    wrong = oracle_layer(F.FMT_NVFP4, dn1, bf16_tensor_to_bits(x), ids, wts, E, 0, H, I)
    assert float(np.abs(wrong - ref).max()) > 10 * float(np.abs(out.float().cpu().numpy() - ref).max())
