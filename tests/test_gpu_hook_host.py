"""The quant-method hook with layers whose experts stay in host memory.

A DeepSeek-V3-shaped FP8 layer (H=7168, I=2048, 256 experts, grouped sigmoid
top-8) that the residency policy keeps off the GPU: the hook packs it on the
host into pinned shards (no device copy) with a 64-expert hot pool; device
memory grows by the pool, then by the tile ring allocated up front
(prealloc_fp8_buffers), then by the call's scratch only -- a second long
prefill allocates nothing but its output.  Per call: T=4 runs the pin split
(pool experts on the GPU, the others on the host engine), T=8192 streams the
layer through the preallocated ring; both against the oracle (for T=8192 a
set of tokens covering every routed expert).  A smaller MXFP4 layer without
a pool runs the host engine alone at decode sizes and the ring (shared
experts none) at prefill sizes."""
import types

import numpy as np
import pytest
import torch

from helpers import bf16_tensor_to_bits, check_close, cover_tokens, threaded_oracle
from xtu_moe_amd import formats as F
from xtu_moe_amd import host_layer as HL
from xtu_moe_amd import ring as R
from xtu_moe_amd.layer import route
from xtu_moe_amd.mixed_experts import XiaotuExpertsFp8, XiaotuExpertsMxfp4

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _host_dense(fmt, E, H, I, seed, chunk=8):
    """Dense checkpoint tensors of E experts in host memory (drawn N(0, 0.02)
    and quantised on the device chunk by chunk)."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    out = {}
    for name, N, K in (("13", 2 * I, H), ("2", H, I)):
        w = s = None
        for e0 in range(0, E, chunk):
            e1 = min(E, e0 + chunk)
            q, sc, _ = F.quantize(fmt, torch.randn((e1 - e0, N, K), generator=g, device=DEV) * 0.02)
            if w is None:
                w = torch.empty((E,) + tuple(q.shape[1:]), dtype=q.dtype)
                s = torch.empty((E,) + tuple(sc.shape[1:]), dtype=sc.dtype)
            w[e0:e1].copy_(q)
            s[e0:e1].copy_(sc)
        out["w" + name], out["s" + name] = w, s
    return out


def _layer(d, scale_names, idx, **kw):
    return types.SimpleNamespace(layer_name=f"model.layers.{idx}.mlp.experts",
                                 w13_weight=d["w13"], w2_weight=d["w2"],
                                 **{scale_names[0]: d["s13"], scale_names[1]: d["s2"]}, **kw)


def _np(d):
    return {"w13": d["w13"].numpy(), "s13": d["s13"].numpy(), "w2": d["w2"].numpy(),
            "s2": d["s2"].numpy(), "gs13": None, "gs2": None}


def test_ds_v3_fp8_host_resident_through_the_hook(monkeypatch):
    H, I, E, K = 7168, 2048, 256, 8
    monkeypatch.setenv(HL.RESIDENT_LAYERS_ENV, "0-2")     # layer 3 stays in host memory
    monkeypatch.setenv(HL.PIN_SLOTS_ENV, "64")
    monkeypatch.delenv(HL.PREFILL_MIN_ENV, raising=False)
    d = _host_dense(F.FMT_FP8, E, H, I, seed=61)
    print("dense layer on the host", flush=True)
    layer = _layer(d, ("w13_weight_scale_inv", "w2_weight_scale_inv"), 3, top_k=K,
                   use_grouped_topk=True, scoring_func="sigmoid", renormalize=True,
                   num_expert_group=8, topk_group=4, routed_scaling_factor=2.5)
    hook = XiaotuExpertsFp8()
    torch.cuda.synchronize()
    m0 = torch.cuda.memory_allocated()
    hook.process_weights_after_loading(layer)
    torch.cuda.synchronize()
    m1 = torch.cuda.memory_allocated()
    hl = hook._host_layer
    assert hook._weights is None and hl is not None and hl.pool.nslots == 64
    assert m1 - m0 <= hl.device_bytes() + (16 << 20), (m1 - m0, hl.device_bytes())
    assert hl.store.pin_hostbufs() >= 2
    print(f"packed on the host; device grew {(m1 - m0) / 2**20:.0f} MiB", flush=True)
    ring_bytes = R.prealloc_fp8_buffers(DEV, E, H, I)
    torch.cuda.synchronize()
    m2 = torch.cuda.memory_allocated()
    assert ring_bytes == R.staging_bytes(E, H, I, ns=2, fmt=F.FMT_FP8)
    assert m2 - m1 <= ring_bytes + (1 << 20)
    ring = R._ring_for(F.FMT_FP8, H, I, R.staging_tile_experts(E), 2, DEV)
    ptrs = [sl.w13.data_ptr() for sl in ring.slots]
    dn = _np(d)
    g = torch.Generator(device=DEV).manual_seed(62)

    # decode: the pin split
    T = 4
    x = torch.randn((T, H), generator=g, device=DEV).to(torch.bfloat16)
    logits = torch.randn((T, E), generator=g, device=DEV)
    wts, ids = route(logits, top_k=K, scoring="sigmoid", n_group=8, topk_group=4,
                     routed_scaling_factor=2.5)
    out = hook.apply(x, None, None, topk_weights=wts, topk_ids=ids)
    torch.cuda.synchronize()
    assert hl.last_path == "split" and out.dtype == torch.bfloat16
    ids_np, wts_np = ids.cpu().numpy(), wts.cpu().numpy()
    assert np.isin(ids_np, np.arange(64)).any() and (~np.isin(ids_np, np.arange(64))).any()
    ref = threaded_oracle(F.FMT_FP8, dn, bf16_tensor_to_bits(x), ids_np, wts_np, E, 0, H, I)
    check_close(out.float().cpu().numpy(), ref, bf16_out=True, what="host-resident T=4 split")
    mono = hook.apply(x, None, None, router_logits=logits)   # routes itself, same experts
    torch.cuda.synchronize()
    assert torch.equal(mono, out)
    print("T=4 split ok", flush=True)

    # prefill: the preallocated ring
    T = 8192
    x = torch.randn((T, H), generator=g, device=DEV).to(torch.bfloat16)
    logits = torch.randn((T, E), generator=g, device=DEV)
    wts, ids = route(logits, top_k=K, scoring="sigmoid", n_group=8, topk_group=4,
                     routed_scaling_factor=2.5)
    torch.cuda.synchronize()
    m3 = torch.cuda.memory_allocated()
    out = hook.apply(x, None, None, topk_weights=wts, topk_ids=ids)
    torch.cuda.synchronize()
    m4 = torch.cuda.memory_allocated()
    assert hl.last_path == "ring"
    assert [sl.w13.data_ptr() for sl in ring.slots] == ptrs   # the preallocated ring
    A = T * K
    scratch = (A * H * 4 + A * I * 2 + A * (2 * I + I // 32) + T * (2 * H + H // 32)
               + T * H * (4 + 2) + (64 << 20))
    assert m4 - m3 <= scratch, (m4 - m3, scratch)
    out2 = hook.apply(x, None, None, topk_weights=wts, topk_ids=ids)
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() - m4 <= T * H * 2 + (8 << 20)   # its output only
    assert torch.equal(out2, out)
    toks, covered = cover_tokens(ids.cpu().numpy(), E, seed=63)
    assert len(covered) == len(set(ids.flatten().tolist()))
    ids_np, wts_np = ids.cpu().numpy()[toks], wts.cpu().numpy()[toks]
    ref = threaded_oracle(F.FMT_FP8, dn, bf16_tensor_to_bits(x[toks]), ids_np, wts_np, E, 0, H, I)
    check_close(out[toks].float().cpu().numpy(), ref, bf16_out=True,
                what="host-resident T=8192 ring")
    print(f"T=8192 ring ok ({len(toks)} tokens over {len(covered)} experts)", flush=True)


def test_host_resident_without_pool_host_engine_and_ring(monkeypatch):
    H, I, E, K = 1024, 512, 64, 6
    monkeypatch.setenv(HL.RESIDENT_LAYERS_ENV, "5")
    monkeypatch.delenv(HL.PIN_SLOTS_ENV, raising=False)
    monkeypatch.setenv(HL.PREFILL_MIN_ENV, "100")
    d = _host_dense(F.FMT_MXFP4, E, H, I, seed=64)
    layer = _layer(d, ("w13_weight_scale", "w2_weight_scale"), 7, top_k=K, renormalize=True,
                   swiglu_limit=7.0)
    hook = XiaotuExpertsMxfp4()
    hook.process_weights_after_loading(layer)
    hl = hook._host_layer
    assert hook._weights is None and hl is not None and hl.pool is None
    dn = _np(d)
    g = torch.Generator(device=DEV).manual_seed(65)
    for T, path in ((3, "host"), (300, "ring")):
        x = torch.randn((T, H), generator=g, device=DEV).to(torch.bfloat16)
        logits = torch.randn((T, E), generator=g, device=DEV)
        out = hook.apply(x.float(), None, None, router_logits=logits)   # fp32 hidden states
        torch.cuda.synchronize()
        assert hl.last_path == path and out.dtype == torch.float32
        wts, ids = route(logits, top_k=K, scoring="softmax", renormalize=True)
        ref = threaded_oracle(F.FMT_MXFP4, dn, bf16_tensor_to_bits(x), ids.cpu().numpy(),
                              wts.cpu().numpy(), E, 0, H, I, limit=7.0)
        check_close(out.cpu().numpy(), ref, bf16_out=False, what=f"host-resident {path} T={T}")
    # the reference's "0": the ring is off, every batch takes the host engine
    monkeypatch.setenv(HL.PREFILL_MIN_ENV, "0")
    x = torch.randn((2, H), generator=g, device=DEV).to(torch.bfloat16)
    out = hook.apply(x, None, None, router_logits=torch.randn((2, E), generator=g, device=DEV))
    torch.cuda.synchronize()
    assert hl.last_path == "host"
