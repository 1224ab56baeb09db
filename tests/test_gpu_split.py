"""Pool-miss split on the GPU: pool-resident experts (and the shared ones) on
the device, every other routed expert on the host engine through the
graph-capturable cpu_decode bridge, the two results added.

* the pin mask bit for bit against its definition (numpy);
* cpu_decode (device -> pinned -> host-function node -> device) equals the
  host engine's direct forward bit for bit, also through the engine object
  with the reference's pointer arguments, and grows its staging outside a
  capture;
* the split layer against the oracle's whole layer, four formats, T = 1, 4,
  24, with a SwiGLU limit, before and after a swap;
* the split layer captured in a HIP graph: every replay (new inputs copied
  into the static buffers, eager work between replays) equals the eager
  split layer on the same inputs bit for bit."""
import numpy as np
import pytest
import torch

from helpers import (bf16_tensor_to_bits, check_close, dense_to_numpy, make_dense_layer,
                     oracle_layer, random_routing)
from xtu_moe_amd import formats as F
from xtu_moe_amd import gpu_prefill as GP
from xtu_moe_amd.cpu_experts import CpuExperts
from xtu_moe_amd.cpu_split import PoolSplitLayer, pin_split
from xtu_moe_amd.engine import MOE_MXFP4, MOEConfigV2
from xtu_moe_amd.expert_pool import LayerPool
from xtu_moe_amd.host_store import HostExpertStore
from xtu_moe_amd.layer import ExpertWeights

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
LAYOUT = {F.FMT_BF16: "bf16", F.FMT_FP8: "fp8", F.FMT_MXFP4: "mxfp4", F.FMT_NVFP4: "nvfp4"}
GROUP_K = {F.FMT_BF16: 1, F.FMT_FP8: 128, F.FMT_MXFP4: 32, F.FMT_NVFP4: 16}


def _layer(fmt, E, NS, H, I, seed):
    d = make_dense_layer(fmt, E + NS, H, I, seed=seed)
    W = ExpertWeights.from_dense(fmt, d["w13"], d["s13"], d["w2"], d["s2"], d["gs13"], d["gs2"],
                                 n_shared=NS, device=DEV)
    return d, W


def _inputs(T, K, E, H, seed):
    ids, wts = random_routing(T, K, E, seed=seed)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((T, H), generator=g).to(torch.bfloat16)
    return x.to(DEV), torch.from_numpy(ids).to(DEV), torch.from_numpy(wts).to(DEV)


def _oracle(fmt, d, x, ids, wts, E, NS, H, I, limit=0.0):
    return oracle_layer(fmt, dense_to_numpy(fmt, d), bf16_tensor_to_bits(x),
                        ids.cpu().numpy(), wts.cpu().numpy(), E, NS, H, I, limit=limit)


def test_pin_split_definition():
    rng = np.random.default_rng(0)
    n_local, n = 40, 700
    sm = np.arange(n_local, dtype=np.int32)
    res = rng.choice(n_local, 9, replace=False)
    sm[res] = n_local + np.arange(9)
    ids = rng.integers(-3, n_local + 4, n).astype(np.int32)
    wts = rng.random(n).astype(np.float32)
    hits = torch.zeros((), dtype=torch.int64, device=DEV)
    got = pin_split(torch.from_numpy(ids).to(DEV), torch.from_numpy(wts).to(DEV),
                    torch.from_numpy(sm).to(DEV), n_local, hits=hits)
    bad = (ids < 0) | (ids >= n_local)
    sl = sm[np.where(bad, 0, ids)]
    r = ~bad & (sl >= n_local)
    want = (np.where(r | bad, 0, ids), np.where(r | bad, 0, wts), np.where(r, sl - n_local, -1),
            np.where(r, wts, 0))
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g.cpu().numpy(), w.astype(g.cpu().numpy().dtype))
    assert int(hits) == int(r.sum())


@pytest.mark.parametrize("fmt", [F.FMT_MXFP4, F.FMT_FP8])
def test_cpu_decode_equals_host_forward(fmt):
    E, NS, H, I, T, K = 12, 0, 512, 256, 9, 4
    d, W = _layer(fmt, E, NS, H, I, seed=2)
    store = HostExpertStore.from_weights(W, ns=2)
    eng = CpuExperts.from_store(store, max_tokens=16, max_topk=K, n_threads=8)
    try:
        x, ids, wts = _inputs(T, K, E, H, seed=3)
        out = torch.full((T, H), float("nan"), device=DEV)
        assert eng.cpu_decode(None, T, K, x, ids, wts, out) == 0
        torch.cuda.synchronize()    # the queued call and a direct one share the engine
        host = eng.forward(x.cpu(), ids.cpu(), wts.cpu())
        assert torch.equal(out.cpu(), host)
        check_close(host.numpy(), _oracle(fmt, d, x, ids, wts, E, NS, H, I), bf16_out=False,
                    what="host engine")
        # the reference's error codes: out too small, staging too small
        assert eng.cpu_decode(None, T, K, x, ids, wts, out[:T - 1]) == -1
        assert eng.cpu_decode(None, 17, K, x, ids, wts, torch.empty((17, H), device=DEV)) == -2
    finally:
        torch.cuda.synchronize()
        eng.close()


def test_engine_cpu_decode_with_pointers_and_growth():
    E, H, I, K = 8, 512, 256, 2
    d = make_dense_layer(F.FMT_MXFP4, E, H, I, seed=4)
    cfg = MOEConfigV2(expert_num=E, top_k=K, hidden_size=H, intermediate_size=I)
    eng = MOE_MXFP4(cfg, d["w13"], d["w2"], d["s13"], d["s2"], device=DEV)
    eng.prepare_decode_buffers(8, K)
    stream = torch.cuda.current_stream()
    for T in (3, 70):    # 70 tokens grow the staging (outside a capture)
        x, ids, wts = _inputs(T, K, E, H, seed=T)
        out = torch.empty((T, H), device=DEV)
        rc = eng.cpu_decode(stream.cuda_stream, T, K, x.data_ptr(), ids.data_ptr(),
                            wts.data_ptr(), out.data_ptr(), layer=0)
        assert rc == 0
        torch.cuda.synchronize()
        check_close(out.cpu().numpy(), _oracle(F.FMT_MXFP4, d, x, ids, wts, E, 0, H, I),
                    bf16_out=False, what=f"engine cpu_decode T={T}")
    assert len(eng._cpu) == 2 and eng._cpu[-1].max_tokens >= 70


@pytest.mark.parametrize("fmt", [F.FMT_MXFP4, F.FMT_FP8, F.FMT_NVFP4, F.FMT_BF16])
def test_split_layer_matches_oracle(fmt):
    E, NS, H, I, K = 16, 1, 512, 256, 4
    limit = 7.0 if fmt == F.FMT_MXFP4 else 0.0
    d, W = _layer(fmt, E, NS, H, I, seed=10 + fmt)
    store = HostExpertStore.from_weights(W)
    pool = LayerPool(store, DEV, H, I, GROUP_K[fmt], E, [1, 5, 6, 11, 14], 0, layout=LAYOUT[fmt])
    cpu = CpuExperts.from_store(store, swiglu_limit=limit, max_tokens=32, max_topk=K)
    split = PoolSplitLayer(pool, cpu)
    try:
        for T in (1, 4, 24):
            x, ids, wts = _inputs(T, K, E, H, seed=20 + T)
            out = split.forward(x, ids, wts, swiglu_limit=limit)
            torch.cuda.synchronize()
            check_close(out.cpu().numpy(), _oracle(fmt, d, x, ids, wts, E, NS, H, I, limit),
                        bf16_out=False, what=f"{F.FMT_NAMES[fmt]} split T={T}")
        # a swap moves expert 3 from the host to the pool; the sum is unchanged in meaning
        pool.swap_out(2)
        pool.swap_in(GP, 3, 2)
        x, ids, wts = _inputs(12, K, E, H, seed=99)
        out = split.forward(x, ids, wts, swiglu_limit=limit)
        torch.cuda.synchronize()
        check_close(out.cpu().numpy(), _oracle(fmt, d, x, ids, wts, E, NS, H, I, limit),
                    bf16_out=False, what=f"{F.FMT_NAMES[fmt]} split after a swap")
        assert split.mask.hits().item() > 0
    finally:
        torch.cuda.synchronize()
        cpu.close()


def test_split_layer_replays_in_a_graph():
    fmt, E, NS, H, I, K, T = F.FMT_MXFP4, 16, 1, 512, 256, 4, 6
    d, W = _layer(fmt, E, NS, H, I, seed=31)
    store = HostExpertStore.from_weights(W)
    pool = LayerPool(store, DEV, H, I, 32, E, [0, 3, 8, 9], 0)
    cpu = CpuExperts.from_store(store, max_tokens=T, max_topk=K)
    split = PoolSplitLayer(pool, cpu)
    sx = torch.zeros((T, H), dtype=torch.bfloat16, device=DEV)
    sids = torch.zeros((T, K), dtype=torch.int32, device=DEV)
    sw = torch.zeros((T, K), dtype=torch.float32, device=DEV)
    sout = torch.zeros((T, H), dtype=torch.float32, device=DEV)
    try:
        batches = [_inputs(T, K, E, H, seed=40 + i) for i in range(4)]
        # warm-up (buffers of the mask and the layer exist before capture)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for b in batches[:2]:
                for dst, src in zip((sx, sids, sw), b):
                    dst.copy_(src)
                split.forward(sx, sids, sw, out=sout, note_routing=False)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            split.forward(sx, sids, sw, out=sout, note_routing=False)
        torch.cuda.synchronize()
        for i, b in enumerate(batches):
            for dst, src in zip((sx, sids, sw), b):
                dst.copy_(src)
            g.replay()
            torch.cuda.synchronize()
            got = sout.clone()
            eager = split.forward(*b, note_routing=False)    # eager work between replays
            torch.cuda.synchronize()
            assert torch.equal(got, eager), f"replay {i} differs from the eager split layer"
            check_close(got.cpu().numpy(), _oracle(fmt, d, *b, E, NS, H, I), bf16_out=False,
                        what=f"graph replay {i}")
        del g
    finally:
        torch.cuda.synchronize()
        cpu.close()
