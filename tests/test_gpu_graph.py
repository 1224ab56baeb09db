"""Layers recorded into a HIP graph (decode, and routed batches on the grouped
GEMMs and the exact-pair kernels): every replay (with eager work and
synchronisations between replays, and fresh inputs copied into the static
buffers) must equal the eager result bit for bit."""
import numpy as np
import pytest
import torch

from xtu_moe_amd import formats as F
from xtu_moe_amd import layer as L
from xtu_moe_amd.layer import moe_forward, route
from xtu_moe_amd.synthetic import synth_layer

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fmt", [F.FMT_MXFP4, F.FMT_FP8])
def test_decode_graph_replays_match_eager(fmt):
    dev = torch.device("cuda")
    H, I, E, NS, K, T = 1024, 256, 64, 1, 8, 4
    W = synth_layer(fmt, E, NS, H, I, seed=3, device=dev)
    rkw = dict(top_k=K, scoring="sigmoid", n_group=8, topk_group=4, routed_scaling_factor=2.5)
    g = torch.Generator(device=dev).manual_seed(0)
    xs = [torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16) for _ in range(4)]
    lgs = [torch.randn((T, E), generator=g, device=dev) for _ in range(4)]
    x_st = torch.empty_like(xs[0])
    lg_st = torch.empty_like(lgs[0])
    ids_st = torch.empty((T, K), dtype=torch.int32, device=dev)
    wts_st = torch.empty((T, K), dtype=torch.float32, device=dev)
    out_st = torch.empty((T, H), dtype=torch.bfloat16, device=dev)

    def step():
        route(lg_st, ids_out=ids_st, wts_out=wts_st, **rkw)
        moe_forward(x_st, ids_st, wts_st, W, out=out_st)

    x_st.copy_(xs[0])
    lg_st.copy_(lgs[0])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()
    for r in range(1, 4):
        # eager reference with the same inputs
        x_st.copy_(xs[r])
        lg_st.copy_(lgs[r])
        step()
        torch.cuda.synchronize()
        eager = out_st.clone()
        junk = torch.randn(1 << 20, device=dev).sum()   # eager work between replays
        out_st.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out_st.view(torch.int16).cpu().numpy(),
                                      eager.view(torch.int16).cpu().numpy())
        del junk


@pytest.mark.parametrize("case", ["decode-split", "gemm-128", "fp8-pair32", "mxfp4-pair32"])
def test_routed_layer_graph_replays_match_eager(case):
    """moe_forward routing from logits inside the graph: the decode layer whose
    routing launch also runs the shared expert (T = 1), a 128-token batch
    routed one thread per token in the routing + segmentation launch on the
    grouped GEMMs, and 300-token batches on the exact-pair 32x32x64 kernels
    (FP8 with its block-scale rescaling, MXFP4)."""
    dev = torch.device("cuda")
    if case == "decode-split":
        fmt, H, I, E, NS, K, T = F.FMT_MXFP4, 1024, 256, 256, 1, 8, 1
        rt = dict(scoring="sigmoid", n_group=8, topk_group=4, routed_scaling_factor=2.5)
    elif case in ("fp8-pair32", "mxfp4-pair32"):
        fmt = F.FMT_FP8 if case == "fp8-pair32" else F.FMT_MXFP4
        H, I, E, NS, K, T = 1024, 512, 16, 1, 4, 300
        rt = dict(scoring="sigmoid", n_group=8, topk_group=4, routed_scaling_factor=2.5)
    else:
        fmt, H, I, E, NS, K, T = F.FMT_BF16, 1024, 512, 8, 0, 2, 128
        rt = dict(scoring="softmax", renormalize=True)
    W = synth_layer(fmt, E, NS, H, I, seed=5, device=dev)
    if case == "fp8-pair32":
        assert L.fp8_pair32_use(W) and L.gemm_tile_m(fmt, False, H, I, W) == 128
    if case == "mxfp4-pair32":
        assert L.mx_pair_kernel(fmt, H, I) and L.gemm_tile_m(fmt, False, H, I) == 128
    g = torch.Generator(device=dev).manual_seed(1)
    xs = [torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16) for _ in range(4)]
    lgs = [torch.randn((T, E), generator=g, device=dev) for _ in range(4)]
    x_st = torch.empty_like(xs[0])
    lg_st = torch.empty_like(lgs[0])
    ids_st = torch.empty((T, K), dtype=torch.int32, device=dev)
    wts_st = torch.empty((T, K), dtype=torch.float32, device=dev)
    out_st = torch.empty((T, H), dtype=torch.bfloat16, device=dev)

    def step():
        moe_forward(x_st, ids_st, wts_st, W, out=out_st, router=dict(rt, logits=lg_st))

    x_st.copy_(xs[0])
    lg_st.copy_(lgs[0])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()
    for r in range(1, 4):
        x_st.copy_(xs[r])
        lg_st.copy_(lgs[r])
        step()
        torch.cuda.synchronize()
        eager = out_st.clone()
        eager_ids = ids_st.clone()
        junk = torch.randn(1 << 20, device=dev).sum()   # eager work between replays
        out_st.zero_()
        ids_st.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(ids_st, eager_ids)
        np.testing.assert_array_equal(out_st.view(torch.int16).cpu().numpy(),
                                      eager.view(torch.int16).cpu().numpy())
        del junk


def test_graph_replay_after_eager_calls_on_many_streams():
    """A layer captured into a graph, then eager calls of larger batches on
    forty fresh streams (more than torch's stream pool, so one of them is
    the capture stream again and its scratch grows), then replays: each
    replay equals the eager result of the captured batch bit for bit, and
    that result matches the oracle (scratch a graph holds is never handed
    back to the allocator)."""
    import oracle
    from helpers import bf16_tensor_to_bits, check_close, dense_to_numpy, make_dense_layer
    dev = torch.device("cuda")
    fmt, H, I, E, K, T = F.FMT_BF16, 1024, 512, 8, 2, 128
    d = make_dense_layer(fmt, E, H, I, seed=41)
    W = L.ExpertWeights.from_dense(fmt, d["w13"], d["s13"], d["w2"], d["s2"], device=dev)
    g = torch.Generator(device=dev).manual_seed(2)
    x_st = torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16)
    lg_st = torch.randn((T, E), generator=g, device=dev)
    ids_st = torch.empty((T, K), dtype=torch.int32, device=dev)
    wts_st = torch.empty((T, K), dtype=torch.float32, device=dev)
    out_st = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    rt = dict(scoring="softmax", renormalize=True, logits=lg_st)

    def step():
        moe_forward(x_st, ids_st, wts_st, W, out=out_st, router=rt)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()
    step()
    torch.cuda.synchronize()
    eager = out_st.clone()
    ids_np, wts_np = ids_st.cpu().numpy(), wts_st.cpu().numpy()
    big = 700
    xb = torch.randn((big, H), generator=g, device=dev).to(torch.bfloat16)
    lb = torch.randn((big, E), generator=g, device=dev)
    for i in range(40):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            Tb = big - 13 * (i % 7)
            ib = torch.empty((Tb, K), dtype=torch.int32, device=dev)
            wb = torch.empty((Tb, K), dtype=torch.float32, device=dev)
            moe_forward(xb[:Tb], ib, wb, W, router=dict(rt, logits=lb[:Tb]))
        torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for _ in range(3):
        out_st.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out_st.view(torch.int16).cpu().numpy(),
                                      eager.view(torch.int16).cpu().numpy())
        junk = torch.randn(1 << 20, device=dev).sum()
        del junk
    dn = dense_to_numpy(fmt, d)
    ref = oracle.moe_layer(fmt, bf16_tensor_to_bits(x_st), ids_np, wts_np, E, 0, H, I,
                           dn["w13"], dn["s13"], dn["w2"], dn["s2"])
    check_close(eager.float().cpu().numpy(), ref, bf16_out=True, what="captured layer")
