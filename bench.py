"""Benchmark of the quantized MoE expert layer on one MI355X.

Default run (ds-v3-mxfp4): DeepSeek-V3-shaped MoE layer at decode with MXFP4
experts (H=7168, 256 routed experts + 1 shared, I=2048, grouped-sigmoid
routing with 8 groups / top-4 groups / top-8 and routed scaling 2.5), T = 1,
2, 4 tokens (the headline line), then every other configuration of SUITE
(the same layer at prefill T = 8192 with MXFP4 and with FP8 (128x128
block-scaled) experts, PREFILL_STEPS timed steps each; the Qwen3-Next layer
with MXFP4 / INT8 ALIGN and with NVFP4 experts; the tiny Mixtral layer; the
streamed FP8 layer), each as its own line with its own roofline and CPU
baseline under config.configs, the two DS-V3 prefill layers also under
config.prefill.
A step is one pass of the layer (routing from logits -> segmentation ->
gate/up+SwiGLU -> down -> combine) over a fresh batch of synthetic tokens
(x ~ N(0,1) bf16, logits ~ N(0,1)), weights N(0,0.02) quantised and resident in
HBM.  Every timed step starts with the 256 MB last-level cache flushed (a
1 GiB read-modify-write of a scratch buffer outside the timed events), so
weights stream from HBM as they do when 61 layers take turns.  Decode layers
are timed inside a HIP graph of 8 such layers with distinct weights (each
layer's output the next one's input, as in a model's forward graph): the
layer time is the graph's time / 8, and the time of a graph of one layer
(which adds one graph launch per layer) is reported beside it.

The JSON line reports tokens/s at the largest T (value), the layer time, and:
  roofline      the dominant kernel (gate/up) against HBM (decode) or MFMA
                (prefill): algorithmic bytes or FLOPs per launch over its
                average duration from HIP events on its stream;
  cpu_baseline  the reference xiaotu-moe AVX-512 engine (oracle/_ref, built
                from the reference sources) on the host cores, on a bounded
                sample of the same workload.
Single workloads (--workload): ds-v3-mxfp4-decode, ds-v3-mxfp4-prefill,
ds-v3-fp8-prefill, qwen3-next-int8, qwen3-next-mxfp4 (INT8 ALIGN off),
qwen3-next-nvfp4, mixtral-tiny-bf16, and ds-v3-fp8-streamed: the FP8 layer at
T = 8192 with Zipf(1.1)-skewed router logits, the 64 most-routed experts (and
the shared one) resident in a pool, every other routed expert streamed from
pinned host memory through a ring of 4 slots of 16 experts on a side stream,
overlapped with the grouped GEMMs; it reports the host-link GB/s of the
copies, the compute time of the same layer all-resident, and their overlap.
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "vllm-xtu-moe_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
PEAK_TFLOPS = {"bf16": 2500.0, "fp8": 5000.0, "int8": 5000.0, "fp4": 10100.0}

WORKLOADS = {
    "ds-v3-mxfp4-decode": dict(fmt="mxfp4", E=256, NS=1, H=7168, I=2048, K=8, router="grouped",
                               Ts=[1, 2, 4], limit=0.0, int8=False, graph=True),
    "ds-v3-fp8-prefill": dict(fmt="fp8", E=256, NS=1, H=7168, I=2048, K=8, router="grouped",
                              Ts=[8192], limit=0.0, int8=False, graph=False),
    "ds-v3-mxfp4-prefill": dict(fmt="mxfp4", E=256, NS=1, H=7168, I=2048, K=8,
                                router="grouped", Ts=[8192], limit=0.0, int8=False,
                                graph=False),
    "qwen3-next-int8": dict(fmt="mxfp4", E=512, NS=1, H=2048, I=512, K=10, router="softmax",
                            Ts=[1, 4, 8192], limit=7.0, int8=True, graph=True),
    "qwen3-next-nvfp4": dict(fmt="nvfp4", E=512, NS=1, H=2048, I=512, K=10, router="softmax",
                             Ts=[1, 4, 8192], limit=7.0, int8=False, graph=True),
    # the same MXFP4 layer with INT8 ALIGN off (the default): triples at T = 8192
    "qwen3-next-mxfp4": dict(fmt="mxfp4", E=512, NS=1, H=2048, I=512, K=10, router="softmax",
                             Ts=[8192], limit=7.0, int8=False, graph=False),
    "mixtral-tiny-bf16": dict(fmt="bf16", E=8, NS=0, H=1024, I=2048, K=2, router="softmax",
                              Ts=[128], limit=0.0, int8=False, graph=True, graph_max_T=128,
                              bound="hbm"),
    "ds-v3-fp8-streamed": dict(fmt="fp8", E=256, NS=1, H=7168, I=2048, K=8, router="grouped",
                               Ts=[8192], limit=0.0, int8=False, graph=False, resident=64,
                               tile_e=16, nslots=4, zipf=1.1),
}
PCIE_GEN5_X16_GBS = 64.0   # per direction, before protocol overhead
DEFAULT_SET = "ds-v3-mxfp4"   # decode T=1,2,4 plus every configuration below
PREFILL_SET = ("ds-v3-mxfp4-prefill", "ds-v3-fp8-prefill")
# the default run's sub-lines: each workload's own line (roofline, cpu_baseline)
# under config.configs, keyed by workload, with the configuration it measures
SUITE = (("ds-v3-mxfp4-prefill", "DS-V3 MXFP4 prefill T=8192"),
         ("ds-v3-fp8-prefill", "C3: DS-V3 FP8 prefill T=8192"),
         ("qwen3-next-int8", "C4: Qwen3-Next MXFP4, decode T=1,4 and INT8 ALIGN T=8192"),
         ("qwen3-next-nvfp4", "C4: Qwen3-Next NVFP4 T=1,4,8192"),
         ("mixtral-tiny-bf16", "C1: tiny Mixtral bf16 T=128"),
         ("ds-v3-fp8-streamed", "C5: DS-V3 FP8 streamed prefill, 64 resident + 192 streamed"))
PREFILL_STEPS = 5
CHAIN = 8                  # layers per decode graph


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default=DEFAULT_SET, choices=sorted(WORKLOADS) + [DEFAULT_SET])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--no-flush", action="store_true", help="keep caches warm between steps")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 counter runs behind roofline.traffic")
    ap.add_argument("--pmc-child", type=int, default=0, help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: the expert path here runs on one GPU "
              "(no collectives or expert-parallel sharding); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    if args.workload == DEFAULT_SET:
        return bench_default(args)
    print(json.dumps(bench_one(args)), flush=True)


def bench_default(args):
    """The headline line (the DS-V3 MXFP4 decode workload, value = tok/s at
    T=4) with every other configuration's line under config.configs (its
    own roofline and cpu_baseline; prefill workloads PREFILL_STEPS timed
    steps), the two DS-V3 prefill layers also under config.prefill."""
    import gc

    import torch

    a = argparse.Namespace(**vars(args))
    a.workload = "ds-v3-mxfp4-decode"
    line = bench_one(a)
    subs = {}
    for wl, what in SUITE:
        gc.collect()
        torch.cuda.empty_cache()
        b = argparse.Namespace(**vars(args))
        b.workload = wl
        if max(WORKLOADS[wl]["Ts"]) > 16 and not WORKLOADS[wl].get("graph"):
            b.steps, b.warmup = min(args.steps, PREFILL_STEPS), min(args.warmup, 2)
        t0 = time.time()
        sub = bench_one(b)
        sub = {k: v for k, v in sub.items() if k not in ("metric", "n_gpus", "higher_is_better",
                                                         "scaling", "vs_baseline")}
        sub["measures"] = what
        sub["bench_s"] = time.time() - t0
        subs[wl] = sub
    pre = {}
    for wl in PREFILL_SET:
        sl = subs[wl]
        r = sl["config"]["per_T"]["8192"]
        pre[wl] = dict(T=8192, steps=sl["steps"], warmup=sl["warmup"], layer_ms=r["layer_ms"],
                       tok_s=r["tok_s"], gate_up_ms=r["gate_up_ms"],
                       gate_up_TFLOPs=r["gate_up_TFLOPs"], dtype=sl["dtype"],
                       distinct_experts=r["distinct_experts"], roofline=sl["roofline"])
    line["config"]["workload"] = DEFAULT_SET
    line["config"]["measures"] = "C2: DS-V3 MXFP4 decode T=1,2,4"
    line["config"]["prefill"] = pre
    line["config"]["configs"] = subs
    print(json.dumps(line), flush=True)


def hook_for(cfg, W):
    """The quant-method hook of this workload's format (XiaotuExperts*) over
    device weights W, with the routing and SwiGLU attributes the layer would
    carry: the state process_weights_after_loading leaves (the checkpoint
    repack is skipped; the weights are already in the kernels' layout)."""
    import types

    from xtu_moe_amd import mixed_experts as ME

    cls = {"mxfp4": ME.XiaotuExpertsMxfp4, "fp8": ME.XiaotuExpertsFp8,
           "nvfp4": ME.XiaotuExpertsNvfp4, "bf16": ME.XiaotuExpertsBF16}[cfg["fmt"]]
    grouped = cfg["router"] == "grouped"
    lay = types.SimpleNamespace(top_k=cfg["K"], renormalize=True, use_grouped_topk=grouped,
                                scoring_func="sigmoid" if grouped else "softmax",
                                num_expert_group=8 if grouped else None,
                                topk_group=4 if grouped else None,
                                routed_scaling_factor=2.5 if grouped else 1.0,
                                swiglu_limit=cfg["limit"] or None)
    hook = cls()
    hook._read_layer_attrs(lay)
    hook._weights = W
    return hook


def bench_one(args):
    """One workload; returns its JSON line (the streamed workload prints its own)."""
    import numpy as np
    import torch

    from xtu_moe_amd import _lib
    from xtu_moe_amd import formats as F
    from xtu_moe_amd.layer import (_fp8pair_bufs, _mxpair_bufs, _p, _stream, fp8_pair32_use,
                                   gemm_tile_m, int8_align_on, moe_forward, mx_act_mode,
                                   mx_pair_kernel, mx_tri, pair_gemm, route, segmentation)
    from xtu_moe_amd.synthetic import synth_layer

    cfg = WORKLOADS[args.workload]
    if "resident" in cfg:
        return streamed(args, cfg)
    if args.pmc_child:
        return pmc_child(args, cfg, args.pmc_child)
    fmt = F.fmt_of(cfg["fmt"])
    E, NS, H, I, K = cfg["E"], cfg["NS"], cfg["H"], cfg["I"], cfg["K"]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    _lib.load()
    t0 = time.time()
    W = synth_layer(fmt, E, NS, H, I, seed=0, device=dev)
    if cfg["int8"]:
        W.int8_planes()
    torch.cuda.synchronize()
    log(f"[bench] built {E}+{NS} experts fmt={cfg['fmt']} in {time.time() - t0:.1f}s")
    # decode: a graph of CHAIN layers with distinct weights, each layer's output
    # the next one's input, as a model's forward graph runs them
    chain_Ws = [W]
    if cfg["graph"]:
        for l in range(1, CHAIN):
            chain_Ws.append(synth_layer(fmt, E, NS, H, I, seed=l, device=dev))
        torch.cuda.synchronize()
        log(f"[bench] built {CHAIN} layers for the layer-chain graph")
    flush = torch.empty(256 << 20, dtype=torch.float32, device=dev)   # 1 GiB
    gen = torch.Generator(device=dev).manual_seed(1234)

    if cfg["router"] == "grouped":
        rkw = dict(top_k=K, scoring="sigmoid", n_group=8, topk_group=4, routed_scaling_factor=2.5)
    else:
        rkw = dict(top_k=K, scoring="softmax")
    router_w = None
    if args.workload == "mixtral-tiny-bf16":
        router_w = torch.randn((E, H), generator=gen, device=dev) * 0.02

    # algorithmic bytes of one expert: gate/up stream, whole expert
    e_bytes13 = F.algorithmic_bytes(fmt, 2 * I, H)
    e_bytes = e_bytes13 + F.algorithmic_bytes(fmt, H, I)
    nsteps = args.warmup + args.steps
    results = {}
    for T in cfg["Ts"]:
        # INT8 activations where the reference engine's token-count gate takes them
        i8 = cfg["int8"] and int8_align_on(T, True)
        xs = [torch.randn((T, H), generator=gen, device=dev).to(torch.bfloat16) for _ in range(min(nsteps, 8))]
        if router_w is not None:
            lgs = [(x.float() @ router_w.t()).contiguous() for x in xs]
        else:
            lgs = [torch.randn((T, E), generator=gen, device=dev) for _ in range(nsteps)]
        x_st = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
        lg_st = torch.empty((T, E), dtype=torch.float32, device=dev)
        out_st = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
        ids_st = torch.empty((T, K), dtype=torch.int32, device=dev)
        wts_st = torch.empty((T, K), dtype=torch.float32, device=dev)

        rt = dict(logits=lg_st, scoring=rkw["scoring"], n_group=rkw.get("n_group", 1),
                  topk_group=rkw.get("topk_group", 1),
                  routed_scaling_factor=rkw.get("routed_scaling_factor", 1.0))

        def step():
            moe_forward(x_st, ids_st, wts_st, W, swiglu_limit=cfg["limit"], out=out_st,
                        int8=i8, router=rt)

        def load(s):
            x_st.copy_(xs[s % len(xs)])
            lg_st.copy_(lgs[s % len(lgs)])

        load(0)
        step()
        torch.cuda.synchronize()
        use_graph = cfg["graph"] and T <= cfg.get("graph_max_T", 16)
        graph = None
        if use_graph:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(2):
                    step()
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                step()
            torch.cuda.synchronize()

        def run_layer():
            if graph is not None:
                graph.replay()
            else:
                step()

        # ---- whole layer, cold cache per step
        for s in range(args.warmup):
            load(s)
            run_layer()
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(args.steps)]
        n_active = []
        wall0 = time.time()
        for s in range(args.steps):
            # weights cold (flush), this step's activations and logits just
            # written (as the previous kernels of a model leave them)
            if not args.no_flush:
                flush.add_(1.0)
            load(args.warmup + s)
            ev[s][0].record()
            run_layer()
            ev[s][1].record()
        torch.cuda.synchronize()
        wall = time.time() - wall0
        layer_ms = [a.elapsed_time(b) for a, b in ev]

        # ---- layer chain: CHAIN distinct layers in one graph, time / CHAIN;
        # once through moe_forward, once through the quant-method hook's
        # apply (the call vLLM makes), each layer's output the next one's input
        chain_ms, hook_ms = [], []
        chain_active = []
        if graph is not None:
            c_lg = [torch.empty((T, E), dtype=torch.float32, device=dev) for _ in chain_Ws]
            c_out = [torch.empty((T, H), dtype=torch.bfloat16, device=dev) for _ in chain_Ws]
            c_ids = [torch.empty((T, K), dtype=torch.int32, device=dev) for _ in chain_Ws]
            c_wts = [torch.empty((T, K), dtype=torch.float32, device=dev) for _ in chain_Ws]

            def fwd_layer(l, xin):
                moe_forward(xin, c_ids[l], c_wts[l], chain_Ws[l], swiglu_limit=cfg["limit"],
                            out=c_out[l], int8=i8, router=dict(rt, logits=c_lg[l]))

            hooks = [hook_for(cfg, Wl) for Wl in chain_Ws] if not i8 else None

            def hook_layer(l, xin):
                hooks[l].apply(xin, None, None, router_logits=c_lg[l], output=c_out[l])

            def chain_load(s):
                x_st.copy_(xs[s % len(xs)])
                for l in range(len(chain_Ws)):
                    c_lg[l].copy_(lgs[(s + l) % len(lgs)])

            def time_chain(layer):
                def chain_step():
                    xin = x_st
                    for l in range(len(chain_Ws)):
                        layer(l, xin)
                        xin = c_out[l]

                chain_load(0)
                side = torch.cuda.Stream()
                side.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(side):
                    for _ in range(2):
                        chain_step()
                torch.cuda.current_stream().wait_stream(side)
                cgraph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(cgraph):
                    chain_step()
                torch.cuda.synchronize()
                for s in range(args.warmup):
                    chain_load(s)
                    cgraph.replay()
                torch.cuda.synchronize()
                cev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                       for _ in range(args.steps)]
                for s in range(args.steps):
                    if not args.no_flush:
                        flush.add_(1.0)
                    chain_load(args.warmup + s)
                    cev[s][0].record()
                    cgraph.replay()
                    cev[s][1].record()
                torch.cuda.synchronize()
                del cgraph
                return [a.elapsed_time(b) / len(chain_Ws) for a, b in cev]

            chain_ms = time_chain(fwd_layer)
            if hooks is not None:
                hook_ms = time_chain(hook_layer)
            for s in range(args.steps):
                for l in range(len(chain_Ws)):
                    w_, i_ = route(lgs[(args.warmup + s + l) % len(lgs)], **rkw)
                    chain_active.append(len(torch.unique(i_)) + NS)
        # distinct experts per step (algorithmic bytes), re-derived outside timing
        for s in range(args.steps):
            load(args.warmup + s)
            w_, i_ = route(lg_st, **rkw)
            n_active.append(len(torch.unique(i_)) + NS)

        # ---- dominant kernel alone (gate/up), cold cache, same stream
        seg = None
        gu_ms = []
        bm = gemm_tile_m(fmt, i8, H, I, W)
        f8q = not (T <= 16 and not i8) and not i8 and fp8_pair32_use(W)
        decode = T <= 16 and not i8
        act = torch.empty((T * K + T * NS, I), dtype=torch.bfloat16, device=dev)
        # one untimed call first: a kernel's code object loads on its first
        # launch (the layer above may have run only other kernels)
        for s in range(-1, args.steps):
            load(args.warmup + max(s, 0))
            w_, i_ = route(lg_st, **rkw)
            seg = segmentation(T, K, E, NS, bm, dev).run(i_, w_)
            st = _stream()
            fp8x = mxx = f8x = None
            if f8q:
                f8x = _mxpair_bufs("xm", T, H, dev)
                _lib.call("xtu_pair_quant_il", _p(x_st), T, H, *[_p(t) for t in f8x], st)
            elif not decode and not i8 and mx_pair_kernel(fmt, H, I):
                mxk = mx_act_mode(fmt, H, I)
                mxx = _mxpair_bufs("xm", T, H, dev)
                s13p, _ = W.mx_pair_scales()
                _lib.call(f"xtu_{'pair' if mxk == 'pair' else 'tri'}_quant_il", _p(x_st), T, H,
                          *[_p(t) for t in mxx], st)
            elif not decode and not i8 and pair_gemm(fmt, H, I):
                fp8x = _fp8pair_bufs("x8", T, H, dev)
                _lib.call("xtu_fp8pair_quant", _p(x_st), T, H, *[_p(t) for t in fp8x], st)
            if i8:
                w13_8, emin13, _, _ = W.int8_planes()
                a8x = torch.empty((T, H), dtype=torch.int8, device=dev)
                crx = torch.empty(T, dtype=torch.int32, device=dev)
                _lib.call("xtu_i8_quant_rows", _p(x_st), T, H, _p(a8x), _p(crx), st)
            if not args.no_flush:
                flush.add_(1.0)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            if decode:
                _lib.call("xtu_decode_gate_up", fmt, _p(x_st), T, H, I, _p(W.w13), _p(W.s13),
                          _p(W.gs13), 0, 0, 0, _p(seg.sorted_tok), _p(seg.seg_start),
                          _p(seg.active), 0, _p(seg.n_active), min(E, T * K) + NS, _p(act),
                          cfg["limit"], 1.0, 0.0, st)
            elif i8:
                lo, hi = seg.tile_range_ptrs(0, E + NS)
                _lib.call("xtu_i8_gemm_gate_up", _p(a8x), _p(crx), _p(seg.sorted_tok), H, I,
                          _p(w13_8), _p(emin13), 0, _p(seg.seg_start), _p(seg.tile_expert),
                          _p(seg.tile_row0), lo, hi, seg.max_tiles, _p(act), 0, cfg["limit"],
                          1.0, 0.0, st)
            elif f8x is not None:
                lo, hi = seg.tile_range_ptrs(0, E + NS)
                _lib.call("xtu_f8_pair_gate_up", *[_p(t) for t in f8x], _p(seg.sorted_tok), H, I,
                          _p(W.w13), _p(W.s13), 0, 0, 0, _p(seg.seg_start), _p(seg.tile_expert),
                          _p(seg.tile_row0), _p(seg.expert_tile_start), lo, hi, seg.max_tiles,
                          _p(act), cfg["limit"], 1.0, 0.0, st)
            elif mxx is not None:
                lo, hi = seg.tile_range_ptrs(0, E + NS)
                _lib.call(f"xtu_mx_{mxk}_gate_up", *[_p(t) for t in mxx], _p(seg.sorted_tok), H, I,
                          _p(W.w13), _p(s13p), 0, 0, 0, _p(seg.seg_start), _p(seg.tile_expert),
                          _p(seg.tile_row0), _p(seg.expert_tile_start), lo, hi, seg.max_tiles,
                          _p(act), cfg["limit"], 1.0, 0.0, st)
            elif fp8x is not None:
                lo, hi = seg.tile_range_ptrs(0, E + NS)
                _lib.call("xtu_gemm_pair_gate_up", fmt, *[_p(t) for t in fp8x],
                          _p(seg.sorted_tok), H, I, _p(W.w13), _p(W.s13), 0, 0, 0,
                          _p(seg.seg_start), _p(seg.tile_expert), _p(seg.tile_row0),
                          _p(seg.expert_tile_start), lo, hi, seg.max_tiles, _p(act),
                          cfg["limit"], 1.0, 0.0, st)
            else:
                lo, hi = seg.tile_range_ptrs(0, E + NS)
                _lib.call("xtu_gemm_gate_up", fmt, _p(x_st), _p(seg.sorted_tok), H, I, _p(W.w13),
                          _p(W.s13), _p(W.gs13), 0, 0, 0, _p(seg.seg_start), _p(seg.tile_expert),
                          _p(seg.tile_row0), lo, hi, seg.max_tiles, _p(act), cfg["limit"], 1.0,
                          0.0, st)
            b.record()
            torch.cuda.synchronize()
            if s >= 0:
                gu_ms.append(a.elapsed_time(b))

        # HIP-event bracket cost on this stream (same flush-then-record pattern,
        # nothing in between), taken off the single-kernel times
        empty_ms = []
        for s in range(max(10, args.steps // 2)):
            if not args.no_flush:
                flush.add_(1.0)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            b.record()
            torch.cuda.synchronize()
            empty_ms.append(a.elapsed_time(b))
        ev_overhead = float(np.median(empty_ms))
        gu_ms = [max(g - ev_overhead, 1e-6) for g in gu_ms]

        A = T * K + T * NS
        single_ms = float(np.mean(layer_ms))
        hook_layer_ms = float(np.mean(hook_ms)) if hook_ms else None
        if chain_ms:   # per-layer time inside the layer-chain graph
            layer_ms, n_active = chain_ms, chain_active
        mean_layer = float(np.mean(layer_ms))
        mean_gu = float(np.mean(gu_ms))
        mean_active = float(np.mean(n_active))
        layer_bytes = mean_active * e_bytes + 2 * T * H * 2
        gu_bytes = mean_active * e_bytes13 + T * H * 2 + A * I * 2
        gu_flops = 2.0 * A * (2 * I) * H
        results[T] = dict(T=T, layer_ms=mean_layer, layer_ms_min=float(np.min(layer_ms)),
                          tok_s=T / (mean_layer / 1e3), distinct_experts=mean_active,
                          layer_GBs=layer_bytes / (mean_layer / 1e3) / 1e9,
                          gate_up_ms=mean_gu, gate_up_GBs=gu_bytes / (mean_gu / 1e3) / 1e9,
                          gate_up_TFLOPs=gu_flops / (mean_gu / 1e3) / 1e12,
                          graph=graph is not None, wall_s=wall,
                          event_overhead_us=ev_overhead * 1e3, gate_up_bytes=gu_bytes,
                          single_layer_graph_ms=single_ms, int8_activation=bool(i8),
                          layer_chain=len(chain_Ws) if chain_ms else 1,
                          hook_layer_ms=hook_layer_ms,
                          layer_hbm_frac=layer_bytes / (mean_layer / 1e3) / 1e9 / HBM_PEAK_GBS,
                          layer_ideal_us=layer_bytes / (HBM_PEAK_GBS * 1e9) * 1e6)
        log(f"[bench] T={T}: layer {mean_layer * 1e3:.1f} us ({results[T]['layer_GBs']:.0f} GB/s; "
            f"single-layer graph {single_ms * 1e3:.1f} us"
            + (f"; through the hook's apply {hook_layer_ms * 1e3:.1f} us" if hook_layer_ms else "")
            + "), "
            f"gate_up {mean_gu * 1e3:.1f} us ({results[T]['gate_up_GBs']:.0f} GB/s, "
            f"{results[T]['gate_up_TFLOPs']:.0f} TFLOP/s), |D|={mean_active:.1f}")

    Th = max(cfg["Ts"])
    r = results[Th]
    decode_head = Th <= 16

    def prefill_traffic(roof, kernel):
        """HBM bytes of one prefill gate/up launch from the counter runs, next
        to its algorithmic bytes (weights of the distinct experts once, the
        quantised activation rows with their scales, the act rows written)."""
        if args.no_traffic:
            return
        tr = measure_traffic(args.workload, Th, timeout=300, kernel=kernel)
        if tr is None:
            return
        roof["traffic"] = tr["bytes"]
        roof["traffic_detail"] = tr
        if tr.get("distinct_experts"):
            tr["algorithmic_bytes"] = (tr["distinct_experts"] * e_bytes13 + Th * (2 * H + H // 32)
                                       + (Th * K + Th * NS) * I * 2)

    if decode_head:
        roof = dict(bound="hbm", achieved=r["gate_up_GBs"], peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=r["gate_up_GBs"] / HBM_PEAK_GBS, traffic=None,
                    kernel="decode_gate_up_kernel")
        if not args.no_traffic:
            tr = measure_traffic(args.workload, Th)
            if tr is not None:
                roof["traffic"] = tr["bytes"]
                roof["traffic_detail"] = tr
                if tr.get("distinct_experts"):   # the counter run's own routing
                    tr["algorithmic_bytes"] = (tr["distinct_experts"] * e_bytes13 + Th * H * 2
                                               + (Th * K + Th * NS) * I * 2)
    elif cfg.get("bound") == "hbm":
        # a batch whose weights outweigh its arithmetic (tiny Mixtral: 128
        # tokens over 8 experts of 12.6 MB): the grouped GEMM against HBM
        roof = dict(bound="hbm", achieved=r["gate_up_GBs"], peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=r["gate_up_GBs"] / HBM_PEAK_GBS, traffic=None, kernel="moe_gemm_kernel",
                    layer_frac=r["layer_GBs"] / HBM_PEAK_GBS)
    elif mx_tri(fmt, H, I) and not cfg["int8"] and not decode_head:
        # fp6 / fp4 A (activation triples, or their first two pieces) x e2m1
        # B on the double-rate 32x32x64 MFMA: the fp6/fp4 peak; every
        # algorithmic product is three (two) MFMA products
        ach = r["gate_up_TFLOPs"]
        npc = 2.0 if mx_act_mode(fmt, H, I) == "duo" else 3.0
        roof = dict(bound="mfma", achieved=ach, peak=PEAK_TFLOPS["fp4"], unit="TFLOP/s",
                    frac=ach / PEAK_TFLOPS["fp4"], traffic=None, kernel="mx_pair_gemm_kernel",
                    activation_pieces=int(npc),
                    mfma_issue_frac=npc * ach / PEAK_TFLOPS["fp4"],
                    frac_of_fp8_peak=ach / PEAK_TFLOPS["fp8"],
                    frac_of_bf16_peak=ach / PEAK_TFLOPS["bf16"])
        prefill_traffic(roof, "mx_pair_gemm_kernel<true")
    elif pair_gemm(fmt, H, I) and not cfg["int8"]:
        # scaled MFMA with an e4m3 A (FP8: e4m3 B; MXFP4: e2m1 B), which runs
        # at the fp8 rate; every algorithmic product is two MFMA products
        # (the activation's hi and lo halves)
        ach = r["gate_up_TFLOPs"]
        roof = dict(bound="mfma", achieved=ach, peak=PEAK_TFLOPS["fp8"], unit="TFLOP/s",
                    frac=ach / PEAK_TFLOPS["fp8"], traffic=None,
                    kernel=("mx_pair_gemm_kernel" if mx_pair_kernel(fmt, H, I)
                            else "f8_pair_gemm_kernel" if fp8_pair32_use(W)
                            else "gemm8_kernel"),
                    mfma_issue_frac=2.0 * ach / PEAK_TFLOPS["fp8"],
                    frac_of_bf16_peak=ach / PEAK_TFLOPS["bf16"])
        if roof["kernel"] == "f8_pair_gemm_kernel":
            prefill_traffic(roof, "f8_pair_gemm_kernel<true")
        if cfg["fmt"] == "mxfp4":
            roof["frac_of_fp4_peak"] = ach / PEAK_TFLOPS["fp4"]
    else:
        dt = "int8" if cfg["int8"] else "bf16"
        roof = dict(bound="mfma", achieved=r["gate_up_TFLOPs"], peak=PEAK_TFLOPS[dt],
                    unit="TFLOP/s", frac=r["gate_up_TFLOPs"] / PEAK_TFLOPS[dt], traffic=None,
                    kernel=("i8_gemm_kernel" if cfg["int8"] else "moe_gemm_kernel"),
                    frac_of_fp8_peak=r["gate_up_TFLOPs"] / PEAK_TFLOPS["fp8"])

    cpu = None
    if not args.no_cpu_baseline:
        try:
            cpu = cpu_baseline(cfg, W, Th, rkw, args.cpu_seconds, dev)
        except Exception as exc:  # noqa: BLE001
            log(f"[bench] cpu baseline unavailable: {type(exc).__name__}: {exc}")
            cpu = None

    line = {
        "metric": "MoE-layer ms & tok/s (decode T=1-4, prefill T=8192); HBM GB/s / MFMA % peak",
        "value": r["tok_s"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r["layer_ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"mxfp4": ("bf16-mfma/e2m1+e8m0"
                            if decode_head or not pair_gemm(fmt, H, I)
                            else "fp6xfp4-mfma/e2m3,e2m3-duo x e2m1+e8m0"
                            if mx_act_mode(fmt, H, I) == "duo"
                            else "fp6xfp4-mfma/e2m3,e2m3,e2m1-triple x e2m1+e8m0"
                            if mx_tri(fmt, H, I)
                            else "fp8xfp4-mfma/e4m3-pair x e2m1+e8m0"),
                  "fp8": ("bf16-mfma/e4m3+f32-block" if decode_head
                          else "fp8-mfma/e4m3-pair x e4m3+f32-block"),
                  "nvfp4": "bf16-mfma/e2m1+e4m3", "bf16": "bf16"}[cfg["fmt"]]
                 if not cfg["int8"] else "int8-mfma/int32-acc",
        "data": "synthetic (seeded N(0,1) tokens and logits, N(0,0.02) weights quantised)",
        "config": {"workload": args.workload, "T": Th, "hidden": H, "intermediate": I,
                   "routed_experts": E, "shared_experts": NS, "top_k": K,
                   "weights": cfg["fmt"], "int8_activation": cfg["int8"],
                   "cache_flushed_per_step": not args.no_flush,
                   "per_T": {str(t): v for t, v in results.items()}},
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    return line


COPY_BYTES = 256 << 20   # calibration copy for the memory counters


def pmc_child(args, cfg, T):
    """Run under rocprofv3 --pmc by measure_traffic: three cold-cache launches
    of the dominant gate/up kernel at T tokens (the decode kernel for T <= 16;
    the MXFP4 triple or FP8 pair prefill kernel otherwise, after its
    quantiser), then one device-to-device copy of COPY_BYTES (the counter
    calibration)."""
    import torch

    from xtu_moe_amd import _lib
    from xtu_moe_amd import formats as F
    from xtu_moe_amd.layer import (_mxpair_bufs, _p, _stream, fp8_pair32_use, gemm_tile_m,
                                   mx_act_mode, mx_tri, route, segmentation)
    from xtu_moe_amd.synthetic import synth_layer

    fmt = F.fmt_of(cfg["fmt"])
    E, NS, H, I, K = cfg["E"], cfg["NS"], cfg["H"], cfg["I"], cfg["K"]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    _lib.load()
    W = synth_layer(fmt, E, NS, H, I, seed=0, device=dev)
    gen = torch.Generator(device=dev).manual_seed(1234)
    x = torch.randn((T, H), generator=gen, device=dev).to(torch.bfloat16)
    lg = torch.randn((T, E), generator=gen, device=dev)
    rkw = dict(top_k=K, scoring="sigmoid", n_group=8, topk_group=4, routed_scaling_factor=2.5)
    w_, i_ = route(lg, **rkw)
    prefill = T > 16
    bm = gemm_tile_m(fmt, False, H, I, W) if prefill else 128
    seg = segmentation(T, K, E, NS, bm, dev).run(i_, w_)
    act = torch.empty((T * K + T * NS, I), dtype=torch.bfloat16, device=dev)
    flush = torch.empty(256 << 20, dtype=torch.float32, device=dev)
    st = _stream()
    if prefill:
        if mx_tri(fmt, H, I):
            kind, s13 = "mx_" + mx_act_mode(fmt, H, I), W.mx_pair_scales(st)[0]
            qname = "xtu_tri_quant_il"
        elif fp8_pair32_use(W):
            kind, s13, qname = "f8_pair", W.s13, "xtu_pair_quant_il"
        else:
            raise SystemExit("no counter child for this prefill kernel")
        xq = _mxpair_bufs("xm", T, H, dev, st)
        _lib.call(qname, _p(x), T, H, *[_p(t) for t in xq], st)
        lo, hi = seg.tile_range_ptrs(0, E + NS)
    for _ in range(3):
        flush.add_(1.0)
        if prefill:
            _lib.call(f"xtu_{kind}_gate_up", *[_p(t) for t in xq], _p(seg.sorted_tok), H, I,
                      _p(W.w13), _p(s13), 0, 0, 0, _p(seg.seg_start), _p(seg.tile_expert),
                      _p(seg.tile_row0), _p(seg.expert_tile_start), lo, hi, seg.max_tiles,
                      _p(act), cfg["limit"], 1.0, 0.0, st)
        else:
            _lib.call("xtu_decode_gate_up", fmt, _p(x), T, H, I, _p(W.w13), _p(W.s13),
                      _p(W.gs13), 0, 0, 0, _p(seg.sorted_tok), _p(seg.seg_start),
                      _p(seg.active), 0, _p(seg.n_active), min(E, T * K) + NS, _p(act),
                      cfg["limit"], 1.0, 0.0, st)
    torch.cuda.synchronize()
    src = torch.ones(COPY_BYTES, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    flush.add_(1.0)
    dst.copy_(src)
    torch.cuda.synchronize()
    print(f"[pmc-child] distinct experts {len(torch.unique(i_)) + NS}", flush=True)


def measure_traffic(workload, T, timeout=150, kernel="decode_gate_up"):
    """HBM bytes per launch of the gate/up kernel whose name contains `kernel`
    from two rocprofv3 counter runs of pmc_child (FETCH_SIZE, then WRITE_SIZE,
    in KiB per dispatch), each scaled by the same counter's reading for a
    device copy of known size.  None when rocprofv3 is unavailable or a run
    fails."""
    import csv
    import shutil
    import subprocess
    import tempfile

    prof = shutil.which("rocprofv3")
    if prof is None:
        return None
    res = {}
    tmp = tempfile.mkdtemp(prefix="xtu_pmc_")
    try:
        for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
            d = os.path.join(tmp, ctr)
            cmd = [prof, "--pmc", ctr, "--output-format", "csv", "-d", d, "-o", "p", "--",
                   sys.executable, os.path.abspath(__file__), "--workload", workload,
                   "--pmc-child", str(int(T))]
            r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout,
                               cwd=tempfile.gettempdir(), env=dict(os.environ, TMPDIR=tempfile.gettempdir()))
            if r.returncode != 0:
                log(f"[bench] {ctr} counter run failed (rc={r.returncode})")
                return None
            for ln in r.stdout.splitlines():
                if ln.startswith("[pmc-child] distinct experts "):
                    res["distinct"] = int(ln.split()[-1])
            path = None
            for root, _, files in os.walk(d):
                for f in files:
                    if f.endswith("counter_collection.csv"):
                        path = os.path.join(root, f)
            if path is None:
                return None
            # the calibration copy is the first copy dispatched after the
            # last launch of the kernel (the weight synthesis before them
            # issues copies of its own)
            rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Dispatch_Id"]))
            kern = [float(r["Counter_Value"]) * 1024.0 for r in rows if kernel in r["Kernel_Name"]]
            last = max((i for i, r in enumerate(rows) if kernel in r["Kernel_Name"]), default=-1)
            copy = [float(r["Counter_Value"]) * 1024.0 for r in rows[last + 1:]
                    if "copy" in r["Kernel_Name"].lower()][:1]
            if not kern or not copy or copy[0] <= 0:
                return None
            factor = COPY_BYTES / copy[0]
            res[ctr] = dict(raw=sum(kern) / len(kern), factor=factor,
                            bytes=sum(kern) / len(kern) * factor)
    except (OSError, subprocess.SubprocessError, ValueError, KeyError) as exc:
        log(f"[bench] traffic counters unavailable: {type(exc).__name__}: {exc}")
        return None
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return dict(bytes=res["FETCH_SIZE"]["bytes"] + res["WRITE_SIZE"]["bytes"],
                distinct_experts=res.get("distinct"),
                fetch_bytes=res["FETCH_SIZE"]["bytes"], write_bytes=res["WRITE_SIZE"]["bytes"],
                fetch_factor=res["FETCH_SIZE"]["factor"], write_factor=res["WRITE_SIZE"]["factor"],
                calibration=f"device copy of {COPY_BYTES} bytes under the same counter")


def streamed(args, cfg):
    """Streamed prefill: resident pool + ring of host-streamed experts."""
    import numpy as np
    import torch

    from xtu_moe_amd import _lib
    from xtu_moe_amd import formats as F
    from xtu_moe_amd.expert_pool import LayerPool
    from xtu_moe_amd.host_store import HostExpertStore
    from xtu_moe_amd.layer import moe_forward, route
    from xtu_moe_amd.ring import RingStats, gpu_moe_layer_from_engine_tiled
    from xtu_moe_amd.synthetic import synth_layer

    fmt = F.fmt_of(cfg["fmt"])
    E, NS, H, I, K = cfg["E"], cfg["NS"], cfg["H"], cfg["I"], cfg["K"]
    T = cfg["Ts"][0]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    _lib.load()
    t0 = time.time()
    W = synth_layer(fmt, E, NS, H, I, seed=0, device=dev)
    store = HostExpertStore.from_weights(W)
    torch.cuda.synchronize()
    log(f"[bench] built {E}+{NS} experts fmt={cfg['fmt']} (device + pinned host) in "
        f"{time.time() - t0:.1f}s")
    rkw = dict(top_k=K, scoring="sigmoid", n_group=8, topk_group=4, routed_scaling_factor=2.5)
    gen = torch.Generator(device=dev).manual_seed(1234)
    # Zipf(s) popularity: logit = -s*ln(rank) + Gumbel noise, so the top-k of a
    # token samples experts without replacement in proportion to rank^-s
    # (exactly so without the group limit)
    rank = torch.randperm(E, generator=torch.Generator().manual_seed(7)) + 1
    skew = (-cfg["zipf"] * torch.log(rank.double())).float().to(dev)
    nsteps = args.warmup + args.steps
    xs = [torch.randn((T, H), generator=gen, device=dev).to(torch.bfloat16) for _ in range(2)]
    batches = []
    for s in range(nsteps):
        u = torch.rand((T, E), generator=gen, device=dev).clamp_(1e-12, 1.0 - 1e-7)
        lg = skew - torch.log(-torch.log(u))
        w_, i_ = route(lg, **rkw)
        batches.append((xs[s % 2], i_, w_))
    # the pool holds the most-routed experts of the first batch (a pin table
    # built from profiled routing)
    counts = torch.bincount(batches[0][1].flatten().long(), minlength=E)
    pinned = torch.argsort(counts, descending=True, stable=True)[:cfg["resident"]].tolist()
    share = float(counts[pinned].sum()) / float(counts.sum())
    pool = LayerPool(store, dev, H, I, 128, E, pinned, 0, layout=cfg["fmt"], topk=K)
    out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    kw = dict(device=dev, nslots=cfg["nslots"], pool=pool, tile_e=cfg["tile_e"], out=out)

    def streamed_layer(b, stats=None):
        x, i_, w_ = b
        return gpu_moe_layer_from_engine_tiled(store, x, i_, w_, H, I, E, K, stats=stats, **kw)

    for s in range(args.warmup):
        streamed_layer(batches[s])
    torch.cuda.synchronize()
    lay_ms, dma_ms, moved, tiles = [], [], [], []
    for s in range(args.steps):
        b = batches[args.warmup + s]
        st = RingStats()
        a, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        streamed_layer(b, st)
        e.record()
        st.finish()
        lay_ms.append(a.elapsed_time(e))
        dma_ms.append(st.dma_ms)
        moved.append(st.bytes)
        tiles.append(st.tiles)
    # the same layers with every expert resident: the compute the copies hide behind
    cmp_ms = []
    for s in range(args.steps):
        x, i_, w_ = batches[args.warmup + s]
        a, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        moe_forward(x, i_, w_, W, out=out)
        e.record()
        torch.cuda.synchronize()
        cmp_ms.append(a.elapsed_time(e))
    # plain pinned host -> device copy of the same size as one tile's weights
    tile_bytes = int(np.mean(moved) / max(np.mean(tiles), 1))
    src = torch.empty(tile_bytes, dtype=torch.uint8, pin_memory=True)
    dst = torch.empty(tile_bytes, dtype=torch.uint8, device=dev)
    cp = []
    for _ in range(5):
        a, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        dst.copy_(src, non_blocking=True)
        e.record()
        torch.cuda.synchronize()
        cp.append(a.elapsed_time(e))
    link_gbs = tile_bytes / (float(np.median(cp)) / 1e3) / 1e9
    L, D, C = float(np.mean(lay_ms)), float(np.mean(dma_ms)), float(np.mean(cmp_ms))
    B = float(np.mean(moved))
    h2d = B / (D / 1e3) / 1e9
    overlap = max(0.0, min(1.0, (D + C - L) / max(min(D, C), 1e-9)))
    log(f"[bench] T={T} streamed: layer {L:.1f} ms, copies {D:.1f} ms for {B / 1e9:.2f} GB "
        f"({h2d:.1f} GB/s; plain pinned copy {link_gbs:.1f} GB/s), all-resident compute {C:.2f} ms, "
        f"overlap {overlap:.2f}, pool share of routed pairs {share:.2f}")
    cpu = None
    if not args.no_cpu_baseline:
        try:
            cpu = cpu_baseline(dict(cfg, Ts=[T]), W, T, rkw, args.cpu_seconds, dev)
        except Exception as exc:  # noqa: BLE001
            log(f"[bench] cpu baseline unavailable: {type(exc).__name__}: {exc}")
    line = {
        "metric": "MoE-layer ms & tok/s (decode T=1-4, prefill T=8192); HBM GB/s / MFMA % peak",
        "value": T / (L / 1e3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": L,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8-mfma/e4m3-pair x e4m3+f32-block",
        "data": "synthetic (seeded N(0,1) tokens, Zipf(1.1)+Gumbel logits, N(0,0.02) weights quantised)",
        "config": {"workload": args.workload, "T": T, "hidden": H, "intermediate": I,
                   "routed_experts": E, "shared_experts": NS, "top_k": K, "weights": cfg["fmt"],
                   "resident_experts": cfg["resident"], "tile_e": cfg["tile_e"],
                   "ring_slots": cfg["nslots"], "streamed_GB": B / 1e9,
                   "streamed_tiles": float(np.mean(tiles)), "copy_ms": D, "compute_ms": C,
                   "overlap": overlap, "pool_share_of_pairs": share,
                   "plain_pinned_copy_GBs": link_gbs},
        "roofline": {"bound": "host-link", "achieved": h2d, "peak": PCIE_GEN5_X16_GBS,
                     "unit": "GB/s", "frac": h2d / PCIE_GEN5_X16_GBS, "traffic": None,
                     "kernel": "xtu_copy_experts (hipMemcpyAsync, side stream)"},
        "cpu_baseline": cpu,
    }
    return line


def cpu_baseline(cfg, W, T, rkw, seconds, dev):
    """Reference engine (oracle/_ref) on the host cores over a bounded sample."""
    import numpy as np
    import torch

    import oracle
    from xtu_moe_amd.layer import route
    from xtu_moe_amd.synthetic import dense_experts

    E, NS, H, I, K = cfg["E"], cfg["NS"], cfg["H"], cfg["I"], cfg["K"]
    Ts = min(T, 256)   # prefill: a 256-token slice of the batch
    g = torch.Generator(device=dev).manual_seed(99)
    logits = torch.randn((Ts, E), generator=g, device=dev)
    w, i = route(logits, **rkw)
    ids = i.cpu().numpy()
    wts = w.cpu().numpy()
    used = np.unique(ids)
    remap = np.full(E, -1, np.int32)
    remap[used] = np.arange(len(used), dtype=np.int32)
    U = len(used)
    experts = list(used) + [E + s for s in range(NS)]
    dn = dense_experts(W, experts)
    cids = remap[ids]
    if NS:
        cids = np.concatenate([cids, np.tile(np.arange(U, U + NS, dtype=np.int32), (Ts, 1))], 1)
        wts = np.concatenate([wts, np.ones((Ts, NS), np.float32)], 1)
    x = oracle.f32_to_bf16_bits(np.random.default_rng(5).standard_normal((Ts, H)).astype(np.float32))
    threads = int(os.environ.get("XIAOTU_MOE_THREADS", "0") or 0) or (os.cpu_count() or 1)
    os.environ["XIAOTU_MOE_THREADS"] = str(threads)
    fmt = {"mxfp4": oracle.FMT_MXFP4, "nvfp4": oracle.FMT_NVFP4, "fp8": oracle.FMT_FP8,
           "bf16": oracle.FMT_BF16}[cfg["fmt"]]
    eng = oracle.RefEngine(fmt, U + NS, K + NS, H, I, dn["w13"], dn["s13"], dn["w2"], dn["s2"],
                           dn["gs13"], dn["gs2"], limit=cfg["limit"])
    L = oracle.ref_lib()
    if cfg["int8"]:
        L.xref_set_int8(1, 1 << 30)
    out = np.zeros((Ts, H), np.float32)
    for _ in range(2):
        eng.forward(x, cids, wts, out)
    times = []
    t_end = time.time() + seconds
    while time.time() < t_end or len(times) < 5:
        t0 = time.perf_counter()
        eng.forward(x, cids, wts, out)
        times.append(time.perf_counter() - t0)
    if cfg["int8"]:
        L.xref_set_int8(0, 0)
    med = float(np.median(times))
    isa = {2: "avx512_vnni", 1: "avx512", 0: "scalar"}[int(L.xref_isa())]
    return dict(value=Ts / med, unit="tok/s", cores=threads, kind="reference",
                ms_per_layer=med * 1e3, host=host_cpu(), engine_isa=isa,
                sample=(f"reference MOE_V2::forward_many ({isa}), {Ts} tokens x {K}+{NS} experts "
                        f"({U + NS} distinct), median of {len(times)} calls after 2 warm-ups"))


def host_cpu():
    """lscpu's model, sockets, NUMA nodes, logical CPUs and AVX-512 / AMX
    flags, plus the CPUs this process may run on."""
    info = {"cpus_allowed": len(os.sched_getaffinity(0))}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
    except (OSError, subprocess.SubprocessError):
        return info
    kv = {}
    for ln in out.splitlines():
        if ":" in ln:
            k, v = ln.split(":", 1)
            kv[k.strip()] = v.strip()
    for key, name in (("Model name", "model"), ("Socket(s)", "sockets"),
                      ("NUMA node(s)", "numa_nodes"), ("CPU(s)", "logical_cpus"),
                      ("Thread(s) per core", "threads_per_core")):
        if key in kv:
            info[name] = kv[key]
    flags = kv.get("Flags", "").split()
    info["isa"] = sorted(f for f in flags if f.startswith(("avx512", "amx")) or f == "avx2")
    return info


if __name__ == "__main__":
    main()
