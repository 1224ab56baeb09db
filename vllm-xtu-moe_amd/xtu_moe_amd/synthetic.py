"""Seeded synthetic expert layers built directly on the device.

Weights are drawn N(0, std) per expert chunk with a seeded device generator,
quantised by the formats module and packed to P16 in place, so a
DeepSeek-V3-sized layer (257 experts, ~6 GB as MXFP4) never exists densely in
host memory.
"""
from __future__ import annotations

import torch

from . import formats as F
from .layer import ExpertWeights


def synth_layer(fmt: int, E: int, n_shared: int, H: int, I: int, *, seed: int = 0,
                std: float = 0.02, device="cuda", chunk: int = 8) -> ExpertWeights:
    fmt = int(fmt)
    dev = torch.device(device)
    n = E + n_shared
    g = torch.Generator(device=dev).manual_seed(seed)

    def alloc(N, K, gu):
        rb = F.row_bytes(fmt, K)
        w = torch.empty((n, N * rb), dtype=torch.uint8, device=dev)
        if fmt in (F.FMT_MXFP4, F.FMT_NVFP4):
            s = torch.empty((n, F.scale_bytes(fmt, N, K)), dtype=torch.uint8, device=dev)
        elif fmt == F.FMT_FP8:
            s = torch.empty((n, (N // 128) * (K // 128)), dtype=torch.float32, device=dev)
        else:
            s = None
        gs = None
        if fmt == F.FMT_NVFP4:   # gate/up: one second-level scale per half
            gs = torch.empty((n, 2) if gu else (n,), dtype=torch.float32, device=dev)
        return w, s, gs

    w13, s13, gs13 = alloc(2 * I, H, True)
    w2, s2, gs2 = alloc(H, I, False)
    for e0 in range(0, n, chunk):
        e1 = min(n, e0 + chunk)
        for (w, s, gs, N, K, gu) in ((w13, s13, gs13, 2 * I, H, True), (w2, s2, gs2, H, I, False)):
            dense = torch.randn((e1 - e0, N, K), generator=g, device=dev) * std
            q, sc, gsc = (F.quantize_w13 if gu else F.quantize)(fmt, dense)
            del dense
            w[e0:e1] = F.pack_weight(fmt, q)
            if s is not None:
                s[e0:e1] = F.pack_scales(fmt, sc, N, K)
            if gs is not None:
                gs[e0:e1] = gsc
    return ExpertWeights(fmt, H, I, E, n_shared, w13, s13, w2, s2, gs13, gs2)


def dense_experts(W: ExpertWeights, experts) -> dict:
    """Dense checkpoint-layout host copies (numpy) of the given experts."""
    import numpy as np

    idx = torch.as_tensor(list(experts), dtype=torch.long, device=W.device)
    fmt = W.fmt
    out = {}
    for name, w, s, gs, N, K in (("13", W.w13, W.s13, W.gs13, 2 * W.I, W.H),
                                 ("2", W.w2, W.s2, W.gs2, W.H, W.I)):
        dw = F.unpack_weight(fmt, w[idx], N, K)
        out["w" + name] = (dw.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
                           if fmt == F.FMT_BF16 else dw.cpu().numpy())
        us = F.unpack_scales(fmt, None if s is None else s[idx], N, K)
        out["s" + name] = None if us is None else us.cpu().numpy()
        out["gs" + name] = None if gs is None else gs[idx].cpu().numpy()
    return out
