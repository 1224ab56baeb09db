"""Pool-miss split: resident experts on the GPU, the rest on the host.

The decode branch of the reference hook with a resident pool
(vllm_xiaotu_moe/mixed_experts.py:2956-3186): a pin mask splits the batch's
pairs into the resident part (pool slots) and the host part; on a side
stream the mask runs, then the resident part of the layer; on the main
stream the host engine's ``cpu_decode`` writes its share into ``out`` and the
resident partial is added once the side stream is done.  Every step is a
stream operation (event fork/join, kernels, copies, one host-function node),
so a whole split layer can be captured into a HIP graph and replayed.

``PinMaskFused`` mirrors the reference's fused mask
(vllm_xiaotu_moe/pin_mask_triton.py:96-148; torch semantics :73-85) on the
library's ``xtu_pin_split`` kernel.
"""
from __future__ import annotations

import torch

from . import _lib
from .cpu_experts import CpuExperts


def _p(t) -> int:
    return int(t.data_ptr())


_SIDE: dict = {}


def side_stream(device) -> torch.cuda.Stream:
    """One side stream per device, shared by every split layer: the layers
    run one after another on the main stream, and each forks onto the side
    stream after the previous layer joined back, so one stream orders them
    all and the library's per-stream scratch is held once, not per layer."""
    dev = torch.device(device)
    key = str(dev)
    s = _SIDE.get(key)
    if s is None:
        s = torch.cuda.Stream(device=dev)
        _SIDE[key] = s
    return s


def pin_split(ids, wts, slotmap, n_local: int, hits=None, out=None):
    """(cpu_ids, cpu_w, part_ids, part_w), each shaped like ids:
    with bad = id < 0 or id >= n_local, sl = slotmap[id], res = !bad and
    sl >= n_local (resident in slot sl - n_local):
    cpu_ids = 0 if res or bad else id; cpu_w = 0 if res or bad else w;
    part_ids = sl - n_local if res else -1; part_w = w if res else 0.
    hits (int64 device scalar, optional) += the number of resident pairs."""
    ids = ids.to(torch.int32).contiguous()
    wts = wts.to(torch.float32).contiguous()
    if slotmap.dtype != torch.int32 or slotmap.numel() < int(n_local):
        raise ValueError("slotmap must be int32 with n_local entries")
    if out is None:
        out = (torch.empty_like(ids), torch.empty_like(wts), torch.empty_like(ids),
               torch.empty_like(wts))
    cpu_ids, cpu_w, part_ids, part_w = out
    if hits is not None and (hits.dtype != torch.int64 or hits.numel() != 1):
        raise ValueError("hits must be one int64")
    _lib.call("xtu_pin_split", _p(ids), _p(wts), ids.numel(), _p(slotmap), int(n_local),
              _p(cpu_ids), _p(cpu_w), _p(part_ids), _p(part_w),
              0 if hits is None else _p(hits), torch.cuda.current_stream(ids.device).cuda_stream)
    return cpu_ids, cpu_w, part_ids, part_w


class PinMaskFused:
    """The reference's fused pin mask: ``step(ids, wts, slotmap, n_local)``
    -> (cpu_ids, cpu_w, part_ids) in buffers reused per (name, size), the
    resident pairs counted in a device int64 (``hits()``); the resident
    weights of the last step are ``part_w``."""

    def __init__(self, device):
        self.device = torch.device(device)
        self._bufs = {}
        self._hits = torch.zeros((), dtype=torch.int64, device=self.device)
        self.part_w = None

    def _buf(self, name, n, dtype):
        key = (name, n, dtype)
        t = self._bufs.get(key)
        if t is None:
            t = torch.empty(n, dtype=dtype, device=self.device)
            self._bufs[key] = t
        return t

    def step(self, ids, wts, slotmap, n_local: int):
        n = ids.numel()
        bufs = (self._buf("cpu_ids", n, torch.int32), self._buf("cpu_w", n, torch.float32),
                self._buf("part_ids", n, torch.int32), self._buf("part_w", n, torch.float32))
        cpu_ids, cpu_w, part_ids, part_w = pin_split(ids.reshape(-1), wts.reshape(-1), slotmap,
                                                     n_local, hits=self._hits, out=bufs)
        shp = ids.shape
        self.part_w = part_w.view(shp)
        return cpu_ids.view(shp), cpu_w.view(shp), part_ids.view(shp)

    def hits(self) -> torch.Tensor:
        """The device int64 count of resident pairs since the last reset, as
        the reference returns it (pin_mask_triton.py:146-148): callers read
        it with ``.item()`` and reset it with ``.zero_()``."""
        return self._hits


class PoolSplitLayer:
    """One layer split between a ``LayerPool`` (resident routed experts and
    the shared experts, on the GPU) and a host engine (every other routed
    expert); ``forward`` returns fp32 [T, H]."""

    def __init__(self, pool, cpu: CpuExperts, device=None):
        if cpu.H != pool.H or cpu.I != pool.I:
            raise ValueError("pool and host engine must be the same layer shape")
        self.pool, self.cpu = pool, cpu
        self.device = torch.device(device) if device is not None else pool.dev
        self.side = side_stream(self.device)
        self.mask = PinMaskFused(self.device)
        self.ev0, self.ev_mask, self.ev_done = (torch.cuda.Event(), torch.cuda.Event(),
                                                torch.cuda.Event())
        # tensors the side stream reads or writes, held until the next call:
        # the next call's fork waits for this call's join, so their memory is
        # never reused while a stream still uses it
        self._live = None

    def forward(self, x, topk_ids, topk_weights, *, out=None, note_routing=True, **kw):
        """out[T, H] fp32 = the layer over (x, topk_ids, topk_weights):
        pairs of resident experts and the shared experts on the GPU, the
        other pairs through the host engine (``kw`` goes to the resident
        layer: swiglu_limit, ...).  Inside a graph capture too."""
        T, K = topk_ids.shape
        H = self.pool.H
        h = x.to(torch.bfloat16).contiguous()
        ids = topk_ids.to(torch.int32).contiguous()
        wts = topk_weights.to(torch.float32).contiguous()
        if out is None:
            out = torch.empty((T, H), dtype=torch.float32, device=self.device)
        if out.dtype != torch.float32 or tuple(out.shape) != (T, H) or not out.is_contiguous():
            raise ValueError("out must be fp32 [T, H] contiguous")
        if note_routing:
            self.pool.note_routing(ids)
        main = torch.cuda.current_stream(self.device)
        self.ev0.record(main)
        with torch.cuda.stream(self.side):
            self.side.wait_event(self.ev0)
            cpu_ids, cpu_w, _ = self.mask.step(ids, wts, self.pool.slotmap, self.pool.n_local)
            self.ev_mask.record(self.side)
            partial = self.pool.forward(h, ids, wts, out_dtype=torch.float32, **kw)
            self.ev_done.record(self.side)
        self._live = (h, ids, wts, partial)
        main.wait_event(self.ev_mask)
        rc = self.cpu.cpu_decode(main.cuda_stream, T, K, h, cpu_ids, cpu_w, out)
        if rc:
            raise RuntimeError(f"host engine did not take the batch (cpu_decode returned {rc})")
        main.wait_event(self.ev_done)
        out.add_(partial)
        return out
