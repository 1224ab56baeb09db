"""Ring stage: a layer whose experts do not all fit in HBM, streamed from
pinned host memory through a ring of device slots while the GPU computes.

Mirrors the reference's layer-wise streamed prefill
(vllm_xiaotu_moe/gpu_prefill.py:2984-3095 ``gpu_moe_layer_from_engine_tiled``,
``stage_tiles`` / ``staging_tile_experts`` :1673-1720, ``staging_bytes``
:1722, ``prealloc_tile_ring`` / ``_tile_ring`` :2911-2981):

* the experts are cut into tiles of ``staging_tile_experts(E)`` experts; tile
  t is copied into slot ``t % nslots`` on a side stream (a ready event per
  slot) while the main stream computes the previous tile (a free event per
  slot keeps a slot from being overwritten before its kernels finish);
* the ring is allocated once per process and never freed (the side stream's
  writes can outlive a call);
* ``None`` means the layer cannot be streamed (caller falls back).

Differences by design: only experts that the batch routes to are copied (the
reference copies every tile); experts resident in a ``LayerPool`` are read in
place; and the layer is segmented once with the streamed experts renumbered
into consecutive buckets, so each tile is one bucket range of the grouped
GEMMs and the weighted unpermute runs once at the end -- the result is bit
for bit the all-resident layer's.
"""
from __future__ import annotations

import os

import torch

from .host_store import HostExpertStore, empty_slots
from .layer import _buf, _p, _stream, combine, expert_pass, gemm_tile_m, segmentation

DEFAULT_TILE_E = 48
_RINGS: dict = {}


def staging_tile_experts(n_experts: int) -> int:
    """Experts per staging tile: XTU_STAGE_TILE_E (clamped to [1, E-1]), else 48."""
    E = int(n_experts)
    if E <= 1:
        return max(1, E)
    try:
        v = int(os.environ.get("XTU_STAGE_TILE_E", "0") or 0)
    except (TypeError, ValueError):
        v = 0
    if v <= 0 or v >= E:
        v = DEFAULT_TILE_E
    return min(max(1, v), E - 1)


def stage_tiles(n_experts: int) -> list:
    """[(e0, e1), ...]: the expert range cut into staging tiles."""
    E = int(n_experts)
    t = staging_tile_experts(E)
    return [(e0, min(e0 + t, E)) for e0 in range(0, E, t)] if E > 0 else []


def staging_bytes(n_experts: int, hidden: int, inter: int, group_k: int = 32, ns: int = 2,
                  fmt=None, tile_e=None) -> int:
    """Device bytes of the ring for one layer shape (nslots x tile x expert)."""
    from . import formats as F
    fmt = F.FMT_MXFP4 if fmt is None else int(fmt)
    te = int(tile_e) if tile_e else staging_tile_experts(n_experts)
    per = (F.row_bytes(fmt, hidden) * 2 * inter + F.row_bytes(fmt, inter) * hidden
           + F.scale_bytes(fmt, 2 * inter, hidden) + F.scale_bytes(fmt, hidden, inter)
           + (8 if fmt == F.FMT_NVFP4 else 0))
    return int(max(2, int(ns)) * te * per)


class TileRing:
    """nslots device slots of tile_e experts each, a side stream and the
    ready / free events of every slot."""

    def __init__(self, store: HostExpertStore, tile_e: int, nslots: int, device):
        self.tile_e, self.nslots = int(tile_e), max(2, int(nslots))
        self.device = torch.device(device)
        self.slots = [empty_slots(store.fmt, store.H, store.I, self.tile_e, store, self.device)
                      for _ in range(self.nslots)]
        self.ready = [None] * self.nslots
        self.free = [None] * self.nslots
        self.side = torch.cuda.Stream(device=self.device)
        # bucket b of tile t sits at slot position b - t * tile_e = b % tile_e
        self._slot_map = {}

    def slot_map(self, n_buckets: int):
        m = self._slot_map.get(n_buckets)
        if m is None:
            m = (torch.arange(n_buckets, dtype=torch.int32, device=self.device) % self.tile_e)
            self._slot_map[n_buckets] = m
        return m

    def nbytes(self) -> int:
        tot = 0
        for s in self.slots:
            for name in ("w13", "s13", "w2", "s2", "gs13", "gs2"):
                t = getattr(s, name)
                tot += 0 if t is None else t.numel() * t.element_size()
        return tot


def _ring_for(store: HostExpertStore, tile_e: int, nslots: int, device) -> TileRing:
    key = (str(device), store.fmt, store.H, store.I, int(tile_e), max(2, int(nslots)))
    r = _RINGS.get(key)
    if r is None:
        r = TileRing(store, tile_e, nslots, device)
        _RINGS[key] = r
    return r


def prealloc_tile_ring(device, E, H, I, group_k=32, nslots: int = 2, store=None) -> int:
    """Allocate the ring before the KV cache is sized; returns its bytes."""
    if store is None:
        return 0
    return _ring_for(store, staging_tile_experts(E), nslots, device).nbytes()


class RingStats:
    """Bytes and timings of the last streamed layer (filled when asked)."""

    def __init__(self):
        self.bytes = 0
        self.tiles = 0
        self.dma_ms = 0.0      # sum over tiles of side-stream copy time
        self.events = []       # (start, end) copy events per tile

    def finish(self):
        torch.cuda.synchronize()
        self.dma_ms = sum(a.elapsed_time(b) for a, b in self.events)


def _as_store(engine):
    """The HostExpertStore behind `engine`: the store itself, or an engine
    object (``MOE_*``) exposing one through ``host_store()``; None else."""
    if isinstance(engine, HostExpertStore):
        return engine
    hs = getattr(engine, "host_store", None)
    return hs() if callable(hs) else None


def gpu_moe_layer_from_engine_tiled(engine, x, topk_ids, topk_weights, H: int, I: int, E: int,
                                    K: int, *, device, group_k: int = 32, nslots: int = 2,
                                    out=None, swiglu_limit: float = 0.0, pool=None, tile_e=None,
                                    out_dtype=torch.bfloat16, stats: RingStats | None = None):
    """One layer's routed (+ shared) experts with the weights streamed from
    `engine` (an ``MOE_*`` engine object or its HostExpertStore) through the
    tile ring; experts resident in `pool` (a LayerPool) are read in place.
    Returns out [T, H]: a new tensor (out_dtype) holding the layer, or the
    given `out` with the layer added to it (the reference accumulates into
    `out`, gpu_prefill.py:3020, gpu_prefill_fp8.py:1478).  None when the
    layer cannot be streamed (no host store, or a shape mismatch)."""
    device = torch.device(device)
    store = _as_store(engine)
    if store is None or store.H != int(H) or store.I != int(I) or store.E != int(E):
        return None
    engine = store
    T = x.shape[0]
    NS = engine.n_shared
    fmt = engine.fmt
    acc = out
    out = torch.empty((T, H), dtype=out_dtype if acc is None else acc.dtype, device=device)
    if T == 0 or K == 0:
        out.zero_()
        return out if acc is None else acc
    st = torch.cuda.current_stream(device)
    ids = topk_ids.to(torch.int32).contiguous()
    wts = topk_weights.float().contiguous()
    # which experts the batch routes to with a non-zero weight (one
    # device-to-host copy of E counts): zero-weight pairs are skipped
    valid = (ids >= 0) & (ids < E) & (wts != 0)
    counts = torch.bincount(ids[valid].long(), minlength=E)
    routed = torch.nonzero(counts > 0).flatten().tolist()
    resident = pool.resident_map() if pool is not None else {}
    streamed = [e for e in routed if e not in resident]
    res_list = [e for e in routed if e in resident]
    # buckets: streamed experts first (tile order), then the resident ones
    id_map_h = torch.full((E,), -1, dtype=torch.int32)
    for b, e in enumerate(streamed + res_list):
        id_map_h[e] = b
    id_map = id_map_h.to(device, non_blocking=True)
    te = int(tile_e) if tile_e else staging_tile_experts(E)
    ring = _ring_for(engine, te, nslots, device)
    f8ok = engine.fp8_scales_bounded()   # slot planes hold the store's scales
    bm = gemm_tile_m(fmt, False, H, I, ring.slots[0], f8ok)
    seg = segmentation(T, K, E, NS, bm, device, st)
    seg.run(ids, wts, id_map, True, st)
    y = _buf("ring_y", (max(seg.A, 1), H), torch.float32, device, st)
    ntile = (len(streamed) + te - 1) // te
    ring_map = ring.slot_map(E + NS)
    moved = 0

    def issue(t):
        nonlocal moved
        s = t % ring.nslots
        if ring.free[s] is not None:
            ring.side.wait_event(ring.free[s])
        exps = streamed[t * te:(t + 1) * te]
        with torch.cuda.stream(ring.side):
            ev0 = torch.cuda.Event(enable_timing=stats is not None)
            ev0.record(ring.side)
            moved += engine.copy_experts(exps, ring.slots[s], 0, ring.side)
            ev = torch.cuda.Event(enable_timing=stats is not None)
            ev.record(ring.side)
        ring.ready[s] = ev
        if stats is not None:
            stats.events.append((ev0, ev))

    ring.side.wait_stream(st)   # ids / routing are ready before the first copy
    for t in range(min(ntile, ring.nslots)):
        issue(t)
    kw = dict(swiglu_limit=swiglu_limit, stream=st, fp8_scales_ok=f8ok)
    # resident and shared experts first, from the pool's planes: they need no
    # copy, so their GEMMs run while the first tiles are in flight
    if res_list or NS:
        if pool is None:
            return None   # shared experts need a resident home
        bmap = pool.bucket_slot_map(streamed + res_list, E, NS)
        b_lo = len(streamed)
        if res_list:
            expert_pass(x, seg, pool.planes, b_lo, b_lo + len(res_list), y, slot_map=bmap, **kw)
        if NS:
            expert_pass(x, seg, pool.planes, E, E + NS, y, slot_map=bmap, **kw)
    for t in range(ntile):
        s = t % ring.nslots
        st.wait_event(ring.ready[s])
        b0, b1 = t * te, min((t + 1) * te, len(streamed))
        expert_pass(x, seg, ring.slots[s], b0, b1, y, slot_map=ring_map, **kw)
        ev = torch.cuda.Event()
        ev.record(st)
        ring.free[s] = ev
        if t + ring.nslots < ntile:
            issue(t + ring.nslots)
    combine(seg, y, wts, out, stream=st)
    if stats is not None:
        stats.bytes, stats.tiles = moved, ntile
    if acc is not None:
        acc.add_(out)
        return acc
    return out
