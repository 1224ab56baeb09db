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

from . import formats as F
from .host_store import HostExpertStore, empty_slots
from .layer import _buf, _p, _stream, combine, expert_pass, gemm_tile_m, segmentation

DEFAULT_TILE_E = 48
NSLOTS_ENV = "XIAOTU_GPF_STAGE_NSLOTS"
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
    fmt = F.FMT_MXFP4 if fmt is None else int(fmt)
    te = int(tile_e) if tile_e else staging_tile_experts(n_experts)
    per = (F.row_bytes(fmt, hidden) * 2 * inter + F.row_bytes(fmt, inter) * hidden
           + F.scale_bytes(fmt, 2 * inter, hidden) + F.scale_bytes(fmt, hidden, inter)
           + (8 if fmt == F.FMT_NVFP4 else 0))
    return int(max(2, int(ns)) * te * per)


class TileRing:
    """nslots device slots of tile_e experts each (in the device layout of
    format fmt for an H x I layer), a side stream and the ready / free events
    of every slot."""

    def __init__(self, fmt, H, I, tile_e: int, nslots: int, device):
        self.fmt, self.H, self.I = int(fmt), int(H), int(I)
        self.tile_e, self.nslots = int(tile_e), max(2, int(nslots))
        self.device = torch.device(device)
        self.slots = [empty_slots(self.fmt, self.H, self.I, self.tile_e, None, self.device)
                      for _ in range(self.nslots)]
        self.ready = [None] * self.nslots
        self.free = [None] * self.nslots
        self.side = torch.cuda.Stream(device=self.device)
        # bucket b of tile t sits at slot position b - t * tile_e = b % tile_e
        self._slot_map = {}
        self._shared_map = {}

    def fits(self, store: HostExpertStore) -> bool:
        """Whether the store's experts have the slots' per-expert layout."""
        return all(int(getattr(self.slots[0], n).shape[1:].numel()) *
                   getattr(self.slots[0], n).element_size() == store.row_bytes(n)
                   for n in ("w13", "s13", "w2", "s2", "gs13", "gs2")
                   if getattr(self.slots[0], n) is not None)

    def bind(self, store: HostExpertStore) -> None:
        """The slots are filled from `store`: their FP8 kernel choice follows
        the store's scale bound."""
        if store.fmt == F.FMT_FP8:
            ok = store.fp8_scales_bounded()
            for sl in self.slots:
                sl.slot_fp8_scales_ok = ok

    def slot_map(self, n_buckets: int):
        m = self._slot_map.get(n_buckets)
        if m is None:
            m = (torch.arange(n_buckets, dtype=torch.int32, device=self.device) % self.tile_e)
            self._slot_map[n_buckets] = m
        return m

    def shared_map(self, E: int, NS: int):
        """Bucket map of the shared experts streamed into one slot: bucket
        E + s -> slot position s."""
        key = (int(E), int(NS))
        m = self._shared_map.get(key)
        if m is None:
            m = torch.zeros(E + NS, dtype=torch.int32)
            m[E:] = torch.arange(NS, dtype=torch.int32)
            m = m.to(self.device)
            self._shared_map[key] = m
        return m

    def nbytes(self) -> int:
        tot = 0
        for s in self.slots:
            for name in ("w13", "s13", "w2", "s2", "gs13", "gs2"):
                t = getattr(s, name)
                tot += 0 if t is None else t.numel() * t.element_size()
        return tot


def _ring_for(fmt, H, I, tile_e: int, nslots: int, device) -> TileRing:
    """The process's ring for (device, format, shape, tile, slot count):
    allocated on first use and never freed."""
    key = (str(torch.device(device)), int(fmt), int(H), int(I), int(tile_e), max(2, int(nslots)))
    r = _RINGS.get(key)
    if r is None:
        r = TileRing(fmt, H, I, tile_e, nslots, device)
        _RINGS[key] = r
    return r


_GROUP_FMT = {32: F.FMT_MXFP4, 16: F.FMT_NVFP4, 1: F.FMT_BF16, 128: F.FMT_FP8}


def _nslots_default(nslots):
    if nslots is not None:
        return max(2, int(nslots))
    try:
        return max(2, int(os.environ.get(NSLOTS_ENV, "2") or 2))
    except (TypeError, ValueError):
        return 2


def prealloc_tile_ring(device, E, H, I, group_k=32, nslots=2, store=None, fmt=None) -> int:
    """Allocate the ring of a layer shape now -- before the KV cache is sized,
    so that the serving engine counts it (gpu_prefill.py:2911-2960) -- and
    return its bytes.  The format comes from the store, from `fmt`, or from
    the scale group as the reference passes it (32: MXFP4 e8m0, 16: NVFP4,
    1: BF16, 128: FP8).  Later ring calls of this shape, tile size and slot
    count use this ring.  nslots=None reads XIAOTU_GPF_STAGE_NSLOTS (2)."""
    E = int(E)
    if store is not None:
        fmt = store.fmt
    elif fmt is None:
        fmt = _GROUP_FMT.get(int(group_k))
        if fmt is None:
            raise ValueError(f"no expert format has scale groups of {group_k}")
    if E <= 1:
        return 0
    ring = _ring_for(fmt, H, I, staging_tile_experts(E), _nslots_default(nslots), device)
    if store is not None:
        if not ring.fits(store):
            raise ValueError("the store's experts do not fit this ring's slots")
        ring.bind(store)
    return ring.nbytes()


def prealloc_fp8_buffers(device, n_experts: int, hidden: int, inter: int, nslots=None) -> int:
    """The FP8 layer's ring, allocated now (gpu_prefill_fp8.py:247-258);
    returns its bytes."""
    return prealloc_tile_ring(device, n_experts, hidden, inter, 128, nslots, fmt=F.FMT_FP8)


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
                                    out=None, swiglu_limit: float = 0.0, swiglu_alpha: float = 1.0,
                                    swiglu_beta: float = 0.0, pool=None, tile_e=None,
                                    out_dtype=torch.bfloat16, stats: RingStats | None = None,
                                    int8: bool = False):
    """One layer's routed (+ shared) experts with the weights streamed from
    `engine` (an ``MOE_*`` engine object or its HostExpertStore) through the
    tile ring; experts resident in `pool` (a LayerPool) are read in place,
    and without a pool the shared experts are streamed as one more tile.
    Returns out [T, H]: a new tensor (out_dtype) holding the layer, or the
    given `out` with the layer added to it (the reference accumulates into
    `out`, gpu_prefill.py:3020, gpu_prefill_fp8.py:1478).  None when the
    layer cannot be streamed (no host store, a shape mismatch, more shared
    experts than a tile holds and no pool for them); nothing is queued then.
    int8: the INT8 ALIGN GEMMs (MXFP4), as the engine's int8_activation."""
    device = torch.device(device)
    store = _as_store(engine)
    if store is None or store.H != int(H) or store.I != int(I) or store.E != int(E):
        return None
    engine = store
    T = x.shape[0]
    NS = engine.n_shared
    fmt = engine.fmt
    te = int(tile_e) if tile_e else staging_tile_experts(E)
    if pool is not None and (pool.H != int(H) or pool.I != int(I) or pool.engine.fmt != fmt
                             or pool.n_local != int(E) or pool.n_shared != NS):
        return None
    if pool is None and NS > te:
        return None   # the shared experts need a slot (or a pool) to run from
    ring = _ring_for(fmt, H, I, te, nslots, device)
    if not ring.fits(engine):
        return None
    ring.bind(engine)
    acc = out
    out = torch.empty((T, H), dtype=out_dtype if acc is None else acc.dtype, device=device)
    if T == 0 or K == 0:
        out.zero_()
        return out if acc is None else acc
    st = torch.cuda.current_stream(device)
    if x.dtype != torch.bfloat16 or not x.is_contiguous():
        x = x.to(torch.bfloat16).contiguous()
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
    f8ok = engine.fp8_scales_bounded()   # slot planes hold the store's scales
    int8 = bool(int8) and fmt == F.FMT_MXFP4
    bm = gemm_tile_m(fmt, int8, H, I, ring.slots[0], f8ok)
    seg = segmentation(T, K, E, NS, bm, device, st)
    seg.run(ids, wts, id_map, True, st)
    y = _buf("ring_y", (max(seg.A, 1), H), torch.float32, device, st)
    ring_map = ring.slot_map(E + NS)
    # the tiles to stream: (experts, bucket range, bucket -> slot position)
    tiles = [(streamed[b0:b0 + te], b0, min(b0 + te, len(streamed)), ring_map)
             for b0 in range(0, len(streamed), te)]
    if pool is None and NS:
        tiles.append((list(range(E, E + NS)), E, E + NS, ring.shared_map(E, NS)))
    moved = 0

    def issue(t):
        nonlocal moved
        s = t % ring.nslots
        if ring.free[s] is not None:
            ring.side.wait_event(ring.free[s])
        with torch.cuda.stream(ring.side):
            ev0 = torch.cuda.Event(enable_timing=stats is not None)
            ev0.record(ring.side)
            moved += engine.copy_experts(tiles[t][0], ring.slots[s], 0, ring.side)
            ev = torch.cuda.Event(enable_timing=stats is not None)
            ev.record(ring.side)
        ring.ready[s] = ev
        if stats is not None:
            stats.events.append((ev0, ev))

    ring.side.wait_stream(st)   # ids / routing are ready before the first copy
    for t in range(min(len(tiles), ring.nslots)):
        issue(t)
    kw = dict(swiglu_limit=swiglu_limit, swiglu_alpha=swiglu_alpha, swiglu_beta=swiglu_beta,
              stream=st, fp8_scales_ok=f8ok, int8=int8)
    # resident and shared experts first, from the pool's planes: they need no
    # copy, so their GEMMs run while the first tiles are in flight
    if pool is not None and (res_list or NS):
        bmap = pool.bucket_slot_map(streamed + res_list, E, NS)
        b_lo = len(streamed)
        if res_list:
            expert_pass(x, seg, pool.planes, b_lo, b_lo + len(res_list), y, slot_map=bmap, **kw)
        if NS:
            expert_pass(x, seg, pool.planes, E, E + NS, y, slot_map=bmap, **kw)
    for t, (_, b0, b1, smap) in enumerate(tiles):
        s = t % ring.nslots
        st.wait_event(ring.ready[s])
        expert_pass(x, seg, ring.slots[s], b0, b1, y, slot_map=smap, **kw)
        ev = torch.cuda.Event()
        ev.record(st)
        ring.free[s] = ev
        if t + ring.nslots < len(tiles):
            issue(t + ring.nslots)
    combine(seg, y, wts, out, stream=st)
    if stats is not None:
        stats.bytes, stats.tiles = moved, len(tiles)
    if acc is not None:
        acc.add_(out)
        return acc
    return out
