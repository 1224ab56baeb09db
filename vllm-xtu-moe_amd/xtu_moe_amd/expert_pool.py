"""Hot-expert resident pool: a fixed set of device slots holding the most
used experts of a layer, the slot map the kernels read, routing counts kept
on the device, and the swap policy.

Mirrors vllm_xiaotu_moe/expert_pool.py: ``plan_swap`` (:60-112),
``load_pin_table`` (:119-137), ``LayerPool`` (:139-448: planes, slotmap,
``as_slot``, ``swap_out``, ``note_routing``, ``swap_in``, ``maybe_adapt``),
``select_local_topk`` (:451) and ``build_layer_pool`` (:479).  Slot-map
encoding as in the reference: one device int32 per local expert, value
< n_local = not resident (the value is the local id), value >= n_local =
resident in slot (value - n_local).

The planes are allocated once and never freed; swaps rewrite slot contents
on a side stream and flip the map only after the copy (an event orders the
main stream behind it).  Shared experts, when the layer has them, take the
slots after the pinned ones and never leave.
"""
from __future__ import annotations

import os
import struct

import torch

from .host_store import HostExpertStore, empty_slots
from .layer import moe_forward

ENV_ON = "XTU_PIN"
ENV_TABLE = "XTU_PIN_TABLE"
ENV_WINDOW = "XTU_PIN_WINDOW"       # forwards between re-plans (0: never)
ENV_HYST = "XTU_PIN_HYST"           # hysteresis: candidate > victim * (1 + hyst)
ENV_MAXSWAP = "XTU_PIN_MAXSWAP"     # swaps per re-plan (<= 0: max(1, nslots // 4))
ENV_PRESERVE = "XTU_PIN_PRESERVE_OLDEST"

_PIN_HDR = "<4sIIII"   # magic, version, n_layers, n_experts, n_entries (20 bytes)


def plan_swap(resident, counts, nslots: int, *, hyst: float = 0.25, maxswap: int = 0,
              min_hits: int = 1, preserve_oldest: bool = False):
    """Which residents to evict and which experts to load, from the window's
    hit counts (a pure policy: no tensors, no device).

    * victims: the coldest residents, ties broken by slot age (oldest first,
      or newest first with preserve_oldest);
    * candidates: non-residents with at least min_hits hits, hottest first;
    * candidate i replaces victim i only if its count exceeds the victim's by
      the hysteresis factor (1 + hyst);
    * at most maxswap (or max(1, nslots // 4)) swaps; empty pool: none.
    """
    if int(nslots) <= 0 or not resident:
        return [], []
    res = list(resident)
    k = int(maxswap) if int(maxswap) > 0 else max(1, int(nslots) // 4)
    age = (lambda i: -i) if preserve_oldest else (lambda i: i)
    victims = sorted(range(len(res)), key=lambda i: (int(counts.get(res[i], 0)), age(i)))[:k]
    in_res = set(res)
    cands = sorted(((e, int(c)) for e, c in counts.items()
                    if e not in in_res and int(c) >= int(min_hits)), key=lambda kv: -kv[1])[:k]
    evict, load = [], []
    for (e, c), vi in zip(cands, victims):
        victim = res[vi]
        if c > int(counts.get(victim, 0)) * (1.0 + float(hyst)):
            evict.append(victim)
            load.append(e)
    # never evict something hotter than what replaces it
    assert not (set(evict) & set(load))
    assert all(int(counts.get(v, 0)) <= int(counts.get(l, 0)) for v, l in zip(evict, load))
    return evict, load


def pin_enabled() -> bool:
    return os.environ.get(ENV_ON, "0") == "1"


def load_pin_table(path: str) -> dict:
    """XTUP v1 pin table -> {layer: [experts, hottest first]}.  Header
    <magic 'XTUP', version 1, n_layers, n_experts, n_entries> (5 x 4 bytes),
    then n_entries (layer u16, expert u16) records in descending frequency."""
    with open(path, "rb") as f:
        buf = f.read()
    magic, ver, _n_layers, _n_exp, n_ent = struct.unpack_from(_PIN_HDR, buf, 0)
    if magic != b"XTUP" or ver != 1:
        raise ValueError(f"bad pin table {magic!r} v{ver}")
    hdr = struct.calcsize(_PIN_HDR)
    if len(buf) < hdr + 4 * n_ent:
        raise ValueError("truncated pin table")
    out: dict = {}
    for i in range(n_ent):
        layer, e = struct.unpack_from("<HH", buf, hdr + 4 * i)
        out.setdefault(int(layer), []).append(int(e))
    return out


def write_pin_table(path: str, table: dict, n_layers: int, n_experts: int) -> int:
    """Inverse of load_pin_table; entries in layer order, each layer's list
    as given (hottest first).  Returns the entry count."""
    entries = [(int(l), int(e)) for l in sorted(table) for e in table[l]]
    with open(path, "wb") as f:
        f.write(struct.pack(_PIN_HDR, b"XTUP", 1, int(n_layers), int(n_experts), len(entries)))
        for l, e in entries:
            f.write(struct.pack("<HH", l, e))
    return len(entries)


def select_local_topk(g_list, em_global_to_local, e_local: int, cap: int) -> list:
    """Up to `cap` local expert ids in table order (hottest first): global ids
    mapped through em_global_to_local (None: identity), out-of-rank and
    repeated ids dropped before the cut; cap <= 0 keeps them all."""
    e_local, cap = int(e_local), int(cap)
    if em_global_to_local is None:
        seq = (int(g) for g in g_list)
    else:
        emt = [int(v) for v in torch.as_tensor(em_global_to_local).flatten().tolist()]
        seq = (emt[int(g)] for g in g_list if 0 <= int(g) < len(emt))
    sel, seen = [], set()
    for loc in seq:
        if 0 <= loc < e_local and loc not in seen:
            seen.add(loc)
            sel.append(loc)
            if cap > 0 and len(sel) >= cap:
                break
    return sel


class ReadySlot:
    """What a layer entry needs of a resident slot set: planes, the event
    after which they are valid, the slot map and the local expert count."""

    def __init__(self, planes, ready, slotmap, n_local):
        self.bufs = planes
        self.ready = ready
        self.busy = None
        self.slotmap = slotmap
        self.n_local = n_local


class LayerPool:
    """One layer's pool (nslots = number of pinned experts)."""

    def __init__(self, engine, device, hidden: int, inter: int, group_k: int,
                 n_local: int, pinned_local: list, layer_idx: int, layout: str = "mxfp4",
                 topk: int = 0):
        from .formats import FMT_NAMES
        from .ring import _as_store
        store = _as_store(engine)
        if store is None:
            raise ValueError("the pool needs an engine with a host store (MOE_* or "
                             "HostExpertStore)")
        engine = store
        if FMT_NAMES.get(engine.fmt) != str(layout):
            raise ValueError(f"pool layout {layout!r} does not match the store's "
                             f"{FMT_NAMES.get(engine.fmt)!r} weights")
        self.engine, self.dev = engine, torch.device(device)
        self.H, self.I, self.gk = int(hidden), int(inter), int(group_k)
        self.n_local, self.layer_idx, self.layout = int(n_local), int(layer_idx), str(layout)
        self.n_shared = engine.n_shared
        self.pinned = [int(e) for e in pinned_local]
        if len(set(self.pinned)) != len(self.pinned) or any(not 0 <= e < self.n_local for e in self.pinned):
            raise ValueError("pinned experts must be distinct local ids")
        self.nslots = len(self.pinned)
        self.expert_of = list(self.pinned)            # slot -> expert (-1: empty)
        self.swaps_in = self.swaps_out = 0
        self._side = None
        self._slot = None
        S = self.nslots + self.n_shared
        self.planes = empty_slots(engine.fmt, self.H, self.I, max(S, 1), engine, self.dev)
        sm = torch.arange(self.n_local, dtype=torch.int32)
        for s, e in enumerate(self.pinned):
            sm[e] = self.n_local + s
        self.slotmap = sm.to(self.dev)
        self._hits = torch.zeros(self.n_local, dtype=torch.int32, device=self.dev)
        self._win_t = torch.zeros((), dtype=torch.int64, device=self.dev)
        # load the pinned experts and the shared ones (after the routed slots)
        engine.copy_experts(self.pinned, self.planes, 0)
        if self.n_shared:
            engine.copy_experts(range(engine.E, engine.E + self.n_shared), self.planes, self.nslots)
        torch.cuda.synchronize(self.dev)
        if 0 < int(topk) and self.nslots < int(topk):
            print(f"[xtu-pin] layer{layer_idx}: {self.nslots} slots < top_k={int(topk)}: the pool "
                  "cannot hold one token's experts", flush=True)

    # ------------------------------------------------------------- views
    def resident_map(self) -> dict:
        return {e: s for s, e in enumerate(self.expert_of) if e >= 0}

    def bucket_slot_map(self, order, E: int, NS: int):
        """Device int32 [E + NS]: bucket b (expert order[b]) -> its slot; the
        shared buckets E.. -> the shared slots."""
        res = self.resident_map()
        m = torch.zeros(E + NS, dtype=torch.int32)
        for b, e in enumerate(order):
            if e in res:
                m[b] = res[e]
        for s in range(NS):
            m[E + s] = self.nslots + s
        return m.to(self.dev, non_blocking=True)

    def as_slot(self) -> ReadySlot:
        if self._slot is None:
            ev = torch.cuda.Event()
            ev.record()
            self._slot = ReadySlot(self.planes, ev, self.slotmap, self.n_local)
        return self._slot

    # ------------------------------------------------------------- layer
    def forward(self, x, topk_ids, topk_weights, **kw):
        """The resident part of the layer: pairs whose expert is resident (and
        the shared experts); pairs of other experts contribute nothing (the
        caller adds their share: ring stage or CPU)."""
        E = self.n_local
        sm = self.slotmap
        id_map = torch.where(sm >= E, torch.arange(E, dtype=torch.int32, device=self.dev),
                             torch.full_like(sm, -1))
        slot_map = torch.cat([torch.where(sm >= E, sm - E, torch.zeros_like(sm)),
                              torch.arange(self.nslots, self.nslots + self.n_shared,
                                           dtype=torch.int32, device=self.dev)])
        from .layer import ExpertWeights
        # bucket b's weights are slot slot_map[b] of the pool planes, which
        # hold nslots + n_shared experts, not E + n_shared
        W = ExpertWeights(self.engine.fmt, self.H, self.I, E, self.n_shared, self.planes.w13,
                          self.planes.s13, self.planes.w2, self.planes.s2, self.planes.gs13,
                          self.planes.gs2, mutable=True)
        kw.setdefault("fp8_scales_ok", self.engine.fp8_scales_bounded())
        return moe_forward(x, topk_ids, topk_weights, W, id_map=id_map, slot_map=slot_map, **kw)

    # ------------------------------------------------------------- swaps
    def swap_out(self, s: int) -> int:
        """Return slot s's expert to the non-resident path; the plane stays."""
        e = self.expert_of[s]
        if e is None or e < 0:
            return -1
        self.slotmap[e] = e
        self.expert_of[s] = -1
        self.swaps_out += 1
        return int(e)

    def note_routing(self, topk_ids) -> None:
        """Accumulate this batch's expert hits on the device (no host sync,
        no allocation of persistent state: safe inside graph capture)."""
        if self.nslots == 0:
            return
        idx = topk_ids.reshape(-1).to(torch.long)
        bad = (idx < 0) | (idx >= self.n_local)
        safe = torch.where(bad, torch.zeros_like(idx), idx)
        w = torch.where(bad, torch.zeros_like(idx, dtype=torch.int32),
                        torch.ones_like(idx, dtype=torch.int32))
        self._hits.index_add_(0, safe, w)
        self._win_t += 1

    def swap_in(self, gp, new_expert: int, s: int):
        """Load new_expert into slot s on a side stream, then flip the map
        (the main stream waits for the copy first).  Returns s, or None if
        the expert is already resident.  `gp` is the reference's loader
        module argument (its gpu_prefill module, expert_pool.py:353); the
        copy here is the host store's own, so it is accepted and unused."""
        if new_expert in self.expert_of:
            return None
        if self._side is None:
            self._side = torch.cuda.Stream(device=self.dev)
        st = torch.cuda.current_stream(self.dev)
        self._side.wait_stream(st)   # the slot's last readers finish first
        with torch.cuda.stream(self._side):
            self.engine.copy_experts([int(new_expert)], self.planes, s, self._side)
            ev = torch.cuda.Event()
            ev.record(self._side)
        st.wait_event(ev)
        self.slotmap[int(new_expert)] = self.n_local + s
        self.expert_of[s] = int(new_expert)
        self.swaps_in += 1
        return s

    def maybe_adapt(self, gp=None, *, staging_active: bool = True, window=None) -> int:
        """Re-plan once per window of forwards (one device-to-host copy of the
        counts); returns the number of experts swapped in.  Does nothing
        unless the caller states that no staging burst is in flight."""
        if self.nslots == 0 or getattr(self, "_hits", None) is None or staging_active:
            return 0
        w = int(window if window is not None else os.environ.get(ENV_WINDOW, "0") or 0)
        if w <= 0 or int(self._win_t.item()) < w:
            return 0
        counts = self._hits.tolist()
        self._hits.zero_()
        self._win_t.zero_()
        cd = {e: c for e, c in enumerate(counts) if c}
        evict, load = plan_swap(self.expert_of, cd, self.nslots,
                                hyst=float(os.environ.get(ENV_HYST, "0.25") or 0.25),
                                maxswap=int(os.environ.get(ENV_MAXSWAP, "0") or 0),
                                preserve_oldest=os.environ.get(ENV_PRESERVE, "0") == "1")
        n = 0
        for victim, e in zip(evict, load):
            if victim not in self.expert_of:
                continue
            s = self.expert_of.index(victim)
            self.swap_out(s)
            if self.swap_in(gp, e, s) is not None:
                n += 1
        return n


def build_layer_pool(engine, device, hidden: int, inter: int, group_k: int, e_local: int,
                     layer_idx: int, em_global_to_local, topk: int = 0, layout: str = "mxfp4",
                     table_path: str = None, require_pin: bool = True, cap: int = 0):
    """A LayerPool for `layer_idx` from the pin table (XTU_PIN_TABLE), or None
    when pinning is off (XTU_PIN != 1 and require_pin), the table is missing,
    or it lists no local expert for this layer."""
    if require_pin and not pin_enabled():
        return None
    path = table_path or os.environ.get(ENV_TABLE, "")
    if not path or not os.path.exists(path):
        return None
    g_list = load_pin_table(path).get(int(layer_idx), [])
    sel = select_local_topk(g_list, em_global_to_local, e_local, cap)
    if not sel:
        return None
    return LayerPool(engine, device, hidden, inter, group_k, e_local, sel, layer_idx,
                     layout=layout, topk=topk)
