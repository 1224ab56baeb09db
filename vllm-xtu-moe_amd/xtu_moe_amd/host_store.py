"""Host-resident expert store: every expert of a layer in pinned host memory,
in the same packed layout the device kernels read (one row of bytes per
expert and weight plane), so that moving an expert to HBM is one contiguous
DMA per plane.

This is the device-side view of what the reference's CPU engine exposes to
its GPU ring (``shard_geometry`` / ``pin_hostbufs`` /
``copy_hostbuf_to_device``, xiaotu_moe/csrc/binding.cpp:1368-1437): there the
rows live in NUMA shards of the engine and are transposed to K-major on the
GPU after the copy; here they are stored ready to use.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .layer import ExpertWeights, _p, _stream

PLANES = ("w13", "s13", "w2", "s2", "gs13", "gs2")


class HostExpertStore:
    """Pinned host copy of a layer's experts (routed [0, E), shared after)."""

    def __init__(self, fmt, H, I, E, n_shared, planes: dict):
        self.fmt, self.H, self.I, self.E, self.n_shared = int(fmt), int(H), int(I), int(E), int(n_shared)
        self.planes = planes   # name -> pinned CPU tensor [E + NS, row] (or None)

    @classmethod
    def from_weights(cls, W: ExpertWeights) -> "HostExpertStore":
        planes = {}
        for name in PLANES:
            t = getattr(W, name)
            if t is None:
                planes[name] = None
                continue
            h = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
            h.copy_(t, non_blocking=False)
            planes[name] = h
        return cls(W.fmt, W.H, W.I, W.E, W.n_shared, planes)

    @property
    def n_experts(self) -> int:
        return self.E + self.n_shared

    def row_bytes(self, name) -> int:
        t = self.planes[name]
        return 0 if t is None else t[0].numel() * t.element_size()

    def expert_bytes(self) -> int:
        return sum(self.row_bytes(n) for n in PLANES)

    # -- the engine host-buffer surface the ring consumes -------------------
    def shard_geometry(self) -> dict:
        """Bytes per expert of each plane (one shard: the whole host store)."""
        return dict(ns=1, **{f"{n}_bytes": self.row_bytes(n) for n in PLANES})

    def pin_hostbufs(self) -> int:
        """Number of pinned host planes (already pinned at construction)."""
        return sum(1 for t in self.planes.values() if t is not None)

    def copy_experts(self, experts, dst: ExpertWeights, first_slot: int = 0, stream=None) -> int:
        """Asynchronously copy `experts` into slots first_slot.. of `dst` on
        `stream`; returns the bytes moved."""
        ex = [int(e) for e in experts]
        if not ex:
            return 0
        if min(ex) < 0 or max(ex) >= self.n_experts:
            raise ValueError(f"expert ids out of range [0, {self.n_experts})")
        arr = (ctypes.c_int32 * len(ex))(*ex)
        st = _stream(stream)
        moved = 0
        for name in PLANES:
            src = self.planes[name]
            d = getattr(dst, name)
            if src is None:
                continue
            if d is None:
                raise ValueError(f"destination has no {name} plane")
            rb = self.row_bytes(name)
            drb = d[0].numel() * d.element_size()
            if first_slot + len(ex) > d.shape[0] or drb != rb:
                raise ValueError(f"{name}: destination slots/rows do not fit")
            _lib.call("xtu_copy_experts", len(ex), ctypes.addressof(arr), _p(src), rb,
                      _p(d) + first_slot * drb, drb, rb, st)
            moved += rb * len(ex)
        return moved

    def copy_hostbuf_to_device(self, which: int, expert: int, dst_ptr: int, stream=None) -> int:
        """One plane of one expert to a device address (which: 0 w13, 1 w2,
        2 s13, 3 s2 -- the reference's plane numbering); returns bytes."""
        name = {0: "w13", 1: "w2", 2: "s13", 3: "s2"}[int(which)]
        src = self.planes[name]
        if src is None:
            return 0
        rb = self.row_bytes(name)
        arr = (ctypes.c_int32 * 1)(int(expert))
        _lib.call("xtu_copy_experts", 1, ctypes.addressof(arr), _p(src), rb, int(dst_ptr), rb, rb,
                  _stream(stream))
        return rb


def empty_slots(fmt, H, I, n_slots, like: HostExpertStore, device) -> ExpertWeights:
    """Device planes for n_slots experts in the store's layout."""
    planes = {}
    for name in PLANES:
        src = like.planes[name]
        planes[name] = None if src is None else torch.empty((n_slots,) + tuple(src.shape[1:]),
                                                            dtype=src.dtype, device=device)
    return ExpertWeights(fmt, H, I, n_slots, 0, planes["w13"], planes["s13"], planes["w2"],
                         planes["s2"], planes["gs13"], planes["gs2"])
