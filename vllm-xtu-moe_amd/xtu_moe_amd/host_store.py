"""Host-resident expert store: every expert of a layer in pinned host memory,
in the packed layout the device kernels read, cut into the reference
engine's NUMA-node shards, so that moving an expert (or a tile of experts)
to HBM is a few contiguous or pitched DMAs.

This is what the reference's CPU engine exposes to its GPU ring
(xiaotu_moe/csrc/python_binding/binding.cpp:1368-1437 ``shard_geometry`` /
``pin_hostbufs`` / ``copy_hostbuf_to_device`` / ``copy_hostbuf_to_device_2d``;
shard layout moe_v2.hpp:1742-1860): node n of ns holds, for every expert
e, gate rows [n*crows, (n+1)*crows) then up rows [I + n*crows, ...) of w13
(crows = I/ns), and rows [n*H/ns, (n+1)*H/ns) of w2; the scale planes are one
copy each.  Here a row of an expert is a row of the P16 panel layout, so
crows must be a multiple of the 16-row panel and the shards, laid side by
side per expert, are exactly the device block: a node's slice of a tile of
consecutive experts is one pitched copy.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from . import formats as F
from .layer import ExpertWeights, _p, _stream, fp8_block_scales_bounded, register_slot_planes

PLANES = ("w13", "s13", "w2", "s2", "gs13", "gs2")
# the reference's plane numbering for copy_hostbuf_to_device(which, ...);
# 4 and 5 (NVFP4 per-expert global scales, one fp32 each) have no
# counterpart there
WHICH = {0: "w13", 1: "w2", 2: "s13", 3: "s2", 4: "gs13", 5: "gs2"}


class HostExpertStore:
    """Pinned host copy of a layer's experts (routed [0, E), shared after)."""

    def __init__(self, fmt, H, I, E, n_shared, planes: dict, ns: int = 1, pin: bool = True,
                 group_k: int = 0):
        """pin=False keeps the shards in pageable memory (a host-only store
        for the host engine; the DMA paths want pinned memory).  group_k:
        INT4's k per scale."""
        self.fmt, self.H, self.I, self.E, self.n_shared = int(fmt), int(H), int(I), int(E), int(n_shared)
        self.group_k = int(group_k)
        ns = int(ns)
        if ns < 1 or self.I % (16 * ns) or self.H % (16 * ns):
            raise ValueError(f"{ns} shards need I={I} and H={H} divisible by 16*{ns}")
        self.ns = ns
        self.rb13 = F.row_bytes(self.fmt, self.H)
        self.rb2 = F.row_bytes(self.fmt, self.I)
        self.w13_crows, self.w2_crows = self.I // ns, self.H // ns
        self.w13_cbytes = self.w13_crows * self.rb13
        self.w2_cbytes = self.w2_crows * self.rb2
        n = self.n_experts
        # node shards of the weight planes, single copies of the scales
        self.w13_shard, self.w2_shard = [], []
        w13, w2 = planes["w13"], planes["w2"]
        for node in range(ns):
            a = torch.empty((n, 2 * self.w13_cbytes), dtype=torch.uint8, pin_memory=pin)
            g0 = node * self.w13_cbytes
            u0 = self.I * self.rb13 + g0
            a[:, :self.w13_cbytes].copy_(w13[:, g0:g0 + self.w13_cbytes])
            a[:, self.w13_cbytes:].copy_(w13[:, u0:u0 + self.w13_cbytes])
            self.w13_shard.append(a)
            b = torch.empty((n, self.w2_cbytes), dtype=torch.uint8, pin_memory=pin)
            d0 = node * self.w2_cbytes
            b.copy_(w2[:, d0:d0 + self.w2_cbytes])
            self.w2_shard.append(b)
        self.planes = {name: planes[name] for name in ("s13", "s2", "gs13", "gs2")}

    @classmethod
    def from_weights(cls, W: ExpertWeights, ns: int = 1, pin: bool = True) -> "HostExpertStore":
        planes = {}
        for name in PLANES:
            t = getattr(W, name)
            if t is None:
                planes[name] = None
                continue
            if name in ("w13", "w2"):   # copied into the pinned node shards
                planes[name] = t.cpu()
                continue
            h = torch.empty(t.shape, dtype=t.dtype, pin_memory=pin)
            h.copy_(t, non_blocking=False)
            planes[name] = h
        return cls(W.fmt, W.H, W.I, W.E, W.n_shared, planes, ns=ns, pin=pin,
                   group_k=getattr(W, "group_k", 0))

    @property
    def n_experts(self) -> int:
        return self.E + self.n_shared

    def fp8_scales_bounded(self) -> bool:
        """FP8: fp8_block_scales_bounded over every expert's scales, read from
        the host copy once (device slot planes filled from this store hold
        these scales, so their kernel choice follows this answer)."""
        if self.fmt != F.FMT_FP8:
            return False
        if getattr(self, "_fp8_pos", None) is None:
            self._fp8_pos = fp8_block_scales_bounded(self.planes["s13"], self.planes["s2"])
        return self._fp8_pos

    def row_bytes(self, name) -> int:
        """Bytes of one expert in plane `name`."""
        if name == "w13":
            return 2 * self.I * self.rb13
        if name == "w2":
            return self.H * self.rb2
        t = self.planes[name]
        return 0 if t is None else t[0].numel() * t.element_size()

    def expert_bytes(self) -> int:
        return sum(self.row_bytes(n) for n in PLANES)

    # -- the engine host-buffer surface the ring consumes -------------------
    def shard_geometry(self) -> dict:
        """Keys and meaning as the reference engine's shard_geometry()."""
        s13, s2 = self.planes["s13"], self.planes["s2"]
        nb = lambda t: 0 if t is None else t.numel() * t.element_size()
        return dict(ns=self.ns,
                    w13_node_bytes=self.n_experts * 2 * self.w13_cbytes,
                    w2_node_bytes=self.n_experts * self.w2_cbytes,
                    w13_scale_bytes=nb(s13), w2_scale_bytes=nb(s2),
                    w13_crows=self.w13_crows, w13_cbytes=self.w13_cbytes,
                    w2_crows=self.w2_crows, w2_cbytes=self.w2_cbytes)

    def pin_hostbufs(self) -> int:
        """Number of pinned host buffers (all are pinned at construction)."""
        bufs = self.w13_shard + self.w2_shard + [t for t in self.planes.values() if t is not None]
        return sum(1 for t in bufs if t.is_pinned())

    def host_wbuf(self, which: int, node: int):
        """The host buffer `which` (0 w13 shard, 1 w2 shard, 2 s13, 3 s2, 4
        gs13, 5 gs2) of `node`; None when there is none."""
        which, node = int(which), int(node)
        if which == 0:
            return self.w13_shard[node] if 0 <= node < self.ns else None
        if which == 1:
            return self.w2_shard[node] if 0 <= node < self.ns else None
        name = WHICH.get(which)
        return None if name is None else self.planes.get(name)

    def copy_hostbuf_to_device(self, which: int, node: int, dst_ptr: int, stream=None) -> int:
        """Whole buffer `which` of `node` to the device address dst_ptr;
        returns the bytes queued (0 when there is no such buffer)."""
        src = self.host_wbuf(which, node)
        if src is None:
            return 0
        n = src.numel() * src.element_size()
        _lib.call("xtu_copy_2d", int(dst_ptr), n, _p(src), n, n, 1, _stream(stream))
        return n

    def copy_hostbuf_to_device_2d(self, which: int, node: int, src_off: int, dst: int,
                                  dpitch: int, spitch: int, width: int, height: int,
                                  stream=None) -> int:
        """Pitched copy out of buffer `which` of `node`, starting `src_off`
        bytes in: height rows of width bytes, source pitch spitch, destination
        pitch dpitch; returns width*height, or 0 on a bad request."""
        src = self.host_wbuf(which, node)
        src_off, dpitch, spitch = int(src_off), int(dpitch), int(spitch)
        width, height = int(width), int(height)
        if src is None or height <= 0 or width <= 0 or spitch <= 0 or dpitch <= 0:
            return 0
        size = src.numel() * src.element_size()
        if src_off < 0 or width > spitch or width > dpitch \
                or src_off + (height - 1) * spitch + width > size:
            return 0
        _lib.call("xtu_copy_2d", int(dst), int(dpitch), _p(src) + int(src_off), int(spitch),
                  int(width), int(height), _stream(stream))
        return int(width) * int(height)

    # -- whole experts into device slots ------------------------------------
    def copy_experts(self, experts, dst: ExpertWeights, first_slot: int = 0, stream=None) -> int:
        """Asynchronously copy `experts` into slots first_slot.. of `dst` on
        `stream` (per node: the gate and up rows of w13 and the rows of w2,
        then the scales); returns the bytes moved."""
        ex = [int(e) for e in experts]
        if not ex:
            return 0
        if min(ex) < 0 or max(ex) >= self.n_experts:
            raise ValueError(f"expert ids out of range [0, {self.n_experts})")
        arr = (ctypes.c_int32 * len(ex))(*ex)
        pa = ctypes.addressof(arr)
        st = _stream(stream)

        def dst_of(name):
            d = getattr(dst, name)
            if d is None:
                raise ValueError(f"destination has no {name} plane")
            drb = d[0].numel() * d.element_size()
            if first_slot + len(ex) > d.shape[0] or drb != self.row_bytes(name):
                raise ValueError(f"{name}: destination slots/rows do not fit")
            return _p(d) + first_slot * drb, drb

        moved = 0
        d13, e13 = dst_of("w13")
        d2, e2 = dst_of("w2")
        c13, c2 = self.w13_cbytes, self.w2_cbytes
        for node in range(self.ns):
            sh = self.w13_shard[node]
            g_off = node * c13
            u_off = self.I * self.rb13 + g_off
            _lib.call("xtu_copy_experts", len(ex), pa, _p(sh), 2 * c13, d13 + g_off, e13, c13, st)
            _lib.call("xtu_copy_experts", len(ex), pa, _p(sh) + c13, 2 * c13, d13 + u_off, e13,
                      c13, st)
            _lib.call("xtu_copy_experts", len(ex), pa, _p(self.w2_shard[node]), c2,
                      d2 + node * c2, e2, c2, st)
            moved += len(ex) * (2 * c13 + c2)
        for name in ("s13", "s2", "gs13", "gs2"):
            src = self.planes[name]
            if src is None:
                continue
            rb = self.row_bytes(name)
            d, drb = dst_of(name)
            _lib.call("xtu_copy_experts", len(ex), pa, _p(src), rb, d, drb, rb, st)
            moved += rb * len(ex)
        return moved


def slot_plane_specs(fmt, H, I) -> dict:
    """Per-expert (shape, dtype) of each device plane of a layer in format
    `fmt` (None: the format has no such plane): the packed P16 weights and
    scale groups, FP8's fp32 block scales, NVFP4's fp32 second-level scales
    (gate and up for w13, one for w2)."""
    fmt, H, I = int(fmt), int(H), int(I)
    u8, f32 = torch.uint8, torch.float32
    spec = {"w13": ((2 * I * F.row_bytes(fmt, H),), u8), "w2": ((H * F.row_bytes(fmt, I),), u8),
            "s13": None, "s2": None, "gs13": None, "gs2": None}
    if fmt == F.FMT_FP8:
        spec["s13"] = (((2 * I // 128) * (H // 128),), f32)
        spec["s2"] = (((H // 128) * (I // 128),), f32)
    elif fmt in (F.FMT_MXFP4, F.FMT_NVFP4):
        spec["s13"] = ((F.scale_bytes(fmt, 2 * I, H),), u8)
        spec["s2"] = ((F.scale_bytes(fmt, H, I),), u8)
        if fmt == F.FMT_NVFP4:
            spec["gs13"], spec["gs2"] = ((2,), f32), ((), f32)   # gate, up / down
    elif fmt != F.FMT_BF16:
        raise ValueError(f"no device slot layout for format {fmt}")
    return spec


def empty_slots(fmt, H, I, n_slots, like: HostExpertStore | None, device) -> ExpertWeights:
    """Device planes for n_slots experts in the store's layout (or, with no
    store, the format's: slot_plane_specs)."""
    if like is not None:
        planes = {"w13": torch.empty((n_slots, like.row_bytes("w13")), dtype=torch.uint8,
                                     device=device),
                  "w2": torch.empty((n_slots, like.row_bytes("w2")), dtype=torch.uint8,
                                    device=device)}
        for name in ("s13", "s2", "gs13", "gs2"):
            src = like.planes[name]
            planes[name] = None if src is None else torch.empty(
                (n_slots,) + tuple(src.shape[1:]), dtype=src.dtype, device=device)
    else:
        planes = {name: None if sp is None else torch.empty((n_slots,) + sp[0], dtype=sp[1],
                                                            device=device)
                  for name, sp in slot_plane_specs(fmt, H, I).items()}
    f8ok = like.fp8_scales_bounded() if (like is not None and int(fmt) == F.FMT_FP8) else None
    return register_slot_planes(
        ExpertWeights(fmt, H, I, n_slots, 0, planes["w13"], planes["s13"], planes["w2"],
                      planes["s2"], planes["gs13"], planes["gs2"], mutable=True,
                      fp8_scales_ok=f8ok))
