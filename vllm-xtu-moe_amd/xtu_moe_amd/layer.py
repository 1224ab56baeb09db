"""One MoE layer's routed (+ shared) experts on the gfx950 HIP library.

    routing output -> segmentation -> gate/up (+ SwiGLU-clamp) -> down
                   -> weighted unpermute (combine)

The shapes follow the reference's layer entry (vllm_xiaotu_moe/gpu_prefill.py:
2566-2780 gpu_moe_layer): x [T, H] bf16, topk_ids [T, K] int32, topk_weights
[T, K] fp32, output [T, H] bf16 (or fp32).  Device buffers are cached per
shape for the life of the process (as the reference does with its
`_reuse_moe` / tile rings), so steady-state calls allocate nothing.
"""
from __future__ import annotations

import math
import os

import torch

from . import _lib
from .formats import (FMT_BF16, FMT_FP8, FMT_INT4, FMT_MXFP4, FMT_NVFP4, INT4_GROUPS,
                      int4_group_of, pack_scales, pack_weight)

DECODE_MAX_TOKENS = 16
DECODE_TILE = 16     # rows per work slot of the decode kernels (one MFMA M tile)
SMALL_MAX_PAIRS = 1024
# The one-launch router routes 4 tokens at a time in one workgroup (the tiny
# path one wave per token); past this many tokens the multi-workgroup router
# plus the three-launch segmentation is faster (measured: 95 us vs ~17 us for
# 128 tokens over 8 experts).
SMALL_ROUTE_MAX_TOKENS = 16
TINY_MAX_PAIRS = 64  # pairs one workgroup routes and segments (xtu_route_segment_small's tiny path)
LANE_ROUTE_MAX_E, LANE_ROUTE_MAX_K = 32, 8   # softmax routed by one thread per token


def _p(t) -> int:
    return 0 if t is None else int(t.data_ptr())


def _stream(stream=None) -> int:
    if stream is None:
        return int(torch.cuda.current_stream().cuda_stream)
    return int(stream.cuda_stream) if hasattr(stream, "cuda_stream") else int(stream)


def _fp8_block_scales(s):
    """FP8 block scales as fp32: uint8 planes holding fp32 bytes (last dim
    x4, the reference pool's form) are reinterpreted, other float dtypes
    converted by value."""
    if s is None or s.dtype == torch.float32:
        return s
    if s.dtype == torch.uint8:
        return s.contiguous().view(torch.float32)
    if not s.is_floating_point():
        raise ValueError(f"FP8 block scales of dtype {s.dtype}")
    return s.float()


def gate_up_scales2(gs13):
    """NVFP4 second-level scales of w13 as fp32 [N, 2] (gate, up), the
    layout the kernels read (gs13[2 slot], gs13[2 slot + 1]): the
    checkpoint's w13_weight_scale_2 [E, 2] as it is, a per-expert [E]
    vector repeated; None stays None."""
    if gs13 is None:
        return None
    g = gs13.to(torch.float32)
    if g.dim() == 1:
        g = g[:, None].expand(-1, 2)
    if g.dim() != 2 or g.shape[1] != 2:
        raise ValueError(f"gate/up second-level scales must be [E] or [E, 2], got {tuple(g.shape)}")
    return g.contiguous()


class ExpertWeights:
    """Resident weights of one layer in the P16 panel layout.

    Experts [0, E) are routed; [E, E + n_shared) are shared experts that every
    token uses with weight 1.  Tensors: w13/w2 u8 [E+NS, bytes], s13/s2 (u8
    P16 scales for fp4, fp32 block scales for fp8, None for bf16), NVFP4
    second-level scales gs13 fp32 [E+NS, 2] (gate, up; a [E+NS] vector is
    taken as one scale for both halves) and gs2 fp32 [E+NS], or None.
    """

    def __init__(self, fmt, H, I, E, n_shared, w13, s13, w2, s2, gs13=None, gs2=None, *,
                 mutable=False, group_k=0, fp8_scales_ok=None):
        self.fmt, self.H, self.I, self.E, self.n_shared = int(fmt), int(H), int(I), int(E), int(n_shared)
        # INT4 (WNA16): k per fp32 scale (the planes keep [N][K/group_k] per expert)
        self.group_k = int(group_k) if self.fmt == FMT_INT4 else 0
        if self.fmt == FMT_INT4 and self.group_k not in INT4_GROUPS:
            raise ValueError(f"INT4 weights need group_k in {INT4_GROUPS}, got {group_k}")
        gs13 = gate_up_scales2(gs13)
        self.w13, self.s13, self.w2, self.s2, self.gs13, self.gs2 = w13, s13, w2, s2, gs13, gs2
        # mutable: the planes are restaged in place (ring / pool slots), so
        # nothing derived from them is cached; their FP8 scale bound is the
        # source's (the host store they are filled from), stated here
        self.mutable = bool(mutable)
        self.slot_fp8_scales_ok = fp8_scales_ok
        self._i8 = None
        self._i8_fb = None
        self._i8_emm = None
        self._mxs = None
        self._fp8_pos = None
        if self.H % 256 or self.I % 128:
            raise ValueError(f"unsupported shape H={H} I={I} (need H % 256 == 0, I % 128 == 0)")
        rows = {t.shape[0] for t in (w13, s13, w2, s2, gs13, gs2) if t is not None}
        if len(rows) != 1:
            raise ValueError(f"weight planes hold different expert counts: {sorted(rows)}")
        # FP8: the prefill kernel choice is fixed when the weights are built,
        # so a graph captured later takes the same kernel as eager calls
        if self.fmt == FMT_FP8 and not self.mutable:
            self.fp8_scales_bounded()

    @property
    def n_experts(self) -> int:
        return self.E + self.n_shared

    @property
    def n_slots(self) -> int:
        """Experts the planes hold.  Equal to n_experts, except for slot
        planes (a pool's, a ring's) read through a slot_map, which may hold
        fewer: whatever is derived from the planes covers these rows only."""
        return int(self.w13.shape[0])

    @property
    def device(self):
        return self.w13.device

    def __iter__(self):
        """(w13, s13, w2, s2): callers that star-unpack a pool's planes into a
        layer entry (``gpu_moe_layer(x, ids, w, *pool.planes, ...)``) pass
        the device-layout planes, which the entries use in place."""
        return iter((self.w13, self.s13, self.w2, self.s2))

    @classmethod
    def from_dense(cls, fmt, w13, s13, w2, s2, gs13=None, gs2=None, *, E=None, n_shared=0,
                   device=None):
        """Pack dense checkpoint tensors (experts [0,E) routed, the rest shared)."""
        fmt = int(fmt)
        Et = w13.shape[0]
        N13 = w13.shape[1]
        I = N13 // 2
        H = w2.shape[1]
        dev = torch.device(device) if device is not None else w13.device

        def mv(t):
            return None if t is None else t.to(dev).contiguous()

        if fmt == FMT_FP8:
            s13, s2 = _fp8_block_scales(s13), _fp8_block_scales(s2)
        gk = 0
        if fmt == FMT_INT4:
            gk = int4_group_of(s13, H)
            if int4_group_of(s2, I) != gk:
                raise ValueError("INT4 gate/up and down scales use different groups")
        w13p = pack_weight(fmt, mv(w13))
        w2p = pack_weight(fmt, mv(w2))
        s13p = pack_scales(fmt, mv(s13), 2 * I, H)
        s2p = pack_scales(fmt, mv(s2), H, I)
        E = Et - n_shared if E is None else E
        return cls(fmt, H, I, E, n_shared, w13p, s13p, w2p, s2p, mv(gs13), mv(gs2), group_k=gk)

    # ------------------------------------------------------ MXFP4 pair GEMM
    def mx_pair_scales(self, stream=None):
        """(s13, s2) re-laid step-major for the MXFP4 exact-pair GEMM:
        [slot][K/64][N/16][16][2] e8m0 bytes.  Built once (a device kernel over
        the packed scale groups) unless the planes are mutable, then per call
        into a scratch buffer."""
        if self._mxs is not None and not self.mutable:
            return self._mxs
        if self.fmt != FMT_MXFP4:
            raise ValueError("step-major pair scales are for MXFP4 weights")
        n, dev, st = self.n_slots, self.device, _stream(stream)
        out = []
        for (sc, N, K, tag) in ((self.s13, 2 * self.I, self.H, "mxs13"), (self.s2, self.H, self.I, "mxs2")):
            shape = (n, N * (K // 32))
            t = (_buf(tag, shape, torch.uint8, dev, st) if self.mutable else
                 torch.empty(shape, dtype=torch.uint8, device=dev))
            _lib.call("xtu_mx_pair_scales", _p(sc), n, N, K, sc.stride(0) * sc.element_size(),
                      _p(t), st)
            out.append(t)
        if self.mutable:
            return tuple(out)
        self._mxs = tuple(out)
        return self._mxs

    # ---------------------------------------------------------------- FP8
    def fp8_scales_bounded(self) -> bool:
        """fp8_block_scales_bounded over this layer's scales (checked once;
        inside a graph capture an unchecked set counts as unbounded, so the
        capture takes the kernel without ratios)."""
        if self._fp8_pos is not None:
            return self._fp8_pos
        if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
            return False
        self._fp8_pos = fp8_block_scales_bounded(self.s13, self.s2)
        return self._fp8_pos

    # ---------------------------------------------------------------- INT8
    def int8_planes(self):
        """Shifted int8 weights + per-row emin for the INT8 ALIGN path (MXFP4
        only).  Rows whose e8m0 spread exceeds 3 are marked (emin 0xFF); their
        output columns take the fp32 fallback (int8_fallback_cols).  Cached,
        except for mutable planes, whose contents change between calls: for
        those each call prepares them again (and int8_fallback_cols then
        returns that call's fallback columns)."""
        if self._i8 is not None and not self.mutable:
            return self._i8
        if self.fmt != FMT_MXFP4:
            raise ValueError("the INT8-activation path needs MXFP4 (e8m0) weights")
        n = self.n_slots
        dev = self.device
        out = []
        st = _stream()
        dmax = torch.zeros(1, dtype=torch.int32, device=dev)
        emm = []
        for (w, s, N, K) in ((self.w13, self.s13, 2 * self.I, self.H), (self.w2, self.s2, self.H, self.I)):
            w8 = torch.empty((n, N * K), dtype=torch.uint8, device=dev)
            emin = torch.empty((n, N), dtype=torch.uint8, device=dev)
            _lib.call("xtu_i8_prepare", _p(w), _p(s), n, N, K, _p(w8), _p(emin), _p(dmax), st)
            out += [w8, emin]
            # each slot's smallest e8m0 byte: the offset guard's weight side
            mm = torch.empty(n, dtype=torch.int32, device=dev)
            _lib.call("xtu_i8_emin_min", _p(s), n, N, K, _p(mm), st)
            emm.append(mm)
        self._i8_emm = tuple(emm)
        self._i8_fb = None
        if int(dmax.item()) > 3:   # marked rows: CSR lists of their output columns per slot
            I = self.I
            m13 = (out[1] == I8_MARKED).cpu()
            m13 = (m13[:, :I] | m13[:, I:])            # column pair n: gate row n or up row n
            m2 = (out[3] == I8_MARKED).cpu()
            self._i8_fb = _csr_cols(m13, dev) + _csr_cols(m2, dev)
        self._i8 = tuple(out)
        return self._i8

    def int8_emin_min(self):
        """(eminmin13, eminmin2): int32 [slots], each slot's smallest e8m0 byte
        of its gate/up and down matrices (the offset guard's weight side),
        from the same preparation as int8_planes (for mutable planes: the
        last one, as int8_fallback_cols)."""
        if self._i8 is None:
            self.int8_planes()
        return self._i8_emm

    def int8_fallback_cols(self):
        """None, or (start13, cols13, start2, cols2): per weight slot, the
        gate/up column pairs and down columns the fp32 fallback computes."""
        if self._i8 is None:
            self.int8_planes()
        return self._i8_fb


# Slot planes (pool, ring) by the address of their w13 plane: a caller that
# hands their tensors to a layer entry (``*pool.planes``) gets these weights
# back, with their FP8 scale bound, instead of a new set checked per call.
# The planes are never freed, so an address cannot be reused under an entry.
_SLOT_PLANES: dict = {}


def register_slot_planes(W: "ExpertWeights") -> "ExpertWeights":
    _SLOT_PLANES[(str(W.w13.device), W.w13.data_ptr())] = W
    return W


def slot_planes_of(w13, s13, w2, s2):
    """The registered slot planes whose four tensors these are, else None."""
    W = _SLOT_PLANES.get((str(w13.device), w13.data_ptr()))
    if W is None:
        return None
    same = all(a is not None and b is not None and a.data_ptr() == b.data_ptr()
               and tuple(a.shape) == tuple(b.shape)
               for a, b in ((W.w13, w13), (W.s13, s13), (W.w2, w2), (W.s2, s2))
               if not (a is None and b is None))
    return W if same and W.w13.shape == w13.shape else None


I8_MARKED = 0xFF   # emin byte of a weight row that takes the fp32 fallback


def _csr_cols(mask, device):
    """Per-row boolean mask [slots][N] -> device (start [slots + 1], cols) int32."""
    counts = mask.sum(1).to(torch.int32)
    start = torch.zeros(mask.shape[0] + 1, dtype=torch.int32)
    start[1:] = torch.cumsum(counts, 0)
    cols = mask.nonzero()[:, 1].to(torch.int32)   # row-major: slot order, then column order
    if cols.numel() == 0:
        cols = torch.zeros(1, dtype=torch.int32)
    return start.to(device), cols.to(device)


def _cap_rows(n: int) -> int:
    """Row capacity for n rows: the next power of two (at least 16), so a
    stream of varying token counts settles on a few allocations."""
    n = max(int(n), 1)
    return max(16, 1 << (n - 1).bit_length())


class _SegBuffers:
    """Device buffers of the segmentation for (K, E, NS, bm) and up to
    `cap_t` tokens (the sizes grow monotonically with T)."""

    def __init__(self, cap_t, K, E, NS, bm, device):
        self.cap_t = cap_t
        A = cap_t * K + cap_t * NS
        NB = E + NS + 1
        i32 = dict(dtype=torch.int32, device=device)
        self.ws = torch.empty(int(_lib.call("xtu_segment_workspace_bytes", cap_t, K, E, NS)),
                              dtype=torch.uint8, device=device)
        Am = max(A, 1)
        self.sorted_pair = torch.empty(Am, **i32)
        self.sorted_tok = torch.empty(Am, **i32)
        self.sorted_wts = torch.empty(Am, dtype=torch.float32, device=device)
        self.inv = torch.empty(Am, **i32)
        self.seg_start = torch.empty(NB + 1, **i32)
        self.active = torch.empty(NB, **i32)
        self.n_active = torch.empty(1, **i32)
        mt = int(_lib.call("xtu_segment_max_tiles", cap_t, K, E, NS, bm))
        self.tile_expert = torch.empty(mt, **i32)
        self.tile_row0 = torch.empty(mt, **i32)
        self.n_tiles = torch.empty(1, **i32)
        self.expert_tile_start = torch.empty(NB + 1, **i32)


class _Segmentation:
    """The segmentation of one call of T tokens, over cached buffers sized
    for at least T tokens (views of their first rows)."""

    def __init__(self, bufs: _SegBuffers, T, K, E, NS, bm):
        self.T, self.K, self.E, self.NS, self.bm = T, K, E, NS, bm
        A = T * K + T * NS
        NB = E + NS + 1
        self.A, self.NB = A, NB
        self._bufs = bufs
        Am = max(A, 1)
        self.ws = bufs.ws
        self.sorted_pair = bufs.sorted_pair[:Am]
        self.sorted_tok = bufs.sorted_tok[:Am]
        self.sorted_wts = bufs.sorted_wts[:Am]
        self.inv = bufs.inv[:Am]
        self.seg_start = bufs.seg_start
        self.active = bufs.active
        self.n_active = bufs.n_active
        # grid bound of the GEMMs for this T (the buffers may hold more)
        self.max_tiles = int(_lib.call("xtu_segment_max_tiles", T, K, E, NS, bm))
        self.tile_expert = bufs.tile_expert[:self.max_tiles]
        self.tile_row0 = bufs.tile_row0[:self.max_tiles]
        self.n_tiles = bufs.n_tiles
        self.expert_tile_start = bufs.expert_tile_start

    def run(self, ids, wts, id_map=None, drop_zero=True, stream=None):
        _lib.call("xtu_segment", _p(ids), _p(wts), _p(id_map), self.T, self.K, self.E, self.NS,
                  int(drop_zero), self.bm, _p(self.ws), _p(self.sorted_pair), _p(self.sorted_tok),
                  _p(self.sorted_wts), _p(self.inv), _p(self.seg_start), _p(self.active),
                  _p(self.n_active), _p(self.tile_expert), _p(self.tile_row0), _p(self.n_tiles),
                  _p(self.expert_tile_start), _stream(stream))
        return self

    def run_small(self, mode, ids, wts, *, logits=None, bias=None, n_group=1, topk_group=1,
                  routed_scaling=1.0, renormalize=True, id_map=None, drop_zero=True, stream=None):
        """Routing (mode 0 softmax / 1 grouped sigmoid, writing ids and wts) or
        given ids (mode 2) plus the whole segmentation, in one launch."""
        _lib.call("xtu_route_segment_small", int(mode), _p(logits), _p(bias), _p(ids), _p(wts),
                  self.T, self.E, self.K, int(n_group), int(topk_group), float(routed_scaling),
                  int(renormalize), _p(id_map), self.NS, int(drop_zero), self.bm,
                  _p(self.sorted_pair), _p(self.sorted_tok), _p(self.sorted_wts), _p(self.inv),
                  _p(self.seg_start), _p(self.active), _p(self.n_active), _p(self.tile_expert),
                  _p(self.tile_row0), _p(self.n_tiles), _p(self.expert_tile_start),
                  _stream(stream))
        return self

    @property
    def small(self) -> bool:
        return self.A <= SMALL_MAX_PAIRS and self.E + self.NS + 1 <= 2048 and self.K <= 16

    def tile_range_ptrs(self, b0: int, b1: int):
        """Device pointers to expert_tile_start[b0] and [b1] (m-tile range of buckets [b0, b1))."""
        base = _p(self.expert_tile_start)
        return base + 4 * int(b0), base + 4 * int(b1)


# Scratch per (shape, device, stream), kept for the life of the process and
# never freed: a captured HIP graph may hold their addresses, and a buffer
# used on a stream other than the one it was allocated on must not return to
# the caching allocator while that stream may still read it.  The streams a
# process runs layers on are few (torch hands out streams from a fixed pool
# per device; the split layers share one side stream per device), so this
# is bounded by a few copies of each buffer.
_SEG_CACHE: dict = {}
_BUF_CACHE: dict = {}
# Buffers replaced by a larger one (kept for the same reason).  Growth is
# geometric (power-of-two rows), so they total less than the live ones.
_RETIRED: list = []


def segmentation(T, K, E, NS, bm, device, stream=None) -> _Segmentation:
    """The segmentation of T tokens, over buffers kept per (shape without T,
    device, stream): calls on one stream run in order and share them;
    another stream gets its own.  Capacity grows to the next power of two
    of T, so varying batch sizes allocate O(log T_max) times in total."""
    st = _stream(stream)
    key = (K, E, NS, bm, str(device), st)
    b = _SEG_CACHE.get(key)
    if b is None or b.cap_t < T:
        if b is not None:
            _RETIRED.append(b)
        b = _SegBuffers(_cap_rows(T), K, E, NS, bm, device)
        _SEG_CACHE[key] = b
    return _Segmentation(b, T, K, E, NS, bm)


def _buf(name, shape, dtype, device, stream=None):
    """Scratch buffer `name` of shape (rows, *tail) for (device, stream): the
    first `rows` rows of a cached buffer whose row capacity is a power of two
    (stream-ordered reuse; concurrent streams get their own)."""
    rows, tail = int(shape[0]), tuple(int(s) for s in shape[1:])
    st = _stream(stream)
    key = (name, tail, dtype, str(device), st)
    t = _BUF_CACHE.get(key)
    if t is None or t.shape[0] < rows:
        if t is not None:
            _RETIRED.append(t)
        t = torch.empty((_cap_rows(rows),) + tail, dtype=dtype, device=device)
        _BUF_CACHE[key] = t
    return t[:rows]


def _same_device(dev, **tensors):
    """Every given tensor lives on CUDA device `dev` (the kernels take raw
    device pointers: a host or other-device pointer must never reach them)."""
    for name, t in tensors.items():
        if t is not None and (not t.is_cuda or t.device != dev):
            raise ValueError(f"{name} is on {t.device}, expected {dev}")


def route(logits, *, top_k, scoring="softmax", renormalize=True, bias=None, n_group=1,
          topk_group=1, routed_scaling_factor=1.0, ids_out=None, wts_out=None, stream=None):
    """Top-k routing on the GPU.  Returns (topk_weights fp32 [T,K], topk_ids int32 [T,K])."""
    lg = logits.float().contiguous() if logits.dtype != torch.float32 or not logits.is_contiguous() else logits
    T, E = lg.shape
    dev = lg.device
    if not lg.is_cuda:
        raise ValueError("logits must be a CUDA tensor")
    _same_device(dev, bias=bias, ids_out=ids_out, wts_out=wts_out)
    ids = ids_out if ids_out is not None else torch.empty((T, top_k), dtype=torch.int32, device=dev)
    wts = wts_out if wts_out is not None else torch.empty((T, top_k), dtype=torch.float32, device=dev)
    st = _stream(stream)
    if scoring == "softmax":
        _lib.call("xtu_route_softmax_topk", _p(lg), T, E, top_k, int(renormalize), _p(ids), _p(wts), st)
    elif scoring == "sigmoid":
        b = None if bias is None else bias.float().contiguous()
        _lib.call("xtu_route_grouped_sigmoid", _p(lg), _p(b), T, E, int(n_group), int(topk_group),
                  top_k, float(routed_scaling_factor), int(renormalize), _p(ids), _p(wts), st)
    else:
        raise ValueError(f"unsupported scoring function {scoring!r}")
    return wts, ids


INT8_MIN_TOKENS_ENV = "XIAOTU_MOE_INT8_VNNI_MIN_TOKENS"
INT8_FORCE_ENV = "XIAOTU_MOE_INT8_ALIGN"


def int8_align_on(T: int, allowed: bool = True) -> bool:
    """Whether a call of T tokens takes the INT8 ALIGN path, as the reference
    engine gates it (xiaotu_moe/csrc/moe/moe_v2_packed4_w4a8.inc:409-433,
    xiaotu_int8_mode.h): XIAOTU_MOE_INT8_ALIGN=1 forces it; otherwise the
    format must allow it (`allowed`) and T must reach
    XIAOTU_MOE_INT8_VNNI_MIN_TOKENS (default 160; <= 0 turns it off).  Below
    the threshold the layer runs with bf16 activations (at decode sizes the
    int8 quantisation buys nothing: the layer streams weights)."""
    try:
        if int(os.environ.get(INT8_FORCE_ENV, "0") or 0) != 0:
            return True
    except ValueError:
        pass
    if not allowed:
        return False
    try:
        m = int(os.environ.get(INT8_MIN_TOKENS_ENV, "160") or 160)
    except ValueError:
        m = 160
    return m > 0 and int(T) >= m


INT8_ENV = "XIAOTU_MOE_INT8"
INT8_VNNI_ENV = "XIAOTU_MOE_INT8_VNNI"


def int8_dispatch(fmt: int):
    """Whether the quant-method hook lets a layer of this format take the
    INT8 ALIGN path, from the reference's switches (vllm_xiaotu_moe/
    mixed_experts.py:1457-1484): XIAOTU_MOE_INT8=0 turns it off (None: not
    even when forced); XIAOTU_MOE_INT8_ALIGN=1 forces it at every batch size
    (int8_align_on); XIAOTU_MOE_INT8=1 allows it from the token gate on.
    Only MXFP4 weights qualify (e8m0 scales make the int8 weights exact).
    Unlike the reference, whose CPU engine allows it by default for MXFP4
    (there int8 runs ~1.5x its fp32 path), it is off by default: on the GPU
    the MXFP4 MFMA path is faster and keeps the layer within the fp32 bar,
    while the power-of-two per-row int8 activations leave ~2e-2 of rel-L2.
    XIAOTU_MOE_INT8_VNNI=1 (the reference's older VNNI scheme) is refused."""
    if int(fmt) != FMT_MXFP4:
        return False
    v = os.environ.get(INT8_ENV)
    if v == "0":
        return None
    if os.environ.get(INT8_VNNI_ENV, "0") == "1" and os.environ.get(INT8_FORCE_ENV, "0") != "1":
        raise NotImplementedError("XIAOTU_MOE_INT8_VNNI=1: the older int8 VNNI scheme is not "
                                  "provided; XIAOTU_MOE_INT8_ALIGN=1 selects the ALIGN path")
    return v == "1"


def decode_max_tiles(A: int, max_active: int) -> int:
    """Upper bound on the 16-row tiles of a decode batch of A pairs over at
    most max_active non-empty expert buckets: a bucket of n rows has
    ceil(n/16) <= 1 + (n-1)//16 tiles, so the total is at most
    b + (A - b)//16 for b non-empty buckets, which grows with b."""
    return int(max_active) + max(int(A) - int(max_active), 0) // DECODE_TILE


MXFP4_PREFILL_ENV = "XTU_MXFP4_PREFILL"
FP8_PREFILL_ENV = "XTU_FP8_PREFILL"


FP8_RATIO_MAX = 2.0 ** 32


def fp8_block_scales_bounded(*scales) -> bool:
    """Every FP8 block scale finite and positive, and the largest at most
    2^32 times the smallest: the 32x32x64 kernel carries its accumulators in
    units of the current block's scale and rescales them by s(kb-1)/s(kb) at
    each block boundary, which this bound keeps far from fp32 overflow."""
    lo, hi = math.inf, 0.0
    for s in scales:
        s = s.float()
        if not bool(torch.isfinite(s).all()):
            return False
        lo, hi = min(lo, float(s.min())), max(hi, float(s.max()))
    return lo > 0 and hi <= lo * FP8_RATIO_MAX


def fp8_pair32_use(W, scales_ok=None) -> bool:
    """Whether an FP8 layer's prefill GEMMs run on the 32x32x64 kernel with
    LDS-staged operands (xtu_f8_pair_*): XTU_FP8_PREFILL "auto" (default) or
    "pair32", the shape fits and the block scales are bounded
    (fp8_block_scales_bounded; the kernel rescales by their ratios), checked
    once on immutable weights and, for slot planes (pool, ring), stated by the
    caller (`scales_ok`) or by the planes themselves (from the host store's
    copy); else the 16x16x128 kernel (xtu_gemm8_*, "v1")."""
    if W is None or W.fmt != FMT_FP8:
        return False
    if os.environ.get(FP8_PREFILL_ENV, "auto") == "v1":
        return False
    if not bool(_lib.call("xtu_f8_pair_fits", int(W.H), int(W.I))):
        return False
    if W.mutable:
        return bool(scales_ok if scales_ok is not None else W.slot_fp8_scales_ok)
    return W.fp8_scales_bounded()


# "auto": the 32x32x64 MXFP4 kernel on activation triples (fp6/fp6/fp4
# pieces, double-rate MFMA) where it takes the shape, else the bf16-operand
# kernels; "tri" the same; "pair" exact e4m3 pairs (the 32x32x64 kernel
# where it fits, else the 16x16x128 one); "bf16" the bf16-operand kernels;
# "duo" the triples' first two pieces only (two double-rate MFMAs instead
# of three; opt-in: measured at DeepSeek-V3 T = 8192 it is 16% faster per
# layer but leaves max-abs 2.6e-2 against the dequantised-fp32 layer, past
# the 2e-2 bar, so it is never chosen by default)
MXFP4_PREFILL_DEFAULT = "auto"
_TRI_MODES = ("auto", "tri", "duo")


def _mx_fits(H: int, I: int) -> bool:
    return bool(_lib.call("xtu_mx_pair_fits", int(H), int(I)))


def pair_gemm(fmt: int, H: int = 0, I: int = 0) -> bool:
    """Whether the grouped GEMMs of this format (layer shape H, I) run on
    the scaled f8f6f4 MFMA: FP8 always (exact e4m3 activation pairs); MXFP4
    per XTU_MXFP4_PREFILL (default MXFP4_PREFILL_DEFAULT: activation triples
    where the 32x32x64 kernel takes the shape, exact pairs with "pair"),
    else the bf16-operand kernels (the e2m1 x e8m0 products are exact in
    bf16 either way)."""
    fmt = int(fmt)
    if fmt == FMT_FP8:
        return True
    if fmt != FMT_MXFP4:
        return False
    mode = os.environ.get(MXFP4_PREFILL_ENV, MXFP4_PREFILL_DEFAULT)
    return mode == "pair" or (mode in _TRI_MODES and _mx_fits(H, I))


def mx_pair_kernel(fmt: int, H: int, I: int) -> bool:
    """Whether the GEMMs of this layer run on the MXFP4 32x32x64 kernel
    (interleaved activation pairs or triples, step-major scales): MXFP4 on
    the pair path where the shape fits it (I % 256, H % 512); otherwise the
    16x16x128 exact-pair kernel."""
    return int(fmt) == FMT_MXFP4 and pair_gemm(fmt, H, I) and _mx_fits(H, I)


def mx_tri(fmt: int, H: int, I: int) -> bool:
    """Whether the MXFP4 32x32x64 kernel takes activation triples (fp6, fp6,
    fp4 pieces on the double-rate MFMA; XTU_MXFP4_PREFILL "auto", "tri" or
    "duo") rather than exact e4m3 pairs ("pair")."""
    mode = os.environ.get(MXFP4_PREFILL_ENV, MXFP4_PREFILL_DEFAULT)
    return mode in _TRI_MODES and mx_pair_kernel(fmt, H, I)


def mx_act_mode(fmt: int, H: int, I: int) -> str:
    """The activation format of the MXFP4 32x32x64 kernel for this layer:
    "tri" (three pieces), "duo" (two) or "pair" (exact e4m3 pairs); its
    GEMM entry points are xtu_mx_<mode>_gate_up / _down and its quantiser
    xtu_tri_quant_il (tri, duo) or xtu_pair_quant_il (pair)."""
    if not mx_tri(fmt, H, I):
        return "pair"
    mode = os.environ.get(MXFP4_PREFILL_ENV, MXFP4_PREFILL_DEFAULT)
    return "duo" if mode == "duo" else "tri"


def gemm_tile_m(fmt: int, int8: bool = False, H: int = 0, I: int = 0, W=None,
                fp8_scales_ok=None) -> int:
    """Rows per M tile of the grouped GEMM that runs for this format and
    layer shape (and weights W, when given): INT8 ALIGN 128, the exact-pair
    kernels (FP8, MXFP4) theirs, else the bf16-operand kernels' (the
    segmentation's tiles must match)."""
    if int8:
        return 128
    if fp8_pair32_use(W, fp8_scales_ok):
        return int(_lib.call("xtu_f8_pair_tile_m"))
    if pair_gemm(fmt, H, I):
        if mx_pair_kernel(fmt, H, I):
            return int(_lib.call("xtu_mx_pair_tile_m"))
        return int(_lib.call("xtu_gemm8_tile_m"))
    return int(_lib.call("xtu_gemm_tile_m", int(fmt)))


FUSED_DOWN_ENV = "XTU_DECODE_FUSED_DOWN"


FUSED_DOWN_MAX_EXPERTS = 24
NVFP4_NARROW_FUSED_MAX = 12   # NVFP4 at I < 1024: the fused down only at T = 1 scale


def decode_fused_down_ok(fmt: int, T: int, A: int, H: int, I: int, max_active: int,
                         trash: int, shared_rows: int = 0) -> bool:
    """Whether the down projection with the weighted combine fused can run
    this batch (its act rows, plus shared_rows staged separately, fit the
    kernel's LDS stage)."""
    return bool(_lib.call("xtu_decode_down_combine_ok", int(fmt), int(T), int(A), int(H), int(I),
                          int(trash), int(max_active), int(shared_rows)))


def decode_fused_down_use(fmt: int, T: int, A: int, H: int, I: int, max_active: int,
                          trash: int, shared_rows: int = 0, one_launch: bool = False) -> bool:
    """Whether the decode path takes the fused down + combine.  Each of its
    waves walks every active expert, so it pays where few experts meet wide
    panels; measured (MI355X): faster for DeepSeek-V3 MXFP4 at T = 1, 2 (9 / 17
    experts) and Qwen3-Next MXFP4 at T = 1 (11), slower with 40 experts.
    NVFP4 at I = 512 takes it only inside the one-launch layer (one_launch:
    the whole layer runs in xtu_decode_layer) at T = 1 scale (at most 12
    experts): Qwen3-Next NVFP4 T = 1 25.3 against 26.0 us (two launches with
    the separate down and combine); as a launch of its own it was slower.
    XTU_DECODE_FUSED_DOWN=1 takes it whenever it fits, =0 never."""
    mode = os.environ.get(FUSED_DOWN_ENV, "auto")
    if mode == "0":
        return False
    if mode != "1":
        if max_active > FUSED_DOWN_MAX_EXPERTS:
            return False
        if int(fmt) == FMT_NVFP4 and I < 1024 and (not one_launch
                                                   or max_active > NVFP4_NARROW_FUSED_MAX):
            return False
    return decode_fused_down_ok(fmt, T, A, H, I, max_active, trash, shared_rows)


SHARED_SPLIT_ENV = "XTU_DECODE_SHARED_SPLIT"
# "0": the separate decode down writes y per sorted position and the combine
# reads it through inv; otherwise y is written in flat pair order
# (xtu_decode_down_by_pair) for the routers' top-k below, with up to two
# shared experts, and the combine issues all its loads at once.
DOWN_BY_PAIR_ENV = "XTU_DECODE_DOWN_BY_PAIR"
COMBINE_BY_PAIR_K = (1, 2, 4, 6, 8, 10)


def _route_shared_ok(fmt, mode, T, E, K, router, H, I, NS) -> bool:
    """Whether the routing launch can also run the shared experts' gate/up
    (tiny batch, one wave per token, fp32 logits / bias rows 16-byte
    aligned); XTU_DECODE_SHARED_SPLIT=0 keeps them with the routed ones."""
    if os.environ.get(SHARED_SPLIT_ENV, "1") == "0":
        return False
    n_group = 1
    if router is not None:
        lg, bias = router.get("logits"), router.get("bias")
        for t in (lg, bias):
            if t is not None and not (t.is_cuda and t.dtype == torch.float32
                                      and t.is_contiguous() and t.data_ptr() % 16 == 0):
                return False
        if lg is None or tuple(lg.shape) != (T, E):
            return False
        if mode == 0 and not router.get("renormalize", True):
            return False
        n_group = int(router.get("n_group", 1))
    return bool(_lib.call("xtu_decode_route_shared_ok", int(fmt), int(mode), int(T), int(E),
                          int(K), n_group, int(NS), int(H), int(I)))


FUSED_ROUTE_ENV = "XTU_DECODE_FUSED_ROUTE"
# gate/up weight bytes (the batch's tile bound x one expert's w13 + scales)
# up to which the one-launch routing + gate/up pays: there the layer is
# latency, and the routing each workgroup does beside its first weight
# stream costs less than the routing launch and its boundary.  Measured on
# MI355X: Qwen3-Next MXFP4 T = 1 (12 MB) 27.2 -> 24.7 us per layer, T = 4
# (48 MB) 33.1 vs 33.4; NVFP4 T = 1 29.1 -> 27.2, T = 4 40.6 -> 37.4;
# DeepSeek-V3 MXFP4 T = 1 (140 MB) 49.2 vs 49.1, T = 2 (265 MB) 75.5 -> 79.8,
# T = 4 (515 MB) 130.3 -> 131.6.
FUSED_ROUTE_MAX_BYTES = 64 << 20


def _w13_bytes(W) -> int:
    """One expert's gate/up weight and scale bytes in W's planes."""
    return sum(int(t[0].numel()) * t.element_size() for t in (W.w13, W.s13) if t is not None)


def _route_gate_up_ok(fmt, mode, T, E, K, router, H, I, NS, gu_bytes=None) -> bool:
    """Whether routing, segmentation and the gate/up share one launch
    (xtu_decode_route_gate_up: the tiny router's envelope and the gate/up
    fast path; fp32 logits / bias rows 16-byte aligned), and, for gu_bytes
    of gate/up weights to stream, pay there (FUSED_ROUTE_MAX_BYTES).
    XTU_DECODE_FUSED_ROUTE=0 keeps separate launches, =1 fuses whenever the
    shape fits."""
    mode_env = os.environ.get(FUSED_ROUTE_ENV, "auto")
    if mode_env == "0":
        return False
    if mode_env != "1" and gu_bytes is not None and gu_bytes > FUSED_ROUTE_MAX_BYTES:
        return False
    n_group = 1
    if router is not None:
        lg, bias = router.get("logits"), router.get("bias")
        for t in (lg, bias):
            if t is not None and not (t.is_cuda and t.dtype == torch.float32
                                      and t.is_contiguous() and t.data_ptr() % 16 == 0):
                return False
        if lg is None or tuple(lg.shape) != (T, E):
            return False
        if mode == 0 and not router.get("renormalize", True):
            return False
        n_group = int(router.get("n_group", 1))
    return bool(_lib.call("xtu_decode_route_gate_up_ok", int(fmt), int(mode), int(T), int(E),
                          int(K), n_group, int(NS), int(H), int(I)))


ONE_LAUNCH_ENV = "XTU_DECODE_ONE_LAUNCH"


def _layer_ok(fmt, mode, T, E, K, router, H, I, NS) -> bool:
    """Whether a decode layer that takes the one-launch routing + gate/up and
    the fused down + combine runs whole in one launch (xtu_decode_layer:
    the down after a barrier across the launch's workgroups, its first
    experts' weights loaded during the wait).  Measured on MI355X:
    Qwen3-Next MXFP4 T = 1 24.4 -> 22.4 us per layer (20.2 us with the
    sorted-list wave router and the barrier generation read at launch
    start; the same changes give the two-launch path's NVFP4 T = 1 26.2
    us).  Where the separate
    launches would not take the fused down it is not taken either (forced:
    Qwen3-Next MXFP4 T = 4 37.5 -> 41.1 us against 33.5 without the fused
    down; NVFP4 T = 1 27.2 against 27.4), and DeepSeek-V3 MXFP4 T = 1 (with
    the routing forced into the gate/up launch) ran 51.9 us against 48.6.
    XTU_DECODE_ONE_LAUNCH=0 keeps the down in its own launch."""
    if os.environ.get(ONE_LAUNCH_ENV, "1") == "0":
        return False
    n_group = int(router.get("n_group", 1)) if router is not None else 1
    return bool(_lib.call("xtu_decode_layer_ok", int(fmt), int(mode), int(T), int(E), int(K),
                          n_group, int(NS), int(H), int(I)))


# Grid-barrier words of the one-launch decode layer per (device, stream):
# zeroed once, on the stream the layer runs on; every launch leaves its
# counters zero (the last 64-word line flags a wait that ran out).  Kept for
# the process's life, as the scratch buffers are.
_BAR_CACHE: dict = {}


def _barrier_words(device, stream=None):
    st = _stream(stream)
    key = (str(device), st)
    t = _BAR_CACHE.get(key)
    if t is None:
        n = int(_lib.call("xtu_decode_layer_barrier_words"))
        if int(torch.cuda.current_stream(device).cuda_stream) == st:
            t = torch.zeros(n, dtype=torch.int32, device=device)
        else:
            with torch.cuda.stream(torch.cuda.ExternalStream(st, device=device)):
                t = torch.zeros(n, dtype=torch.int32, device=device)
        _BAR_CACHE[key] = t
    return t


def barrier_timeouts() -> int:
    """Grid-barrier waits of the one-launch decode layer that ran out (the
    launch could not be resident): 0 in every healthy process."""
    return sum(int(t[-64].item()) for t in _BAR_CACHE.values())


def _mxpair_bufs(tag, M, K, dev, stream=None):
    """Interleaved activation pairs [M][2K] and their e8m0 bytes [M][K/32]."""
    return (_buf(tag + "_hilo", (max(M, 1), 2 * K), torch.uint8, dev, stream),
            _buf(tag + "_shi", (max(M, 1), K // 32), torch.uint8, dev, stream))


def _fp8pair_bufs(tag, M, K, dev, stream=None):
    return (_buf(tag + "_hi", (max(M, 1), K), torch.uint8, dev, stream),
            _buf(tag + "_lo", (max(M, 1), K), torch.uint8, dev, stream),
            _buf(tag + "_shi", (max(M, 1), K // 32), torch.uint8, dev, stream),
            _buf(tag + "_slo", (max(M, 1), K // 32), torch.uint8, dev, stream))


def moe_forward(x, topk_ids, topk_weights, W: ExpertWeights, *, swiglu_limit=0.0, swiglu_alpha=1.0,
                swiglu_beta=0.0, out=None, out_dtype=torch.bfloat16, path="auto", int8=False,
                drop_zero=True, id_map=None, slot_map=None, stream=None, return_seg=False,
                router=None, fp8_scales_ok=None):
    """Routed (+shared) experts of one layer; returns out [T, H].

    path: "auto" (decode kernels for T <= 16, grouped GEMMs otherwise),
    "decode" or "gemm".  int8: INT8-activation x FP4-code ALIGN path (MXFP4):
    True forces it, "auto" applies the reference's token-count gate
    (int8_align_on).
    id_map: int32 [E] applied to topk_ids before bucketing; slot_map: int32
    [E+NS] bucket -> weight slot.  router: dict(logits=, scoring=, bias=,
    n_group=, topk_group=, routed_scaling_factor=, renormalize=) routes from
    logits first, writing topk_ids / topk_weights (int32 / fp32 buffers).
    fp8_scales_ok: for FP8 slot planes, whether their block scales are
    bounded (fp8_block_scales_bounded).
    """
    if x.dtype != torch.bfloat16 or not x.is_contiguous():
        raise ValueError("x must be contiguous bf16 [T, H]")
    if W.fmt == FMT_INT4:
        raise ValueError("INT4 (WNA16) experts run on the host engine (cpu_experts.CpuExperts, "
                         "engine.MOE_WNA16), as the reference's MOE_WNA16 does")
    T, K = topk_ids.shape
    H, I, E, NS = W.H, W.I, W.E, W.n_shared
    if x.shape != (T, H):
        raise ValueError(f"x shape {tuple(x.shape)} != ({T}, {H})")
    dev = x.device
    if not x.is_cuda:
        raise ValueError("x must be a CUDA tensor")
    _same_device(dev, topk_ids=topk_ids, topk_weights=topk_weights, w13=W.w13, w2=W.w2,
                 s13=W.s13, s2=W.s2, gs13=W.gs13, gs2=W.gs2, id_map=id_map, slot_map=slot_map,
                 out=out)
    if router is not None:
        _same_device(dev, logits=router.get("logits"), bias=router.get("bias"))
    if router is not None and not (topk_ids.dtype == torch.int32 and topk_ids.is_contiguous()
                                   and topk_weights.dtype == torch.float32
                                   and topk_weights.is_contiguous()):
        raise ValueError("with router=, topk_ids / topk_weights are int32 / fp32 output buffers")
    ids = topk_ids if (topk_ids.dtype == torch.int32 and topk_ids.is_contiguous()) else topk_ids.to(torch.int32).contiguous()
    wts = topk_weights if (topk_weights.dtype == torch.float32 and topk_weights.is_contiguous()) else topk_weights.float().contiguous()
    st = _stream(stream)
    fmt = W.fmt
    if int8 == "auto":
        int8 = int8_align_on(T, True)
    int8 = bool(int8)
    if path == "auto":
        path = "decode" if (T <= DECODE_MAX_TOKENS and not int8) else "gemm"
    if path == "decode" and T > DECODE_MAX_TOKENS:
        raise ValueError(f"decode path handles at most {DECODE_MAX_TOKENS} tokens")
    # decode: the gate/up and down kernels take the segmentation's 16-row
    # tiles as work slots (every row of a bucket, however many)
    bm = DECODE_TILE if path == "decode" else gemm_tile_m(fmt, int8, W.H, W.I, W, fp8_scales_ok)
    seg = segmentation(T, K, E, NS, bm, dev, st)
    odt = out_dtype if out is None else out.dtype
    max_active = min(E, T * K) + NS
    # decode with shared experts: their gate/up runs in the routing launch
    # (they need no routing), the routed gate/up leaves them out and the fused
    # down takes their rows from act_sh
    rmode = 2 if router is None else (1 if router.get("scoring", "softmax") == "sigmoid" else 0)
    # decode of a tiny batch: routing, segmentation and the gate/up in one
    # launch (every gate/up workgroup routes the batch for itself)
    fused = (path == "decode" and T > 0 and seg.small
             and _route_gate_up_ok(fmt, rmode, T, E, K, router, H, I, NS,
                                   gu_bytes=min(seg.max_tiles, TINY_MAX_PAIRS) * _w13_bytes(W)))
    layer_ok = fused and _layer_ok(fmt, rmode, T, E, K, router, H, I, NS)
    split = (path == "decode" and T > 0 and NS > 0 and seg.small
             and odt in (torch.bfloat16, torch.float32)
             and decode_fused_down_use(fmt, T, seg.A, H, I, max_active, E + NS, NS * T,
                                       one_launch=layer_ok)
             and (fused or _route_shared_ok(fmt, rmode, T, E, K, router, H, I, NS)))
    lim, al, be = float(swiglu_limit or 0.0), float(swiglu_alpha), float(swiglu_beta)
    if split:
        act_sh = _buf("act_sh", (NS * T, I), torch.bfloat16, dev, st)
    # ... and the down with the weighted combine in the same launch, after a
    # barrier across its workgroups
    one = layer_ok and (split or (odt in (torch.bfloat16, torch.float32)
                                  and decode_fused_down_use(fmt, T, seg.A, H, I, max_active,
                                                            E + NS, one_launch=True)))
    if one:
        r = router or {}
        act = _buf("act", (max(seg.A, 1), I), torch.bfloat16, dev, st)
        if out is None:
            out = torch.empty((T, H), dtype=odt, device=dev)
        _lib.call("xtu_decode_layer", rmode, _p(r.get("logits")), _p(r.get("bias")),
                  _p(ids), _p(wts), T, E, K, int(r.get("n_group", 1)),
                  int(r.get("topk_group", 1)), float(r.get("routed_scaling_factor", 1.0)),
                  int(r.get("renormalize", True)), _p(id_map), NS, int(drop_zero), seg.bm,
                  _p(seg.sorted_pair), _p(seg.sorted_tok), _p(seg.sorted_wts), _p(seg.inv),
                  _p(seg.seg_start), _p(seg.active), _p(seg.n_active), _p(seg.tile_expert),
                  _p(seg.tile_row0), _p(seg.n_tiles), _p(seg.expert_tile_start), fmt, _p(x), H,
                  I, _p(W.w13), _p(W.s13), _p(W.gs13), 0, 0, _p(slot_map),
                  min(seg.max_tiles, TINY_MAX_PAIRS), _p(act), _p(act_sh) if split else 0,
                  lim, al, be, _p(W.w2), _p(W.s2), _p(W.gs2), 0, 0, _p(out),
                  int(out.dtype == torch.bfloat16), _p(_barrier_words(dev, st)), st)
        return (out, seg) if return_seg else out
    if fused:
        r = router or {}
        act = _buf("act", (max(seg.A, 1), I), torch.bfloat16, dev, st)
        _lib.call("xtu_decode_route_gate_up", rmode, _p(r.get("logits")), _p(r.get("bias")),
                  _p(ids), _p(wts), T, E, K, int(r.get("n_group", 1)),
                  int(r.get("topk_group", 1)), float(r.get("routed_scaling_factor", 1.0)),
                  int(r.get("renormalize", True)), _p(id_map), NS, int(drop_zero), seg.bm,
                  _p(seg.sorted_pair), _p(seg.sorted_tok), _p(seg.sorted_wts), _p(seg.inv),
                  _p(seg.seg_start), _p(seg.active), _p(seg.n_active), _p(seg.tile_expert),
                  _p(seg.tile_row0), _p(seg.n_tiles), _p(seg.expert_tile_start), fmt, _p(x), H,
                  I, _p(W.w13), _p(W.s13), _p(W.gs13), 0, 0, _p(slot_map),
                  min(seg.max_tiles, TINY_MAX_PAIRS), _p(act), _p(act_sh) if split else 0,
                  lim, al, be, st)
    elif split:
        r = router or {}
        _lib.call("xtu_decode_route_shared", rmode, _p(r.get("logits")), _p(r.get("bias")),
                  _p(ids), _p(wts), T, E, K, int(r.get("n_group", 1)),
                  int(r.get("topk_group", 1)), float(r.get("routed_scaling_factor", 1.0)),
                  int(r.get("renormalize", True)), _p(id_map), NS, int(drop_zero), seg.bm,
                  _p(seg.sorted_pair), _p(seg.sorted_tok), _p(seg.sorted_wts), _p(seg.inv),
                  _p(seg.seg_start), _p(seg.active), _p(seg.n_active), _p(seg.tile_expert),
                  _p(seg.tile_row0), _p(seg.n_tiles), _p(seg.expert_tile_start), fmt, _p(x), H,
                  I, _p(W.w13), _p(W.s13), _p(W.gs13), 0, 0, _p(slot_map), _p(act_sh), lim, al,
                  be, st)
    elif router is not None:
        mode = rmode
        # the fused route + segmentation: tiny batches, or softmax over few
        # experts (one thread per token) for any batch the small path holds
        if seg.small and T > 0 and (T <= SMALL_ROUTE_MAX_TOKENS
                                    or (mode == 0 and E <= LANE_ROUTE_MAX_E
                                        and K <= LANE_ROUTE_MAX_K)):
            seg.run_small(mode, ids, wts, logits=router["logits"], bias=router.get("bias"),
                          n_group=router.get("n_group", 1), topk_group=router.get("topk_group", 1),
                          routed_scaling=router.get("routed_scaling_factor", 1.0),
                          renormalize=router.get("renormalize", True), id_map=id_map,
                          drop_zero=drop_zero, stream=st)
        else:
            route(router["logits"], top_k=K, scoring=router.get("scoring", "softmax"),
                  renormalize=router.get("renormalize", True), bias=router.get("bias"),
                  n_group=router.get("n_group", 1), topk_group=router.get("topk_group", 1),
                  routed_scaling_factor=router.get("routed_scaling_factor", 1.0), ids_out=ids,
                  wts_out=wts, stream=st)
            if seg.small:   # the whole segmentation in one launch
                seg.run_small(2, ids, wts, id_map=id_map, drop_zero=drop_zero, stream=st)
            else:
                seg.run(ids, wts, id_map, drop_zero, st)
    elif seg.small and T > 0:
        seg.run_small(2, ids, wts, id_map=id_map, drop_zero=drop_zero, stream=st)
    else:
        seg.run(ids, wts, id_map, drop_zero, st)
    A = seg.A
    if out is None:
        out = torch.empty((T, H), dtype=odt, device=dev)
    if T == 0:
        return (out, seg) if return_seg else out
    if path == "decode":
        act = _buf("act", (max(A, 1), I), torch.bfloat16, dev, st)
        max_dt = decode_max_tiles(A, max_active)
        if fused:
            pass   # the routing launch ran the gate/up too
        elif split:
            _lib.call("xtu_decode_gate_up_routed", fmt, _p(x), T, H, I, _p(W.w13), _p(W.s13),
                      _p(W.gs13), 0, 0, _p(slot_map), _p(seg.sorted_tok), _p(seg.seg_start),
                      _p(seg.tile_expert), _p(seg.tile_row0), _p(seg.n_tiles), max_dt, NS,
                      _p(act), lim, al, be, st)
        else:
            _lib.call("xtu_decode_gate_up", fmt, _p(x), T, H, I, _p(W.w13), _p(W.s13),
                      _p(W.gs13), 0, 0, _p(slot_map), _p(seg.sorted_tok), _p(seg.seg_start),
                      _p(seg.tile_expert), _p(seg.tile_row0), _p(seg.n_tiles), max_dt, _p(act),
                      lim, al, be, st)
        if split or (odt in (torch.bfloat16, torch.float32)
                     and decode_fused_down_use(fmt, T, A, H, I, max_active, E + NS)):
            # down projection and weighted combine in one pass, out written whole
            _lib.call("xtu_decode_down_combine", fmt, _p(act),
                      _p(act_sh) if split else 0, NS, T, A, H, I, _p(W.w2), _p(W.s2),
                      _p(W.gs2), 0, 0, _p(slot_map), _p(seg.sorted_tok), _p(seg.sorted_wts),
                      _p(seg.seg_start), E + NS, _p(seg.active), _p(seg.n_active), max_active,
                      _p(out), int(out.dtype == torch.bfloat16), st)
            return (out, seg) if return_seg else out
        y = _buf("y", (max(A, 1), H), torch.float32, dev, st)
        if (os.environ.get(DOWN_BY_PAIR_ENV, "1") != "0" and K in COMBINE_BY_PAIR_K
                and NS <= 2 and out.dtype in (torch.bfloat16, torch.float32)):
            # y rows in flat pair order: the combine's loads need no inv first
            _lib.call("xtu_decode_down_by_pair", fmt, _p(act), T, H, I, _p(W.w2), _p(W.s2),
                      _p(W.gs2), 0, 0, _p(slot_map), _p(seg.seg_start), _p(seg.tile_expert),
                      _p(seg.tile_row0), _p(seg.n_tiles), max_dt, _p(seg.sorted_pair), _p(y),
                      st)
            _lib.call("xtu_combine_by_pair", _p(y), _p(seg.inv), _p(wts),
                      _p(seg.seg_start) + 4 * (seg.E + seg.NS), T, K, NS, H, _p(out),
                      int(out.dtype == torch.bfloat16), st)
            return (out, seg) if return_seg else out
        _lib.call("xtu_decode_down", fmt, _p(act), T, H, I, _p(W.w2), _p(W.s2), _p(W.gs2), 0, 0,
                  _p(slot_map), _p(seg.seg_start), _p(seg.tile_expert), _p(seg.tile_row0),
                  _p(seg.n_tiles), max_dt, _p(y), st)
    else:
        y = _buf("y", (max(A, 1), H), torch.float32, dev, st)
        expert_pass(x, seg, W, 0, E + NS, y, slot_map=slot_map, int8=int8,
                    swiglu_limit=swiglu_limit, swiglu_alpha=swiglu_alpha,
                    swiglu_beta=swiglu_beta, stream=st, fp8_scales_ok=fp8_scales_ok)
    combine(seg, y, wts, out, stream=st)
    return (out, seg) if return_seg else out


ACT_QUANT_ENV = "XTU_ACT_QUANT_FUSED"
_MX_MODE_IDS = {"pair": 0, "tri": 1, "duo": 2}   # xtu_mx_gate_up_q's mode


def act_quant_fused() -> bool:
    """Whether the MXFP4 / FP8 32x32x64 gate/up epilogues write the down
    pass's activation pairs / triples themselves (the same bytes as the
    separate quantiser over the bf16 rows, without the rows' round trip);
    XTU_ACT_QUANT_FUSED=0 writes bf16 rows and quantises them apart."""
    return os.environ.get(ACT_QUANT_ENV, "1") != "0"


def expert_pass(x, seg, W: ExpertWeights, b0: int, b1: int, y, *, slot_map=None, int8=False,
                swiglu_limit=0.0, swiglu_alpha=1.0, swiglu_beta=0.0, stream=None,
                fp8_scales_ok=None):
    """Grouped gate/up (+ SwiGLU-clamp) and down GEMMs for the sorted pairs of
    buckets [b0, b1), weights of bucket b at slot slot_map[b] of W (identity
    without a map); writes their fp32 rows of y [A, H].  The segmentation's
    tile height must be gemm_tile_m(..., W, fp8_scales_ok)'s."""
    T, H = x.shape
    I = W.I
    A = seg.A
    if A == 0 or b1 <= b0:
        return
    dev = x.device
    st = _stream(stream)
    lim, al, be = float(swiglu_limit or 0.0), float(swiglu_alpha), float(swiglu_beta)
    act = _buf("act", (max(A, 1), I), torch.bfloat16, dev, st)
    lo, hi = seg.tile_range_ptrs(b0, b1)
    if int8:
        w13_8, emin13, w2_8, emin2 = W.int8_planes()
        a8x = _buf("a8x", (T, H), torch.int8, dev, st)
        crx = _buf("crx", (T,), torch.int32, dev, st)
        a8a = _buf("a8a", (max(A, 1), I), torch.int8, dev, st)
        cra = _buf("cra", (max(A, 1),), torch.int32, dev, st)
        _lib.call("xtu_i8_quant_rows", _p(x), T, H, _p(a8x), _p(crx), st)
        fb = W.int8_fallback_cols()
        emm13, emm2 = W.int8_emin_min()
        _lib.call("xtu_i8_gemm_gate_up", _p(a8x), _p(crx), _p(seg.sorted_tok), H, I, _p(w13_8),
                  _p(emin13), _p(slot_map), _p(seg.seg_start), _p(seg.tile_expert),
                  _p(seg.tile_row0), lo, hi, seg.max_tiles, _p(act), 0, lim, al, be, st)
        if fb is not None:   # marked weight rows: their columns in fp32
            _lib.call("xtu_i8_fallback", 1, _p(x), _p(seg.sorted_tok), H, I, _p(W.w13),
                      _p(W.s13), _p(slot_map), _p(seg.seg_start), _p(seg.tile_expert),
                      _p(seg.tile_row0), lo, hi, seg.max_tiles, seg.bm, _p(fb[0]), _p(fb[1]),
                      _p(act), lim, al, be, st)
        # rows past the offset guard: the whole row in fp32
        _lib.call("xtu_i8_row_fallback", 1, _p(x), _p(seg.sorted_tok), _p(crx), _p(emm13), H, I,
                  _p(W.w13), _p(W.s13), _p(slot_map), _p(seg.seg_start), _p(seg.tile_expert),
                  _p(seg.tile_row0), lo, hi, seg.max_tiles, seg.bm, _p(act), lim, al, be, st)
        _lib.call("xtu_i8_quant_rows", _p(act), A, I, _p(a8a), _p(cra), st)
        _lib.call("xtu_i8_gemm_down", _p(a8a), _p(cra), H, I, _p(w2_8), _p(emin2), _p(slot_map),
                  _p(seg.seg_start), _p(seg.tile_expert), _p(seg.tile_row0), lo, hi,
                  seg.max_tiles, _p(y), 0, st)
        if fb is not None:
            _lib.call("xtu_i8_fallback", 0, _p(act), 0, H, I, _p(W.w2), _p(W.s2), _p(slot_map),
                      _p(seg.seg_start), _p(seg.tile_expert), _p(seg.tile_row0), lo, hi,
                      seg.max_tiles, seg.bm, _p(fb[2]), _p(fb[3]), _p(y), 0.0, 1.0, 0.0, st)
        _lib.call("xtu_i8_row_fallback", 0, _p(act), 0, _p(cra), _p(emm2), H, I, _p(W.w2),
                  _p(W.s2), _p(slot_map), _p(seg.seg_start), _p(seg.tile_expert),
                  _p(seg.tile_row0), lo, hi, seg.max_tiles, seg.bm, _p(y), 0.0, 1.0, 0.0, st)
        return
    fmt = W.fmt
    if fp8_pair32_use(W, fp8_scales_ok):
        # exact pairs, interleaved, on the FP8 32x32x64 kernel (block scales
        # applied by accumulator rescaling)
        xq = _mxpair_bufs("xm", T, H, dev, st)
        aq = _mxpair_bufs("am", A, I, dev, st)
        _lib.call("xtu_pair_quant_il", _p(x), T, H, *[_p(t) for t in xq], st)
        if act_quant_fused():   # the gate/up epilogue writes the down pass's pairs
            _lib.call("xtu_f8_pair_gate_up_q", *[_p(t) for t in xq], _p(seg.sorted_tok), H, I,
                      _p(W.w13), _p(W.s13), 0, 0, _p(slot_map), _p(seg.seg_start),
                      _p(seg.tile_expert), _p(seg.tile_row0), _p(seg.expert_tile_start), lo,
                      hi, seg.max_tiles, *[_p(t) for t in aq], lim, al, be, st)
        else:
            _lib.call("xtu_f8_pair_gate_up", *[_p(t) for t in xq], _p(seg.sorted_tok), H, I,
                      _p(W.w13), _p(W.s13), 0, 0, _p(slot_map), _p(seg.seg_start),
                      _p(seg.tile_expert), _p(seg.tile_row0), _p(seg.expert_tile_start), lo,
                      hi, seg.max_tiles, _p(act), lim, al, be, st)
            _lib.call("xtu_pair_quant_il", _p(act), A, I, *[_p(t) for t in aq], st)
        _lib.call("xtu_f8_pair_down", *[_p(t) for t in aq], H, I, _p(W.w2), _p(W.s2), 0, 0,
                  _p(slot_map), _p(seg.seg_start), _p(seg.tile_expert), _p(seg.tile_row0),
                  _p(seg.expert_tile_start), lo, hi, seg.max_tiles, _p(y), st)
        return
    if mx_pair_kernel(fmt, H, I):
        # activation triples (double-rate fp6/fp4 MFMA) or exact pairs,
        # interleaved, on the MXFP4 32x32x64 kernel
        kind = mx_act_mode(fmt, H, I)
        qk = "pair" if kind == "pair" else "tri"
        s13p, s2p = W.mx_pair_scales(st)
        xq = _mxpair_bufs("xm", T, H, dev, st)
        aq = _mxpair_bufs("am", A, I, dev, st)
        _lib.call(f"xtu_{qk}_quant_il", _p(x), T, H, *[_p(t) for t in xq], st)
        if act_quant_fused():   # the gate/up epilogue writes the down pass's pieces
            _lib.call("xtu_mx_gate_up_q", _MX_MODE_IDS[kind], *[_p(t) for t in xq],
                      _p(seg.sorted_tok), H, I, _p(W.w13), _p(s13p), 0, 0, _p(slot_map),
                      _p(seg.seg_start), _p(seg.tile_expert), _p(seg.tile_row0),
                      _p(seg.expert_tile_start), lo, hi, seg.max_tiles, *[_p(t) for t in aq],
                      lim, al, be, st)
        else:
            _lib.call(f"xtu_mx_{kind}_gate_up", *[_p(t) for t in xq], _p(seg.sorted_tok), H, I,
                      _p(W.w13), _p(s13p), 0, 0, _p(slot_map), _p(seg.seg_start),
                      _p(seg.tile_expert), _p(seg.tile_row0), _p(seg.expert_tile_start), lo,
                      hi, seg.max_tiles, _p(act), lim, al, be, st)
            _lib.call(f"xtu_{qk}_quant_il", _p(act), A, I, *[_p(t) for t in aq], st)
        _lib.call(f"xtu_mx_{kind}_down", *[_p(t) for t in aq], H, I, _p(W.w2), _p(s2p), 0, 0,
                  _p(slot_map), _p(seg.seg_start), _p(seg.tile_expert), _p(seg.tile_row0),
                  _p(seg.expert_tile_start), lo, hi, seg.max_tiles, _p(y), st)
        return
    if pair_gemm(fmt, H, I):
        # exact pairs: activations split into e4m3 (hi, lo) with e8m0 scales;
        # FP8 weights on the fp8 MFMA with the fp32 block scale folded per
        # 128 k, MXFP4 weights as fp4 B operands with their e8m0 B scale
        xq = _fp8pair_bufs("x8", T, H, dev, st)
        aq = _fp8pair_bufs("a8", A, I, dev, st)
        _lib.call("xtu_fp8pair_quant", _p(x), T, H, *[_p(t) for t in xq], st)
        _lib.call("xtu_gemm_pair_gate_up", fmt, *[_p(t) for t in xq], _p(seg.sorted_tok), H, I,
                  _p(W.w13), _p(W.s13), 0, 0, _p(slot_map), _p(seg.seg_start),
                  _p(seg.tile_expert), _p(seg.tile_row0), _p(seg.expert_tile_start), lo, hi,
                  seg.max_tiles, _p(act), lim, al, be, st)
        _lib.call("xtu_fp8pair_quant", _p(act), A, I, *[_p(t) for t in aq], st)
        _lib.call("xtu_gemm_pair_down", fmt, *[_p(t) for t in aq], H, I, _p(W.w2), _p(W.s2), 0,
                  0, _p(slot_map), _p(seg.seg_start), _p(seg.tile_expert), _p(seg.tile_row0),
                  _p(seg.expert_tile_start), lo, hi, seg.max_tiles, _p(y), st)
        return
    _lib.call("xtu_gemm_gate_up", fmt, _p(x), _p(seg.sorted_tok), H, I, _p(W.w13), _p(W.s13),
              _p(W.gs13), 0, 0, _p(slot_map), _p(seg.seg_start), _p(seg.tile_expert),
              _p(seg.tile_row0), lo, hi, seg.max_tiles, _p(act), lim, al, be, st)
    _lib.call("xtu_gemm_down", fmt, _p(act), H, I, _p(W.w2), _p(W.s2), _p(W.gs2), 0, 0,
              _p(slot_map), _p(seg.seg_start), _p(seg.tile_expert), _p(seg.tile_row0), lo, hi,
              seg.max_tiles, _p(y), st)


def combine(seg, y, topk_weights, out, *, stream=None):
    """out[t] = sum_k w[t,k] * y[pos(t,k)] (+ shared rows), pairs in the trash
    bucket or of weight 0 skipped; bf16 or fp32 out."""
    T, K = seg.T, seg.K
    _lib.call("xtu_combine", _p(y), _p(seg.inv), _p(topk_weights),
              _p(seg.seg_start) + 4 * (seg.E + seg.NS), T, K, seg.NS, out.shape[1], _p(out),
              int(out.dtype == torch.bfloat16), _stream(stream))
