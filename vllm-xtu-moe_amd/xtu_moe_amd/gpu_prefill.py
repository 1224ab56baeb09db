"""Layer entries with the reference's signatures, over the HIP library.

* ``gpu_moe_layer`` -- vllm_xiaotu_moe/gpu_prefill.py:2566-2780: one layer's
  routed experts from fp4 checkpoint planes (MXFP4: e8m0 scales, group 32;
  NVFP4: e4m3 scales, group 16, per-expert global scales s13_ts / s2_ts),
  on the device or on the host, or from a resident slot (``slot.bufs``,
  topk_ids then index the slot's rows); out [T, H] (bf16 by default).
* ``gpu_moe_layer_fp8`` -- gpu_prefill_fp8.py:458: FP8 block-scaled
  experts from K-major planes w13t [S, H, 2I] / s13t [S, H/128, 2I/128] and
  w2t [S, I, H] / s2t [S, I/128, H/128]; out fp32.  Scale planes may be fp32
  or -- as the reference's pool and ring hold them -- uint8 planes of fp32
  bytes [S, H/128, 2I/128*4], which are viewed as fp32
  (gpu_prefill_fp8.py:489-496).
* ``gpu_moe_decode_fp8`` -- decode_moe_fp8.py:103: the same planes, no token
  limit (the reference caller uses it up to 32 tokens,
  mixed_experts.py:2133-2141): the skinny-M decode kernels up to 16 tokens,
  the grouped GEMMs above; out fp32.
* ``moe_layer`` -- moe4_smallm.py:151-341: small-M fp4 experts from K-major
  planes [S, H/2, 2I], [S, H/32, 2I], [S, I/2, H], [S, I/32, H]; returns
  None (caller falls back) outside T <= 8, top-k <= 8, group 32, e8m0.
* The ring-stage entries are re-exported from ``ring``.

Planes may also be the device layout itself (an ``ExpertWeights``' 2-D P16
planes, e.g. ``*pool.planes``): they are used in place.  A pool's or ring's
slot planes are recognised as such (mutable, with the FP8 scale bound of
the store that fills them, so nothing is checked per call and eager and
captured calls take the same kernels); other device-layout planes are
wrapped once per storage and version, like checkpoint planes.  Checkpoint planes
on the device are packed into the device layout once and cached in a small
LRU keyed by their storage; an entry holds the source tensors (so their
memory cannot be reused under the key) and their in-place version counters
(a rewritten plane is packed again) -- as the reference keys its K-major
copies on the source storage it holds (gpu_prefill.py:1078 ``_pin_key``).
Planes on the host are packed per call and not kept on the device.
"""
from __future__ import annotations

from collections import OrderedDict

import torch

from . import formats as F
from .layer import DECODE_MAX_TOKENS, ExpertWeights, moe_forward, slot_planes_of
from .ring import (gpu_moe_layer_from_engine_tiled, prealloc_tile_ring,  # noqa: F401
                   stage_tiles, staging_bytes, staging_tile_experts)

PACK_CACHE_MAX = 64
_PACKED: "OrderedDict" = OrderedDict()


def _src_key(t):
    if t is None:
        return None
    return (t.untyped_storage().data_ptr(), t.storage_offset(), tuple(t.shape),
            tuple(t.stride()), str(t.dtype), str(t.device))


def _pack(fmt, device, w13, s13, w2, s2, g13, g2, kmajor):
    if kmajor:   # [S, K(packed), N] -> [S, N, K(packed)]
        tr = lambda t: None if t is None else t.transpose(1, 2).contiguous()
        w13, s13, w2, s2 = tr(w13), tr(s13), tr(w2), tr(s2)
    mv = lambda t, f=None: None if t is None else (t.to(device).float() if f else t.to(device))
    return ExpertWeights.from_dense(fmt, mv(w13), mv(s13), mv(w2), mv(s2), mv(g13, 1),
                                    mv(g2, 1), device=device)


def _packed(fmt, device, w13, s13, w2, s2, g13=None, g2=None, kmajor=False, H=None, I=None):
    """ExpertWeights for these planes (see the module docstring)."""
    device = torch.device(device)
    if w13.dim() == 2:   # already the device layout: [S, bytes] P16 planes
        if H is None or I is None:
            raise ValueError("device-layout planes need H and I")
        W = slot_planes_of(w13, s13, w2, s2)
        if W is not None and W.fmt == int(fmt):   # pool / ring slots: used as they are
            return W
        # other device-layout planes: built once per (storage, version) below
        key = (fmt, str(device), "p16", int(H), int(I)) + tuple(
            _src_key(t) for t in (w13, s13, w2, s2, g13, g2))
        vers = tuple(None if t is None else t._version for t in (w13, s13, w2, s2, g13, g2))
        ent = _PACKED.get(key)
        if ent is not None and ent[2] == vers:
            _PACKED.move_to_end(key)
            return ent[0]
        W = ExpertWeights(fmt, H, I, w13.shape[0], 0, w13, s13, w2, s2,
                          None if g13 is None else g13.float(),
                          None if g2 is None else g2.float())
        _PACKED[key] = (W, (w13, s13, w2, s2, g13, g2), vers)
        while len(_PACKED) > PACK_CACHE_MAX:
            _PACKED.popitem(last=False)
        return W
    srcs = (w13, s13, w2, s2, g13, g2)
    if not all(t is None or (t.is_cuda and t.device == device) for t in srcs):
        return _pack(fmt, device, *srcs, kmajor)   # host planes: per call
    key = (fmt, str(device), kmajor) + tuple(_src_key(t) for t in srcs)
    vers = tuple(None if t is None else t._version for t in srcs)
    ent = _PACKED.get(key)
    if ent is not None and ent[2] == vers:
        _PACKED.move_to_end(key)
        return ent[0]
    W = _pack(fmt, device, *srcs, kmajor)
    _PACKED[key] = (W, srcs, vers)
    _PACKED.move_to_end(key)
    while len(_PACKED) > PACK_CACHE_MAX:
        _PACKED.popitem(last=False)
    return W


def _fp4_kind(s13, scale_kind):
    if scale_kind is not None:
        return str(scale_kind)
    return "e4m3" if getattr(s13, "dtype", None) == torch.float8_e4m3fn else "e8m0"


def gpu_moe_layer(x, topk_ids, topk_weights, w13, s13, w2, s2, H: int, I: int, K: int, *,
                  device, slot=None, out_dtype=None, swiglu_limit: float = 0.0,
                  group_k: int = 32, scale_kind=None, s13_ts=None, s2_ts=None, out=None):
    device = torch.device(device)
    T = x.shape[0]
    odt = out_dtype or torch.bfloat16
    if out is None:
        out = torch.empty((T, int(H)), dtype=odt, device=device)
    if T == 0 or K == 0:
        out.zero_()
        return out
    if slot is not None:   # the slot's own planes, in its format
        if not torch.cuda.is_current_stream_capturing():
            torch.cuda.current_stream(device).wait_event(slot.ready)
        W = slot.bufs
    else:
        kind = _fp4_kind(s13, scale_kind)
        fmt = F.FMT_NVFP4 if kind == "e4m3" else F.FMT_MXFP4
        if int(group_k) != (16 if fmt == F.FMT_NVFP4 else 32):
            raise ValueError(f"{kind} scales come in groups of "
                             f"{16 if fmt == F.FMT_NVFP4 else 32}")
        W = _packed(fmt, device, w13, s13, w2, s2, s13_ts, s2_ts, H=int(H), I=int(I))
    if W.H != int(H) or W.I != int(I):
        raise ValueError(f"weights are H={W.H} I={W.I}, call says H={H} I={I}")
    moe_forward(x.to(torch.bfloat16).contiguous(), topk_ids, topk_weights, W,
                swiglu_limit=swiglu_limit, out=out)
    if slot is not None and not torch.cuda.is_current_stream_capturing():
        slot.busy = torch.cuda.Event()
        slot.busy.record(torch.cuda.current_stream(device))
    return out


def _fp8_scale_plane(s, nk: int, nn: int, name: str):
    """A K-major FP8 scale plane as fp32 [S, nk, nn]: fp32 as given, or a
    uint8 plane of fp32 bytes [S, nk, nn*4] viewed as fp32 (no value
    conversion: the bytes are the scales)."""
    if s.dtype == torch.uint8:
        if s.dim() != 3 or s.shape[2] % 4:
            raise ValueError(f"{name}: uint8 scale plane must be [S, {nk}, {nn}*4] bytes, "
                             f"got {tuple(s.shape)}")
        s = s.contiguous().view(torch.float32)
    elif s.dtype != torch.float32:
        s = s.float()
    if s.dim() != 3 or tuple(s.shape[1:]) != (nk, nn):
        raise ValueError(f"{name}: expected fp32 scales [S, {nk}, {nn}], got {tuple(s.shape)}")
    return s


def _fp8_weights(w13t, s13t, w2t, s2t, H, I, device):
    u8 = lambda t: t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t
    if w13t.dim() == 2:   # device-layout planes (P16 + fp32 block scales)
        return _packed(F.FMT_FP8, device, u8(w13t), s13t, u8(w2t), s2t, H=H, I=I)
    s13 = _fp8_scale_plane(s13t, H // 128, 2 * I // 128, "s13t")
    s2 = _fp8_scale_plane(s2t, I // 128, H // 128, "s2t")
    return _packed(F.FMT_FP8, device, u8(w13t), s13, u8(w2t), s2, kmajor=True)


def gpu_moe_layer_fp8(x, topk_ids, topk_weights, w13t, s13t, w2t, s2t, H: int, I: int, K: int,
                      *, device, swiglu_limit: float = 0.0, path="auto"):
    device = torch.device(device)
    H, I = int(H), int(I)
    W = _fp8_weights(w13t, s13t, w2t, s2t, H, I, device)
    if W.H != H or W.I != I:
        raise ValueError(f"weights are H={W.H} I={W.I}, call says H={H} I={I}")
    return moe_forward(x.to(torch.bfloat16).contiguous(), topk_ids, topk_weights, W,
                       swiglu_limit=swiglu_limit, out_dtype=torch.float32, path=path)


def gpu_moe_decode_fp8(x, topk_ids, topk_weights, w13t, s13t, w2t, s2t, H: int, I: int, K: int,
                       *, device, swiglu_limit: float = 0.0):
    path = "decode" if x.shape[0] <= DECODE_MAX_TOKENS else "gemm"
    return gpu_moe_layer_fp8(x, topk_ids, topk_weights, w13t, s13t, w2t, s2t, H, I, K,
                             device=device, swiglu_limit=swiglu_limit, path=path)


def moe_layer(bufs, x, topk_ids, topk_weights, H: int, I: int, *, out=None,
              out_dtype=torch.bfloat16, num_experts: int = 0, swiglu_limit: float = 0.0,
              group_k: int = 32, scale_kind=None, s13_ts=None, s2_ts=None):
    """Small-M fp4 experts from K-major planes; None when outside its envelope
    (T <= 8, top-k <= 8, MXFP4 e8m0 scales in groups of 32)."""
    T, K = topk_ids.shape
    w13t, s13t, w2t, s2t = bufs
    if T > 8 or K > 8 or int(group_k) != 32 or _fp4_kind(s13t, scale_kind) != "e8m0":
        return None
    if s13_ts is not None or s2_ts is not None:
        return None
    dev = x.device
    W = _packed(F.FMT_MXFP4, dev, w13t, s13t, w2t, s2t, kmajor=True, H=int(H), I=int(I))
    if W.H != int(H) or W.I != int(I) or (num_experts and W.n_experts < int(num_experts)):
        return None
    if out is None:
        out = torch.empty((T, int(H)), dtype=out_dtype, device=dev)
    return moe_forward(x.to(torch.bfloat16).contiguous(), topk_ids, topk_weights, W,
                       swiglu_limit=swiglu_limit, out=out, path="decode")
