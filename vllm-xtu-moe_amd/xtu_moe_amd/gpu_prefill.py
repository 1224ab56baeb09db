"""Layer entries with the reference's signatures, over the HIP library.

* ``gpu_moe_layer`` -- vllm_xiaotu_moe/gpu_prefill.py:2566-2780: one layer's
  routed experts from fp4 checkpoint planes (MXFP4: e8m0 scales, group 32;
  NVFP4: e4m3 scales, group 16, per-expert global scales s13_ts / s2_ts),
  on the device or on the host, or from a resident slot (``slot.bufs``,
  topk_ids then index the slot's rows); out [T, H] (bf16 by default).
* ``gpu_moe_layer_fp8`` -- gpu_prefill_fp8.py:458: FP8 block-scaled
  experts from K-major planes w13t [S, H, 2I] / s13t [S, H/128, 2I/128] and
  w2t [S, I, H] / s2t [S, I/128, H/128]; out fp32.
* ``gpu_moe_decode_fp8`` -- decode_moe_fp8.py:103: the same planes on the
  skinny-M decode kernels; out fp32.
* ``moe_layer`` -- moe4_smallm.py:151-341: small-M fp4 experts from K-major
  planes [S, H/2, 2I], [S, H/32, 2I], [S, I/2, H], [S, I/32, H]; returns
  None (caller falls back) outside T <= 8, top-k <= 8, group 32, e8m0.
* The ring-stage entries are re-exported from ``ring``.

Checkpoint planes are packed once into the device layout and cached by
their storage (address, shape, strides), as the reference caches its
K-major copies.
"""
from __future__ import annotations

import torch

from . import formats as F
from .layer import DECODE_MAX_TOKENS, ExpertWeights, moe_forward
from .ring import (gpu_moe_layer_from_engine_tiled, prealloc_tile_ring,  # noqa: F401
                   stage_tiles, staging_bytes, staging_tile_experts)

_PACKED: dict = {}


def _key(*ts):
    return tuple((None if t is None else (t.data_ptr(), tuple(t.shape), tuple(t.stride()),
                                          str(t.dtype), str(t.device))) for t in ts)


def _packed(fmt, device, w13, s13, w2, s2, g13=None, g2=None, kmajor=False):
    key = (fmt, str(device), kmajor) + _key(w13, s13, w2, s2, g13, g2)
    W = _PACKED.get(key)
    if W is None:
        if kmajor:   # [S, K(packed), N] -> [S, N, K(packed)]
            tr = lambda t: None if t is None else t.transpose(1, 2).contiguous()
            w13, s13, w2, s2 = tr(w13), tr(s13), tr(w2), tr(s2)
        W = ExpertWeights.from_dense(fmt, w13.to(device), None if s13 is None else s13.to(device),
                                     w2.to(device), None if s2 is None else s2.to(device),
                                     None if g13 is None else g13.to(device).float(),
                                     None if g2 is None else g2.to(device).float(), device=device)
        _PACKED[key] = W
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
    kind = _fp4_kind(s13, scale_kind)
    fmt = F.FMT_NVFP4 if kind == "e4m3" else F.FMT_MXFP4
    if int(group_k) != (16 if fmt == F.FMT_NVFP4 else 32):
        raise ValueError(f"{kind} scales come in groups of {16 if fmt == F.FMT_NVFP4 else 32}")
    if slot is not None:
        if not torch.cuda.is_current_stream_capturing():
            torch.cuda.current_stream(device).wait_event(slot.ready)
        W = slot.bufs
    else:
        W = _packed(fmt, device, w13, s13, w2, s2, s13_ts, s2_ts)
    if W.H != int(H) or W.I != int(I):
        raise ValueError(f"weights are H={W.H} I={W.I}, call says H={H} I={I}")
    moe_forward(x.to(torch.bfloat16).contiguous(), topk_ids, topk_weights, W,
                swiglu_limit=swiglu_limit, out=out)
    if slot is not None and not torch.cuda.is_current_stream_capturing():
        slot.busy = torch.cuda.Event()
        slot.busy.record(torch.cuda.current_stream(device))
    return out


def gpu_moe_layer_fp8(x, topk_ids, topk_weights, w13t, s13t, w2t, s2t, H: int, I: int, K: int,
                      *, device, swiglu_limit: float = 0.0, path="auto"):
    device = torch.device(device)
    u8 = lambda t: t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t
    W = _packed(F.FMT_FP8, device, u8(w13t), s13t.float(), u8(w2t), s2t.float(), kmajor=True)
    if W.H != int(H) or W.I != int(I):
        raise ValueError(f"weights are H={W.H} I={W.I}, call says H={H} I={I}")
    return moe_forward(x.to(torch.bfloat16).contiguous(), topk_ids, topk_weights, W,
                       swiglu_limit=swiglu_limit, out_dtype=torch.float32, path=path)


def gpu_moe_decode_fp8(x, topk_ids, topk_weights, w13t, s13t, w2t, s2t, H: int, I: int, K: int,
                       *, device, swiglu_limit: float = 0.0):
    if x.shape[0] > DECODE_MAX_TOKENS:
        raise ValueError(f"decode path takes at most {DECODE_MAX_TOKENS} tokens")
    return gpu_moe_layer_fp8(x, topk_ids, topk_weights, w13t, s13t, w2t, s2t, H, I, K,
                             device=device, swiglu_limit=swiglu_limit, path="decode")


def moe_layer(bufs, x, topk_ids, topk_weights, H: int, I: int, *, out=None,
              out_dtype=torch.bfloat16, num_experts: int = 0, swiglu_limit: float = 0.0,
              group_k: int = 32, scale_kind=None, s13_ts=None, s2_ts=None):
    """Small-M fp4 experts from K-major planes; None when outside its envelope
    (T <= 8, top-k <= 8, MXFP4 e8m0 scales in groups of 32)."""
    T, K = topk_ids.shape
    w13t, s13t, w2t, s2t = bufs
    if T > 8 or K > 8 or int(group_k) != 32 or _fp4_kind(s13t, scale_kind) != "e8m0":
        return None
    dev = x.device
    W = _packed(F.FMT_MXFP4, dev, w13t, s13t, w2t, s2t, kmajor=True)
    if W.H != int(H) or W.I != int(I) or (num_experts and W.n_experts != int(num_experts)):
        return None
    if out is None:
        out = torch.empty((T, int(H)), dtype=out_dtype, device=dev)
    return moe_forward(x.to(torch.bfloat16).contiguous(), topk_ids, topk_weights, W,
                       swiglu_limit=swiglu_limit, out=out, path="decode")
