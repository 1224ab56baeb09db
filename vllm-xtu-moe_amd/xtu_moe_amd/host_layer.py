"""Layers whose experts stay in host memory, and which layers stay there.

The reference hook keeps a layer's experts on the GPU only when asked to
(``XIAOTU_MOE_GPU_RESIDENT_LAYERS``, vllm_xiaotu_moe/hybrid_model.py:52-75,
mixed_experts.py:1169-1230); every other layer lives in the CPU engine's
host shards and, per call (mixed_experts.py:1990-2163, :2416-2440,
:2908-3186):

* a long prefill (at least ``VLLM_XIAOTU_GPU_PREFILL_MIN_TOKENS`` tokens, not
  under graph capture) streams the layer's experts through the tile ring;
* otherwise, with a hot-expert pool for the layer, the pool's experts run on
  the GPU and the rest on the host engine (the pin split), the pool noting
  the routing and re-planning (``maybe_adapt``) outside capture;
* otherwise the host engine computes the whole layer (``cpu_decode``).

``HostResidentLayer`` is that per-call choice over one layer's
``HostExpertStore`` (pinned NUMA-node shards, packed on the host with no
device copy), its ``CpuExperts`` host engine, the process's tile ring and
an optional ``LayerPool``.  ``resident_decision`` is the load-time choice:
the reference's layer list when it is set, else a budget of device memory
for resident experts (``XTU_EXPERT_HBM_FRACTION`` of the device, 0.6 by
default): layers are resident in load order while they fit, so a model whose
experts exceed HBM loads with its later layers host-resident.
"""
from __future__ import annotations

import os
import re

import torch

from . import formats as F
from .cpu_experts import CpuExperts
from .cpu_split import PoolSplitLayer
from .expert_pool import LayerPool, build_layer_pool
from .host_store import HostExpertStore
from .layer import ExpertWeights, _buf
from .ring import _nslots_default, gpu_moe_layer_from_engine_tiled

RESIDENT_LAYERS_ENV = "XIAOTU_MOE_GPU_RESIDENT_LAYERS"
HBM_FRACTION_ENV = "XTU_EXPERT_HBM_FRACTION"
HBM_FRACTION_DEFAULT = 0.6
PREFILL_MIN_ENV = "VLLM_XIAOTU_GPU_PREFILL_MIN_TOKENS"   # the reference's knob
PREFILL_MIN_DEFAULT = 256
PIN_SLOTS_ENV = "XTU_PIN_SLOTS"
PIN_STATIC_ENV = "XIAOTU_PIN_STATIC"
PREALLOC_TOKENS_ENV = "XTU_CD_PREALLOC_TOKENS"
LAYER_IDX_RE = re.compile(r"layers\.(\d+)\.")

# expert bytes made resident through the hook so far, per device
_RESIDENT_BYTES: dict = {}


def parse_layer_set(spec: str) -> set:
    """"0-4,10" -> {0, 1, 2, 3, 4, 10} (bad parts are skipped, as the
    reference's gpu_resident_layers does)."""
    out: set = set()
    for part in (spec or "").split(","):
        part = part.strip()
        if not part:
            continue
        try:
            if "-" in part:
                a, b = part.split("-", 1)
                out.update(range(int(a), int(b) + 1))
            else:
                out.add(int(part))
        except ValueError:
            continue
    return out


def layer_index(layer):
    """The decoder-layer index in a vLLM layer name ("model.layers.3.mlp...")
    or None."""
    m = LAYER_IDX_RE.search(getattr(layer, "layer_name", "") or "")
    return int(m.group(1)) if m else None


def resident_decision(layer, nbytes: int, device, total=None) -> bool:
    """Whether a layer's experts (nbytes in the device layout) are kept in
    HBM: listed in XIAOTU_MOE_GPU_RESIDENT_LAYERS when that is set (unnamed
    layers are then host-resident, as in the reference), else while the
    experts made resident so far plus these fit XTU_EXPERT_HBM_FRACTION of
    the device's memory (`total` bytes; the device's own by default)."""
    spec = os.environ.get(RESIDENT_LAYERS_ENV)
    if spec is not None and spec.strip():
        idx = layer_index(layer)
        return idx is not None and idx in parse_layer_set(spec)
    try:
        frac = float(os.environ.get(HBM_FRACTION_ENV, HBM_FRACTION_DEFAULT))
    except ValueError:
        frac = HBM_FRACTION_DEFAULT
    dev = torch.device(device)
    if total is None:
        if not torch.cuda.is_available():
            return True   # no device to budget: the caller's device placement decides
        total = torch.cuda.get_device_properties(dev).total_memory
    used = _RESIDENT_BYTES.get(str(dev), 0)
    if used + int(nbytes) > frac * total:
        return False
    _RESIDENT_BYTES[str(dev)] = used + int(nbytes)
    return True


def gpu_prefill_min_tokens() -> int:
    """Tokens from which a host-resident layer streams through the ring: the
    reference's VLLM_XIAOTU_GPU_PREFILL_MIN_TOKENS when set (0 turns the ring
    off, gpu_prefill.py:61-85), else 256 (the ring beats the host engine from
    a few hundred tokens on: a DeepSeek-V3 FP8 layer streams in ~0.2 s over
    the host link, while the host engine spends ~0.5 ms per token)."""
    v = os.environ.get(PREFILL_MIN_ENV)
    if v is None or not v.strip():
        return PREFILL_MIN_DEFAULT
    try:
        return int(v)
    except ValueError:
        return 0


class HostResidentLayer:
    """One layer whose experts live in pinned host memory (see the module
    docstring for the per-call choice)."""

    def __init__(self, fmt, w13, s13, w2, s2, g13=None, g2=None, *, device, top_k: int,
                 layer_idx=None, swiglu_limit=0.0, swiglu_alpha=1.0, swiglu_beta=0.0,
                 expert_map=None, group_k: int = 32, ns: int = 1):
        self.fmt = int(fmt)
        self.device = torch.device(device)
        # packed on the host (the same P16 layout the kernels read), copied
        # into the pinned node shards, then dropped
        W = ExpertWeights.from_dense(self.fmt, w13, s13, w2, s2, g13, g2, device="cpu")
        self.H, self.I, self.E = W.H, W.I, W.E
        self.store = HostExpertStore.from_weights(W, ns=ns, pin=True)
        del W
        self.top_k = int(top_k)
        self.act = dict(swiglu_limit=float(swiglu_limit), swiglu_alpha=float(swiglu_alpha),
                        swiglu_beta=float(swiglu_beta))
        pre = int(os.environ.get(PREALLOC_TOKENS_ENV, "512") or 512)
        self.cpu = CpuExperts.from_store(self.store, max_tokens=max(pre, 1),
                                         max_topk=max(self.top_k, 1), **self.act)
        self.pool = self._build_pool(layer_idx, expert_map, group_k)
        self.split = PoolSplitLayer(self.pool, self.cpu, self.device) if self.pool else None
        self.last_path = None

    def _build_pool(self, layer_idx, expert_map, group_k):
        """The layer's hot-expert pool: from the pin table (XTU_PIN=1 and
        XTU_PIN_TABLE, expert_pool.build_layer_pool), else XTU_PIN_SLOTS slots
        starting with experts 0.. (the adaptation then swaps the hot ones
        in), else none."""
        layout = F.FMT_NAMES[self.fmt]
        if layer_idx is not None:
            pool = build_layer_pool(self.store, self.device, self.H, self.I, group_k, self.E,
                                    int(layer_idx), expert_map, topk=self.top_k, layout=layout)
            if pool is not None:
                return pool
        n = int(os.environ.get(PIN_SLOTS_ENV, "0") or 0)
        if n <= 0:
            return None
        return LayerPool(self.store, self.device, self.H, self.I, group_k, self.E,
                         list(range(min(n, self.E))), -1 if layer_idx is None else int(layer_idx),
                         layout=layout, topk=self.top_k)

    def device_bytes(self) -> int:
        """Device bytes this layer holds itself (its pool's slots)."""
        if self.pool is None:
            return 0
        planes = [getattr(self.pool.planes, n) for n in ("w13", "s13", "w2", "s2", "gs13", "gs2")]
        return sum(t.numel() * t.element_size() for t in planes if t is not None)

    def forward(self, x, ids, wts, *, int8=False):
        """out fp32 [T, H] of the layer for device x (bf16 [T, H]), ids (int32)
        and weights (fp32) [T, K]."""
        T, K = ids.shape
        capturing = torch.cuda.is_current_stream_capturing()
        gp_min = gpu_prefill_min_tokens()
        gpu_pf = gp_min > 0 and T >= gp_min and not capturing
        if self.pool is not None:
            # routing counts on the device (capturable), re-planned outside
            # capture; not while this call streams (mixed_experts.py:2911-2921)
            self.pool.note_routing(ids)
            if not capturing and os.environ.get(PIN_STATIC_ENV, "0") != "1":
                self.pool.maybe_adapt(None, staging_active=gpu_pf)
        if gpu_pf:
            out = gpu_moe_layer_from_engine_tiled(
                self.store, x, ids, wts, self.H, self.I, self.E, K, device=self.device,
                nslots=_nslots_default(None), pool=self.pool, out_dtype=torch.float32,
                int8=int8, **self.act)
            if out is not None:
                self.last_path = "ring"
                return out
        if self.split is not None and T <= self.cpu.max_tokens and K <= self.cpu.max_topk:
            self.last_path = "split"
            return self.split.forward(x, ids, wts, note_routing=False, **self.act)
        out = _buf("host_layer_out", (T, self.H), torch.float32, self.device)
        if T <= self.cpu.max_tokens and K <= self.cpu.max_topk:
            rc = self.cpu.cpu_decode(torch.cuda.current_stream(self.device).cuda_stream, T, K,
                                     x, ids, wts, out)
            if rc:
                raise RuntimeError(f"host engine did not take the batch (cpu_decode {rc})")
            self.last_path = "host"
            return out.clone()
        if capturing:
            raise RuntimeError(f"a {T}-token batch exceeds the host engine's staging "
                               f"({self.cpu.max_tokens} tokens) inside a graph capture")
        torch.cuda.current_stream(self.device).synchronize()
        self.last_path = "host-sync"
        return self.cpu.forward(x.cpu(), ids.cpu(), wts.cpu()).to(self.device)
