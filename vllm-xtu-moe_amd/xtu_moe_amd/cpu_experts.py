"""Host expert engine: the CPU half of the pool-miss split.

``CpuExperts`` runs a layer's experts on the host, reading the weights where
the host store keeps them (the P16 rows of ``HostExpertStore``'s NUMA-node
shards and its scale planes; no second copy), through the library's
``xtu_cpu_*`` entry points.  ``cpu_decode`` is the reference engine's
graph-capturable stream bridge (xiaotu_moe/csrc/python_binding/binding.cpp:
859-1296, called at vllm_xiaotu_moe/mixed_experts.py:3146-3160): device rows,
ids and weights are copied to pinned staging, a host-function node runs the
engine, and its fp32 result is copied into ``out_gpu``.

The reference's deferred mode (``defer=1``: return the previous layer's
result, queue this one) and its sidecar ``layer`` routing are not part of
this engine: ``layer`` is accepted and unused, ``defer`` must be 0.
"""
from __future__ import annotations

import ctypes
import os

import torch

from . import _lib

ISA_AUTO, ISA_PORTABLE, ISA_AVX512 = -1, 0, 2


def _ptr(t) -> int:
    return 0 if t is None else int(t.data_ptr())


def host_threads() -> int:
    """Threads the engine uses by default: the CPUs this process may run on,
    at most XTU_CPU_THREADS when that is set."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    cap = int(os.environ.get("XTU_CPU_THREADS", "0") or 0)
    return max(1, min(n, cap) if cap > 0 else n)


class CpuExperts:
    """Host engine over one layer's experts.

    planes: ``w13_nodes`` / ``w2_nodes`` (lists of ns host uint8 tensors
    ``[n_experts, bytes]``: per expert the node's gate rows then its up rows
    of w13, and its rows of w2, P16), ``s13`` / ``s2`` (packed scale groups or
    fp32 block scales, ``[n_experts, ...]``), ``gs13`` / ``gs2`` (NVFP4).
    ``max_tokens`` > 0 allocates the pinned staging ``cpu_decode`` needs
    (needs a GPU runtime); 0 makes a host-only engine (``forward``)."""

    def __init__(self, fmt, H, I, n_experts, w13_nodes, w2_nodes, s13=None, s2=None, gs13=None,
                 gs2=None, *, group_k=0, swiglu_limit=0.0, swiglu_alpha=1.0, swiglu_beta=0.0,
                 n_threads=None, isa=ISA_AUTO, max_tokens=0, max_topk=16):
        self.fmt, self.H, self.I, self.n_experts = int(fmt), int(H), int(I), int(n_experts)
        ns = len(w13_nodes)
        if ns != len(w2_nodes) or not 1 <= ns <= 8:
            raise ValueError("w13_nodes and w2_nodes must list the same 1..8 node buffers")
        for t in list(w13_nodes) + list(w2_nodes) + [s13, s2, gs13, gs2]:
            if t is not None and (t.device.type != "cpu" or not t.is_contiguous()):
                raise ValueError("host engine planes must be contiguous host tensors")
        # the engine reads these in place: keep them alive with it
        self._keep = [list(w13_nodes), list(w2_nodes), s13, s2, gs13, gs2]
        n13 = (ctypes.c_void_p * ns)(*[_ptr(t) for t in w13_nodes])
        n2 = (ctypes.c_void_p * ns)(*[_ptr(t) for t in w2_nodes])
        self._node_arrays = (n13, n2)
        es = lambda t: 0 if t is None else t[0].numel() * t.element_size()
        self.max_tokens, self.max_topk = int(max_tokens), int(max_topk)
        self.limit = float(swiglu_limit)
        eng = ctypes.c_void_p()
        _lib.call("xtu_cpu_engine_create", self.fmt, self.H, self.I, self.n_experts, ns,
                  ctypes.addressof(n13), es(w13_nodes[0]), ctypes.addressof(n2), es(w2_nodes[0]),
                  _ptr(s13), es(s13), _ptr(s2), es(s2), _ptr(gs13), _ptr(gs2), int(group_k),
                  float(swiglu_limit), float(swiglu_alpha), float(swiglu_beta),
                  int(n_threads or host_threads()), int(isa), self.max_tokens, self.max_topk,
                  ctypes.addressof(eng))
        self._eng = eng
        isa_o, thr = ctypes.c_int(), ctypes.c_int()
        _lib.call("xtu_cpu_engine_info", eng, ctypes.addressof(isa_o), ctypes.addressof(thr))
        self.isa, self.n_threads = isa_o.value, thr.value

    @classmethod
    def from_store(cls, store, **kw) -> "CpuExperts":
        """Over a ``HostExpertStore`` (its node shards and scale planes)."""
        p = store.planes
        kw.setdefault("group_k", getattr(store, "group_k", 0))
        return cls(store.fmt, store.H, store.I, store.n_experts, store.w13_shard, store.w2_shard,
                   p.get("s13"), p.get("s2"), p.get("gs13"), p.get("gs2"), **kw)

    @classmethod
    def from_weights(cls, W, **kw) -> "CpuExperts":
        """Over host copies of an ``ExpertWeights`` (one node shard)."""
        h = lambda t: None if t is None else t.detach().to("cpu").contiguous()
        kw.setdefault("group_k", getattr(W, "group_k", 0))
        return cls(W.fmt, W.H, W.I, W.E + W.n_shared, [h(W.w13)], [h(W.w2)], h(W.s13), h(W.s2),
                   h(W.gs13), h(W.gs2), **kw)

    # ----------------------------------------------------------------- use
    def forward(self, x, topk_ids, topk_weights, out=None):
        """Host tensors: x bf16 [T, H], ids int32 / weights fp32 [T, K] ->
        out fp32 [T, H] (pairs with invalid ids or zero weight add nothing)."""
        T, K = topk_ids.shape
        x = x.to(torch.bfloat16).contiguous()
        ids = topk_ids.to(torch.int32).contiguous()
        wts = topk_weights.to(torch.float32).contiguous()
        if out is None:
            out = torch.empty((T, self.H), dtype=torch.float32)
        for t, d in ((x, "cpu"), (ids, "cpu"), (wts, "cpu"), (out, "cpu")):
            if t.device.type != d:
                raise ValueError("forward takes host tensors (cpu_decode takes device ones)")
        if tuple(x.shape) != (T, self.H) or out.dtype != torch.float32 or \
                tuple(out.shape) != (T, self.H) or not out.is_contiguous():
            raise ValueError("x must be [T, H] and out fp32 [T, H] contiguous")
        _lib.call("xtu_cpu_forward", self._eng, int(T), int(K), _ptr(x), _ptr(ids), _ptr(wts),
                  _ptr(out))
        return out

    def cpu_decode(self, stream, qlen, top_k, hidden, expert_ids, weights, out_gpu, layer=-1,
                   defer=0) -> int:
        """The reference engine's cpu_decode: on `stream` (a handle or None
        for the current stream), out_gpu[:qlen] (fp32 [qlen, H], device) =
        the host engine over hidden (bf16 [qlen, H]), expert_ids (int32) and
        weights (fp32) [qlen, top_k], all device memory; arguments may be
        tensors or data pointers.  Returns 0 when queued, -1 when out_gpu has
        fewer than qlen rows, -2 when qlen or top_k exceeds the staging the
        engine was built with (the layer is then not computed, as the
        reference's non-zero codes say)."""
        if int(defer):
            raise NotImplementedError("deferred cpu_decode (defer=1) is not provided")
        qlen, top_k = int(qlen), int(top_k)
        if qlen <= 0 or top_k <= 0:
            return 0
        if torch.is_tensor(out_gpu) and (out_gpu.dtype != torch.float32 or out_gpu.dim() != 2
                                         or out_gpu.shape[0] < qlen
                                         or out_gpu.shape[1] != self.H
                                         or not out_gpu.is_contiguous()):
            return -1
        if qlen > self.max_tokens or top_k > self.max_topk:
            return -2
        for t in (hidden, expert_ids, weights):
            if torch.is_tensor(t) and not t.is_contiguous():
                raise ValueError("cpu_decode needs contiguous device tensors")
        if torch.is_tensor(hidden) and hidden.dtype != torch.bfloat16:
            raise ValueError("hidden must be bf16")
        if torch.is_tensor(expert_ids) and expert_ids.dtype != torch.int32:
            raise ValueError("expert_ids must be int32")
        if torch.is_tensor(weights) and weights.dtype != torch.float32:
            raise ValueError("weights must be fp32")
        p = lambda a: int(a.data_ptr()) if torch.is_tensor(a) else int(a)
        if stream is None:
            stream = torch.cuda.current_stream().cuda_stream
        _lib.call("xtu_cpu_decode", self._eng, qlen, top_k, p(hidden), p(expert_ids),
                  p(weights), p(out_gpu), int(stream))
        return 0

    def close(self):
        """Free the engine (after its streams are synchronised and the
        graphs that captured its cpu_decode calls are gone)."""
        if getattr(self, "_eng", None) is not None and self._eng.value:
            _lib.call("xtu_cpu_engine_destroy", self._eng)
        self._eng = None

