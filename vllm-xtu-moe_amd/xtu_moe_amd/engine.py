"""Engine surface: the configuration record and the per-format engine
classes the plugin constructs once per layer, with a ``cpu_prefill``-style
forward over the flat routing of a batch.

Mirrors the reference engine's Python binding
(xiaotu_moe/csrc/python_binding/binding.cpp:760-808 class constructor,
:1438-1450 ``cpu_prefill`` -> ``MOE_V2::forward_many`` (moe_v2.hpp:651-957),
:1478-1501 ``MOEConfigV2``; config fields moe_v2.hpp:125-147) and its host
buffer ABI (:1368-1437 ``shard_geometry`` / ``pin_hostbufs`` /
``copy_hostbuf_to_device`` / ``copy_hostbuf_to_device_2d``).  The reference engine computes on the CPU; here
the same call runs the HIP kernels on the weights' device copy, and the
pinned host copy serves the ring stage and the resident pool.  An engine
built ``host_resident=True`` keeps the experts in the pinned host shards
only, as the reference engine does, and streams them through the ring.
"""
from __future__ import annotations

import glob
import os
from dataclasses import dataclass

import torch

from . import formats as F
from .host_store import HostExpertStore
from .layer import ExpertWeights, int8_align_on, moe_forward


@dataclass
class MOEConfigV2:
    num_processes: int = 1
    process_id: int = 0
    gpu_id: int = 0
    has_gate_proj: bool = True
    expert_num: int = 0
    top_k: int = 0
    hidden_size: int = 0
    intermediate_size: int = 0
    max_batch_size: int = 0
    max_num_seqs: int = 0
    stride: int = 32
    group_min_len: int = 10
    group_max_len: int = 4096
    groupN: int = 0
    groupK: int = 0
    swiglu_alpha: float = 1.0    # sigmoid scale inside the gated activation
    swiglu_beta: float = 0.0     # added to `up` before the multiply
    swiglu_limit: float = 0.0    # gate clamped above, up on both sides; 0 = off
    activation_type: int = 0     # 0 plain gated SiLU, 1 clamped SwiGLU
    use_gpu_prefill: bool = False
    int8_activation: int = 0     # 1 = INT8-activation x FP4-code ALIGN path (MXFP4)


class _Engine:
    FMT = None
    GROUP = (1, 1)   # (groupN, groupK) the checkpoint scales use
    HOST = False     # weights kept in host memory, computed by the host engine

    def __init__(self, cfg: MOEConfigV2, w13_weight, w2_weight, w13_scale=0, w2_scale=0,
                 w13_global_scale=0, w2_global_scale=0, device=None, host_resident=False):
        """host_resident: keep the experts in pinned host memory only (the
        reference engine's own residency, moe_v2.hpp:454-640, :1804-1860):
        they are packed on the host straight into the NUMA-node shards of the
        host store, with no device copy; forward_many then streams them
        through the tile ring for device inputs and runs the host engine for
        host inputs, and cpu_decode reads the same shards."""
        if cfg.expert_num <= 0 or cfg.hidden_size <= 0 or cfg.intermediate_size <= 0:
            raise ValueError("MOEConfigV2: expert_num, hidden_size, intermediate_size must be set")
        gn, gk = self.GROUP
        if self.FMT == F.FMT_INT4:
            if cfg.groupN not in (0, 1) or (cfg.groupK and cfg.groupK not in F.INT4_GROUPS):
                raise ValueError(f"MOE_WNA16: groupN must be 1 and groupK one of {F.INT4_GROUPS}")
        elif cfg.groupN and (cfg.groupN, cfg.groupK) != (gn, gk):
            raise ValueError(f"{type(self).__name__}: groupN/groupK must be {gn}/{gk}")
        if cfg.int8_activation and self.FMT != F.FMT_MXFP4:
            raise ValueError("int8_activation needs MXFP4 (e8m0) weights")
        self.cfg = cfg
        opt = lambda v: None if (v is None or isinstance(v, int)) else v
        self.host_resident = bool(host_resident) and not self.HOST
        self.device = (torch.device(device) if device is not None else
                       (w13_weight.device if getattr(w13_weight, "is_cuda", False)
                        else torch.device("cuda")))
        dev = torch.device("cpu") if (self.HOST or self.host_resident) else self.device
        W = ExpertWeights.from_dense(self.FMT, w13_weight, opt(w13_scale), w2_weight,
                                     opt(w2_scale), opt(w13_global_scale), opt(w2_global_scale),
                                     device=dev)
        self.H, self.I, self.E = W.H, W.I, W.E
        self._store = None
        self._cpu = []          # host engines; the last one is current (see _host_engine)
        self._fwd = None        # host-only engine of forward_many (host-format engines)
        if self.host_resident:
            # the packed host copy goes straight into the pinned shards and
            # is dropped: the shards are the only copy of the experts
            self._store = HostExpertStore.from_weights(W, ns=self.shard_count(),
                                                       pin=torch.cuda.is_available())
            self.weights = None
        else:
            self.weights = W

    # ------------------------------------------------------------ forward
    def forward_many(self, qlen: int, top_k: int, expert_ids, weights, x, out):
        """out[qlen, H] fp32 = sum_k weights * expert(ids)(x) (ids >= expert_num
        and zero weights contribute nothing)."""
        c = self.cfg
        ids = expert_ids.reshape(qlen, top_k).to(torch.int32)
        ids = torch.where(ids < 0, torch.full_like(ids, -1), ids)
        lim = c.swiglu_limit if c.activation_type == 1 else 0.0
        if self.host_resident:
            return self._forward_host_resident(qlen, top_k, ids, weights, x, out, lim)
        res = moe_forward(x.reshape(qlen, c.hidden_size).to(torch.bfloat16).contiguous(), ids,
                          weights.reshape(qlen, top_k).float(), self.weights, swiglu_limit=lim,
                          swiglu_alpha=c.swiglu_alpha, swiglu_beta=c.swiglu_beta,
                          out_dtype=torch.float32, int8="auto" if c.int8_activation else False, path="auto")
        out.view(qlen, c.hidden_size).copy_(res)
        return out

    def _forward_host_resident(self, qlen, top_k, ids, weights, x, out, lim):
        """forward_many of a host-resident engine: device inputs stream the
        routed experts through the tile ring (the reference's long-prefill
        path, gpu_prefill.py:2984-3095); host inputs, or a layer the ring
        cannot take, run the host engine over the same shards."""
        from .ring import gpu_moe_layer_from_engine_tiled
        c = self.cfg
        xs = x.reshape(qlen, c.hidden_size).to(torch.bfloat16).contiguous()
        w = weights.reshape(qlen, top_k).float().contiguous()
        res = None
        if xs.is_cuda and not torch.cuda.is_current_stream_capturing():
            res = gpu_moe_layer_from_engine_tiled(
                self._store, xs, ids.to(xs.device), w.to(xs.device), self.H, self.I, self.E,
                top_k, device=xs.device, out_dtype=torch.float32, swiglu_limit=lim,
                swiglu_alpha=c.swiglu_alpha, swiglu_beta=c.swiglu_beta,
                int8=bool(c.int8_activation) and int8_align_on(qlen))
        if res is None:
            if self._fwd is None:
                from .cpu_experts import CpuExperts
                self._fwd = CpuExperts.from_store(self._store, swiglu_limit=lim,
                                                  swiglu_alpha=c.swiglu_alpha,
                                                  swiglu_beta=c.swiglu_beta)
            if xs.is_cuda:
                torch.cuda.current_stream(xs.device).synchronize()
            res = self._fwd.forward(xs.cpu(), ids.cpu(), w.cpu())
        out.view(qlen, c.hidden_size).copy_(res)
        return out

    def cpu_prefill(self, qlen, top_k, expert_ids, weights, input, output):
        """Same call and meaning as the reference engine's cpu_prefill (the
        work runs on the GPU here)."""
        return self.forward_many(qlen, top_k, expert_ids, weights, input, output)

    # ------------------------------------------------------ host buffers
    def host_store(self) -> HostExpertStore:
        """The pinned host copy of the experts, in shard_count() NUMA-node
        shards (built on first use)."""
        if self._store is None:
            self._store = HostExpertStore.from_weights(self.weights, ns=self.shard_count())
        return self._store

    def shard_count(self) -> int:
        """Shards of the host copy: XIAOTU_MOE_NSHARD when >= 2, else the
        host's NUMA node count; 1 when I and H do not split into 16-row
        panels that many ways (as the reference engine falls back to one
        copy, moe_v2.hpp:584-604)."""
        try:
            ns = int(os.environ.get("XIAOTU_MOE_NSHARD", "0") or 0)
        except ValueError:
            ns = 0
        if ns < 2:
            ns = max(1, len(glob.glob("/sys/devices/system/node/node[0-9]*")))
        if ns < 2 or self.I % (16 * ns) or self.H % (16 * ns):
            return 1
        return ns

    # ------------------------------------------------ host decode bridge
    def _host_engine(self, max_qlen: int = 0, top_k: int = 0):
        """The host engine with staging for at least max_qlen tokens of
        top_k pairs (at least 64 tokens, as the reference pre-sizes), or None
        when it would have to grow inside a graph capture.  A grown engine
        replaces the current one; the old one stays alive, since captured
        graphs may still replay into its staging."""
        from .cpu_experts import CpuExperts
        c = self.cfg
        need_t = max(64, int(max_qlen))
        need_k = max(int(c.top_k or 0), int(top_k), 1)
        cur = self._cpu[-1] if self._cpu else None
        if cur is not None and cur.max_tokens >= need_t and cur.max_topk >= need_k:
            return cur
        if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
            return None
        lim = c.swiglu_limit if c.activation_type == 1 else 0.0
        if cur is not None:
            need_t, need_k = max(need_t, cur.max_tokens), max(need_k, cur.max_topk)
        eng = CpuExperts.from_store(self.host_store(), swiglu_limit=lim,
                                    swiglu_alpha=c.swiglu_alpha, swiglu_beta=c.swiglu_beta,
                                    max_tokens=need_t, max_topk=need_k)
        self._cpu.append(eng)
        return eng

    def prepare_decode_buffers(self, max_qlen: int, top_k: int) -> None:
        """Size the pinned decode staging before any graph capture
        (binding.cpp:848-858)."""
        if int(max_qlen) > 0 and int(top_k) > 0:
            self._host_engine(max_qlen, top_k)

    def cpu_decode(self, stream, qlen, top_k, hidden, expert_ids, weights, out_gpu,
                   layer: int = -1, defer: int = 0) -> int:
        """binding.cpp:859-1296: on `stream`, out_gpu[:qlen] (fp32 [qlen, H],
        device) = this layer's experts computed on the host for hidden (bf16
        [qlen, H]), expert_ids (int32) and weights (fp32) [qlen, top_k] (device
        tensors or pointers), through pinned staging and a host-function node
        (graph-capturable).  0 = queued; -1 = out_gpu too small; -2 = the
        staging would have to grow during a capture (call
        prepare_decode_buffers first).  Ids outside [0, expert_num + shared)
        and zero weights add nothing."""
        eng = self._host_engine(qlen, top_k)
        if eng is None:
            return -2
        return eng.cpu_decode(stream, qlen, top_k, hidden, expert_ids, weights, out_gpu, layer,
                              defer)

    def shard_geometry(self) -> dict:
        return self.host_store().shard_geometry()

    def pin_hostbufs(self) -> int:
        return self.host_store().pin_hostbufs()

    def copy_hostbuf_to_device(self, which: int, node: int, dst: int, stream=None) -> int:
        """Buffer `which` (0 w13 shard, 1 w2 shard, 2 s13, 3 s2) of NUMA node
        `node` -> device address dst on `stream`; returns bytes (0: none)."""
        return self.host_store().copy_hostbuf_to_device(which, node, dst, stream)

    def copy_hostbuf_to_device_2d(self, which: int, node: int, src_off: int, dst: int,
                                  dpitch: int, spitch: int, width: int, height: int,
                                  stream=None) -> int:
        """Pitched copy out of buffer `which` of `node` (0 on a bad request)."""
        return self.host_store().copy_hostbuf_to_device_2d(which, node, src_off, dst, dpitch,
                                                           spitch, width, height, stream)


class MOE_WNA16(_Engine):
    """INT4 W4A16 (WNA16) experts: code - 8 times an fp32 scale per (row,
    group_k k).  The reference's MOE_WNA16 is a CPU engine
    (binding.cpp:1514; moe_v2_packed4_base.inc:1594), and so is this one: the
    weights stay in host memory and forward_many / cpu_prefill / cpu_decode
    run the host engine (cpu_experts.CpuExperts)."""
    FMT = F.FMT_INT4
    GROUP = (1, 128)
    HOST = True

    def forward_many(self, qlen: int, top_k: int, expert_ids, weights, x, out):
        c = self.cfg
        if self._fwd is None:
            from .cpu_experts import CpuExperts
            lim = c.swiglu_limit if c.activation_type == 1 else 0.0
            self._fwd = CpuExperts.from_weights(self.weights, swiglu_limit=lim,
                                                swiglu_alpha=c.swiglu_alpha,
                                                swiglu_beta=c.swiglu_beta)
        ids = expert_ids.reshape(qlen, top_k).to(torch.int32).cpu()
        res = self._fwd.forward(x.reshape(qlen, c.hidden_size).to(torch.bfloat16).cpu(), ids,
                                weights.reshape(qlen, top_k).float().cpu())
        out.view(qlen, c.hidden_size).copy_(res)
        return out


class MOE_BF16(_Engine):
    FMT = F.FMT_BF16
    GROUP = (1, 1)


class MOE_FP8(_Engine):
    FMT = F.FMT_FP8
    GROUP = (128, 128)


class MOE_MXFP4(_Engine):
    FMT = F.FMT_MXFP4
    GROUP = (1, 32)


class MOE_NVFP4(_Engine):
    FMT = F.FMT_NVFP4
    GROUP = (1, 16)


ENGINES = {"MOE_BF16": MOE_BF16, "MOE_FP8": MOE_FP8, "MOE_MXFP4": MOE_MXFP4,
           "MOE_NVFP4": MOE_NVFP4, "MOE_WNA16": MOE_WNA16}
