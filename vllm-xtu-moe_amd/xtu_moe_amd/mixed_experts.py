"""The FusedMoE quant-method hook: what vLLM's MoE layer calls.

Mirrors vllm_xiaotu_moe/mixed_experts.py: ``_XiaotuExpertsMixin``
(:618-3306) -- ``process_weights_after_loading`` (:692-804) reads the layer's
checkpoint weights, scales, routing and SwiGLU attributes;
``apply(hidden_states, w1, w2, router_logits=None, ...)`` (:1919-2123) takes
given (topk_weights, topk_ids) (modular path) or routes from router_logits
(monolithic path), maps global ids through expert_map (misses get weight
0), and returns [T, H] in hidden_states.dtype, written into `output` when
given; ``apply_router_weight_on_input`` raises.  Format subclasses fix the
scale attribute names and the scale groups (:3308-3476): BF16 1x1, MXFP4
1x32, FP8 128x128, NVFP4 1x16 with per-expert second-level scales, and INT4
(WNA16) 1xgroup with the GPTQ / compressed-tensors repack.

Here the experts run on the HIP library with the layer's weights packed once
into the device layout when the layer is resident, or kept in pinned host
shards behind ``host_layer.HostResidentLayer`` (tile ring for long prefill,
pool split or host engine otherwise) when it is not (INT4 always on the
host engine, as the reference's MOE_WNA16); vLLM itself is not needed (an
``activation`` of None or a string name is accepted when vLLM's enum is
absent).  The INT8 ALIGN path follows the reference's environment switches
(``int8_dispatch``).
"""
from __future__ import annotations

import enum

import torch

from . import formats as F
from .host_layer import HostResidentLayer, layer_index, resident_decision
from .layer import ExpertWeights, _buf as _scratch, int8_align_on, int8_dispatch, moe_forward, route

_ROUTING_ATTRS = ("use_grouped_topk", "renormalize", "scoring_func", "custom_routing_function",
                  "num_expert_group", "topk_group", "e_score_correction_bias",
                  "routed_scaling_factor")
_SWIGLU_ATTRS = ("swiglu_limit", "swiglu_alpha", "swiglu_beta")

try:   # vLLM's activation enum when vLLM is installed
    from vllm.model_executor.layers.fused_moe.activation import MoEActivation  # type: ignore
except Exception:  # noqa: BLE001
    class MoEActivation(enum.Enum):
        SILU = "silu"
        SWIGLUOAI_UNINTERLEAVE = "swigluoai_uninterleave"


class XiaotuExperts:
    """Base hook: subclasses set the format, scale attributes and groups."""

    _fmt = F.FMT_BF16
    _scale_attrs: tuple = ("", "")
    _global_scale_attrs: tuple = ("", "")
    _group_n, _group_k = 1, 1

    def __init__(self, moe_config=None, quant_config=None):
        self.moe_config, self.quant_config = moe_config, quant_config
        self._layer_ref = None
        self._weights: ExpertWeights | None = None
        self._host_layer = None      # HostResidentLayer of a layer kept in host memory
        self._int8_allowed = False
        self.use_grouped_topk = False
        self.renormalize = False
        self.scoring_func = "softmax"
        self.custom_routing_function = None
        self.num_expert_group = None
        self.topk_group = None
        self.e_score_correction_bias = None
        self.routed_scaling_factor = 1.0
        self.swiglu_limit = None
        self.swiglu_alpha = None
        self.swiglu_beta = None
        self.top_k = None

    @staticmethod
    def _supports_routing_method(routing_method=None, weight_key=None, activation_key=None) -> bool:
        return True

    @staticmethod
    def _supports_activation(activation) -> bool:
        name = getattr(activation, "name", activation)
        return str(name).upper() in ("SILU", "SWIGLUOAI_UNINTERLEAVE")

    # ---------------------------------------------------------- loading
    def process_weights_after_loading(self, layer) -> None:
        """Packs the layer's experts for the kernels: into HBM when the layer
        is resident (host_layer.resident_decision: the reference's
        XIAOTU_MOE_GPU_RESIDENT_LAYERS list, else a device-memory budget),
        otherwise into pinned host shards behind a HostResidentLayer (ring for
        long prefill, pool split or host engine for the rest)."""
        self._read_layer_attrs(layer)
        self._int8_allowed = int8_dispatch(self._fmt)
        w13, w2 = layer.w13_weight, layer.w2_weight
        s13 = self._find(layer, self._scale_attrs[0])
        s2 = self._find(layer, self._scale_attrs[1])
        g13, g2 = self._global_scales(layer)
        dev = torch.device("cuda") if not w13.is_cuda else w13.device
        w13v, w2v = self._weight_view(w13), self._weight_view(w2)
        H, I = int(w2v.shape[1]), int(w13v.shape[1]) // 2
        nbytes = int(w13v.shape[0]) * F.expert_bytes(self._fmt, H, I)
        if resident_decision(layer, nbytes, dev):
            self._weights = ExpertWeights.from_dense(self._fmt, w13v, s13, w2v, s2, g13, g2,
                                                     device=dev)
            self._host_layer = None
            return
        self._weights = None
        self._host_layer = HostResidentLayer(
            self._fmt, w13v, s13, w2v, s2, g13, g2, device=dev, top_k=int(self.top_k or 1),
            layer_idx=layer_index(layer), group_k=int(self._group_k),
            swiglu_limit=float(self.swiglu_limit or 0.0),
            swiglu_alpha=float(self.swiglu_alpha if self.swiglu_alpha is not None else 1.0),
            swiglu_beta=float(self.swiglu_beta or 0.0))
        self._release_device_sources(layer)

    _SOURCE_ATTRS = ("w13_weight", "w2_weight", "w13_weight_scale", "w2_weight_scale",
                     "w13_weight_scale_inv", "w2_weight_scale_inv", "w13_weight_scale_2",
                     "w2_weight_scale_2")

    def _release_device_sources(self, layer) -> None:
        """A host-resident layer's checkpoint tensors that sit in device
        memory are emptied once the host shards hold the experts (the
        reference releases the source after building its engine,
        mixed_experts.py:2083-2094): the layer's HBM then holds only its pool
        slots.  Their shapes are kept in ``_released_shapes``."""
        if getattr(self, "_released_shapes", None) is None:
            self._released_shapes = {}
        for name in self._SOURCE_ATTRS:
            t = getattr(layer, name, None)
            if not isinstance(t, torch.Tensor) or not t.is_cuda or t.numel() == 0:
                continue
            self._released_shapes[name] = tuple(t.shape)
            t.data = torch.empty(0, dtype=t.dtype, device=t.device)

    def _global_scales(self, layer):
        return None, None

    def _read_layer_attrs(self, layer) -> None:
        self._layer_ref = layer
        for name in _ROUTING_ATTRS + _SWIGLU_ATTRS + ("top_k",):
            if hasattr(layer, name):
                setattr(self, name, getattr(layer, name))
        if self.e_score_correction_bias is None:
            gate = getattr(layer, "gate", None)
            for owner, attr in ((gate, "e_score_correction_bias"), (gate, "bias"),
                                (getattr(layer, "router", None), "e_score_correction_bias")):
                b = getattr(owner, attr, None) if owner is not None else None
                if isinstance(b, torch.Tensor):
                    self.e_score_correction_bias = b
                    break

    @staticmethod
    def _find(layer, name):
        if not name:
            return None
        t = getattr(layer, name, None)
        return t.data if isinstance(t, torch.nn.Parameter) else t

    def _weight_view(self, w):
        w = w.data if isinstance(w, torch.nn.Parameter) else w
        if self._fmt == F.FMT_FP8 and w.dtype == torch.float8_e4m3fn:
            return w.view(torch.uint8)
        return w

    # ----------------------------------------------------------- routing
    def _select_topk(self, hidden_states, router_logits):
        if self.custom_routing_function is not None:
            w, i = self.custom_routing_function(hidden_states, router_logits, self.top_k,
                                                self.renormalize)
            return w.to(torch.float32), i.to(torch.int32)
        if router_logits is None:
            raise ValueError("no topk_ids / topk_weights and no router_logits")
        if self.use_grouped_topk or str(self.scoring_func) == "sigmoid":
            bias = self.e_score_correction_bias
            if bias is not None:
                bias = bias.to(router_logits.device)
            return route(router_logits, top_k=int(self.top_k), scoring=str(self.scoring_func),
                         renormalize=bool(self.renormalize), bias=bias,
                         n_group=int(self.num_expert_group or 1),
                         topk_group=int(self.topk_group or 1),
                         routed_scaling_factor=float(self.routed_scaling_factor or 1.0))
        return route(router_logits, top_k=int(self.top_k), scoring="softmax",
                     renormalize=bool(self.renormalize))

    @staticmethod
    def _local_ids(expert_map, topk_ids, topk_weights):
        em = expert_map.to(device=topk_ids.device, dtype=torch.long)
        local = em[topk_ids.to(torch.long)]
        miss = local < 0
        topk_weights = torch.where(miss, torch.zeros_like(topk_weights), topk_weights)
        local = torch.where(miss, torch.zeros_like(local), local)
        return local.to(torch.int32), topk_weights

    # ------------------------------------------------------------- apply
    def apply(self, hidden_states, w1, w2, router_logits=None, activation=None,
              global_num_experts: int = 0, expert_map=None, a1q_scale=None,
              apply_router_weight_on_input: bool = False, num_expert_group=None,
              e_score_correction_bias=None, routed_scaling_factor=None, topk_group=None, *,
              output=None, topk_weights=None, topk_ids=None, a2_scale=None, workspace13=None,
              workspace2=None, expert_tokens_meta=None):
        if apply_router_weight_on_input:
            raise NotImplementedError("the xiaotu experts backend does not support "
                                      "apply_router_weight_on_input")
        if activation is not None and not self._supports_activation(activation):
            raise NotImplementedError(f"unsupported activation {activation}")
        if self._weights is None and self._host_layer is None:
            raise RuntimeError("apply called before process_weights_after_loading")
        if num_expert_group is not None:
            self.num_expert_group = num_expert_group
        if topk_group is not None:
            self.topk_group = topk_group
        if e_score_correction_bias is not None:
            self.e_score_correction_bias = e_score_correction_bias
        if routed_scaling_factor is not None:
            self.routed_scaling_factor = routed_scaling_factor
        T = hidden_states.shape[0]
        x = hidden_states
        if x.dtype != torch.bfloat16 or not x.is_contiguous():
            x = x.to(torch.bfloat16).contiguous()
        odt = hidden_states.dtype if hidden_states.dtype in (torch.bfloat16, torch.float32) \
            else torch.float32
        H = self._weights.H if self._weights is not None else self._host_layer.H
        direct = (output is not None and output.dtype == odt and output.is_contiguous()
                  and tuple(output.shape) == (T, H) and output.device == x.device)
        kw = dict(swiglu_limit=float(self.swiglu_limit or 0.0),
                  swiglu_alpha=float(self.swiglu_alpha if self.swiglu_alpha is not None else 1.0),
                  swiglu_beta=float(self.swiglu_beta or 0.0),
                  out=output if direct else None, out_dtype=odt)
        if topk_weights is not None and topk_ids is not None:
            res = self._experts(x, topk_ids.to(torch.int32).contiguous(),
                                topk_weights.to(torch.float32).contiguous(), kw)
        elif (self._monolithic and self._weights is not None and expert_map is None
              and self.custom_routing_function is None and router_logits is not None):
            # monolithic path: routing (+ segmentation, + the shared experts'
            # gate/up at decode sizes) inside the layer's own launches
            ids = _scratch("hook_ids", (T, int(self.top_k)), torch.int32, x.device)
            wts = _scratch("hook_wts", (T, int(self.top_k)), torch.float32, x.device)
            res = moe_forward(x, ids, wts, self._weights, router=self._router_args(router_logits),
                              int8=self._int8(T), **kw)
        else:
            topk_weights, topk_ids = self._select_topk(hidden_states, router_logits)
            if expert_map is not None:
                topk_ids, topk_weights = self._local_ids(expert_map, topk_ids, topk_weights)
            res = self._experts(x, topk_ids.contiguous(), topk_weights.contiguous(), kw)
        if direct:
            return output
        res = res.to(hidden_states.dtype)
        if output is not None:
            output.copy_(res)
            return output
        return res

    # routing, segmentation and the experts in the layer's own launches when
    # the router logits are given (GPU formats)
    _monolithic = True

    def _int8(self, T: int) -> bool:
        """Whether a call of T tokens takes the INT8 ALIGN path (MXFP4 only;
        int8_dispatch, then the token gate of int8_align_on)."""
        if self._fmt != F.FMT_MXFP4 or self._int8_allowed is None:
            return False
        return int8_align_on(T, bool(self._int8_allowed))

    def _experts(self, x, ids, wts, kw):
        """The experts over routed pairs: out [T, H] (kw: swiglu_*, out,
        out_dtype)."""
        if self._host_layer is None:
            return moe_forward(x, ids, wts, self._weights, int8=self._int8(x.shape[0]), **kw)
        res = self._host_layer.forward(x, ids, wts, int8=self._int8(x.shape[0]))
        out = kw.get("out")
        if out is not None:
            out.copy_(res)
            return out
        return res.to(kw.get("out_dtype", torch.float32))

    def _router_args(self, router_logits) -> dict:
        lg = router_logits
        if lg.dtype != torch.float32 or not lg.is_contiguous():
            lg = lg.float().contiguous()
        if self.use_grouped_topk or str(self.scoring_func) == "sigmoid":
            bias = self.e_score_correction_bias
            if bias is not None:
                bias = bias.to(device=lg.device, dtype=torch.float32).contiguous()
            return dict(logits=lg, scoring=str(self.scoring_func), bias=bias,
                        n_group=int(self.num_expert_group or 1),
                        topk_group=int(self.topk_group or 1),
                        routed_scaling_factor=float(self.routed_scaling_factor or 1.0),
                        renormalize=bool(self.renormalize))
        return dict(logits=lg, scoring="softmax", renormalize=bool(self.renormalize))


class XiaotuExpertsBF16(XiaotuExperts):
    _fmt = F.FMT_BF16
    _group_n, _group_k = 1, 1


class XiaotuExpertsMxfp4(XiaotuExperts):
    _fmt = F.FMT_MXFP4
    _scale_attrs = ("w13_weight_scale", "w2_weight_scale")
    _group_n, _group_k = 1, 32


class XiaotuExpertsFp8(XiaotuExperts):
    _fmt = F.FMT_FP8
    _scale_attrs = ("w13_weight_scale_inv", "w2_weight_scale_inv")
    _group_n, _group_k = 128, 128


class XiaotuExpertsNvfp4(XiaotuExperts):
    _fmt = F.FMT_NVFP4
    _scale_attrs = ("w13_weight_scale", "w2_weight_scale")
    _global_scale_attrs = ("w13_weight_scale_2", "w2_weight_scale_2")
    _group_n, _group_k = 1, 16

    def _weight_view(self, w):
        return w.data if isinstance(w, torch.nn.Parameter) else w

    def _global_scales(self, layer):
        return nvfp4_global_scales(self._find(layer, self._global_scale_attrs[0]),
                                   self._find(layer, self._global_scale_attrs[1]),
                                   getattr(layer, "prefix", "?"))


def nvfp4_global_scales(g13, g2, where: str = "?"):
    """The per-expert fp32 second-level scales (weight_scale_2) as the
    kernels take them: gate/up as [E, 2] (gate, up) and down as [E].

    Checkpoints give w13's as [E, 2] (w1, w3) or [E]; the kernels multiply
    the gate results by column 0 and the up results by column 1, the
    reference's fold of scale_2 into the fp32 group scales per half
    (vllm_xiaotu_moe/hybrid_model.py:1546-1563: fp32 e4m3(s) * scale_2,
    applied to the e2m1 value), so w1 and w3 scales that differ are taken as
    they are.  All-zero scales mean the loader did not fill them and are
    refused (hybrid_model.py:1550-1556)."""
    if g13 is None or g2 is None:
        raise ValueError(f"[xtu-nvfp4] {where}: weight_scale_2 planes missing")
    g13 = g13.detach().to(torch.float32)
    g2 = g2.detach().to(torch.float32).reshape(-1)
    if g13.dim() == 2 and g13.shape[1] == 1:
        g13 = g13.reshape(-1)
    if g13.dim() == 1:
        g13 = g13[:, None].expand(-1, 2)
    if g13.dim() != 2 or g13.shape[1] != 2:
        raise ValueError(f"[xtu-nvfp4] {where}: w13 weight_scale_2 must be [E] or [E, 2], "
                         f"got {tuple(g13.shape)}")
    if float(g13.abs().max()) == 0.0 or float(g2.abs().max()) == 0.0:
        raise RuntimeError(f"[xtu-nvfp4] {where}: weight_scale_2 is all zero (not loaded)")
    if g13.shape[0] != g2.shape[0]:
        raise ValueError(f"[xtu-nvfp4] {where}: {g13.shape[0]} gate/up vs {g2.shape[0]} down "
                         "second-level scales")
    return g13.contiguous(), g2.contiguous()


# ----------------------------------------------------------------- INT4 / WNA16
def repack_gptq_int4(w, s):
    """GPTQ / compressed-tensors INT4 to the engine layout
    (vllm_xiaotu_moe/mixed_experts.py:3394-3418): weights int32 [E, K/8, N]
    (eight nibbles per int32 along K, the lowest nibble the first k) become
    uint8 [E, N, K/2] (low nibble = even k), scales [E, K/group, N] become
    fp32 [E, N, K/group].  Weights already uint8 [E, N, K/2] pass through with
    their scales [E, N, K/group]."""
    w = w.data if isinstance(w, torch.nn.Parameter) else w
    s = s.data if isinstance(s, torch.nn.Parameter) else s
    if w.dtype == torch.int32:
        w = w.detach().to("cpu").transpose(1, 2).contiguous().view(torch.uint8)
        s = s.detach().to("cpu").transpose(1, 2)
    elif w.dtype != torch.uint8:
        raise NotImplementedError(f"INT4 experts take int32 (GPTQ / compressed-tensors) or uint8 "
                                  f"(engine layout) weights, got {w.dtype}")
    return w.detach().to("cpu").contiguous(), s.detach().to("cpu").to(torch.float32).contiguous()


def require_symmetric_zero_points(layer, names) -> None:
    """Refuse asymmetric int4: the engine's value is code - 8, which is
    symmetric quantisation (effective zero point 8).  GPTQ packs zero points
    minus one in int32 (so a symmetric checkpoint holds 7s); compressed-tensors
    may hold 8 directly; either is accepted (mixed_experts.py:3420-3452)."""
    for name in names:
        qz = getattr(layer, name, None)
        if qz is None:
            continue
        b = (qz.data if isinstance(qz, torch.nn.Parameter) else qz).detach().to("cpu").contiguous()
        packed = b.dtype in (torch.int32, torch.int16)
        u8 = b.view(torch.uint8) if b.dtype != torch.uint8 else b
        nib = torch.cat(((u8 & 15).reshape(-1), (u8 >> 4).reshape(-1))).to(torch.int16)
        if packed:
            nib = nib + 1
        vals = torch.unique(nib)
        if not bool(torch.all((vals == 7) | (vals == 8))):
            raise NotImplementedError(
                f"INT4 experts implement symmetric quantisation only (zero point 8); {name} "
                f"holds zero points {sorted(int(v) for v in vals.tolist())[:8]}")


class XiaotuExpertsInt4(XiaotuExperts):
    """INT4 W4A16 group-quantised experts (WNA16): the reference's
    XiaotuCPUExpertsInt4 / MOE_WNA16 (vllm_xiaotu_moe/mixed_experts.py:
    3363-3476).  The checkpoint is repacked once at load (GPTQ /
    compressed-tensors int32 -> engine bytes, scales transposed), symmetric
    zero points and sequential K order (no desc_act) are required, and the
    experts run where the reference runs them, on the host engine: through
    the graph-capturable cpu_decode bridge for device tensors (batches up to
    the pre-sized staging, XTU_CD_PREALLOC_TOKENS, default 512), synchronously
    beyond it, directly for host tensors."""

    _fmt = F.FMT_INT4
    _scale_attrs = (("w13_scales", "w13_weight_scale"), ("w2_scales", "w2_weight_scale"))
    _w_names = (("w13_qweight", "w13_weight_packed", "w13_weight"),
                ("w2_qweight", "w2_weight_packed", "w2_weight"))
    _z_names = ("w13_qzeros", "w13_weight_zero_point", "w2_qzeros", "w2_weight_zero_point")
    _group_n, _group_k = 1, 128
    _monolithic = False

    def __init__(self, moe_config=None, quant_config=None):
        super().__init__(moe_config, quant_config)
        self._host = None

    @classmethod
    def _find_any(cls, layer, names):
        for n in names:
            t = cls._find(layer, n)
            if t is not None:
                return t
        return None

    def process_weights_after_loading(self, layer) -> None:
        from .cpu_experts import CpuExperts
        from .host_store import HostExpertStore
        import os
        self._read_layer_attrs(layer)
        w13 = self._find_any(layer, self._w_names[0])
        w2 = self._find_any(layer, self._w_names[1])
        if w13 is None or w2 is None:
            raise NotImplementedError("INT4 experts found no int4 weight tensors on the layer "
                                      f"(looked for {self._w_names[0]} / {self._w_names[1]})")
        if bool(getattr(self.quant_config, "desc_act", False)):
            raise NotImplementedError("INT4 experts assume sequential K order (GPTQ desc_act / "
                                      "g_idx reordering is not supported)")
        group = int(getattr(self.quant_config, "group_size", 0) or 0) or 128
        if w13.dtype == torch.int32:
            require_symmetric_zero_points(layer, self._z_names)
        s13 = self._find_any(layer, self._scale_attrs[0])
        s2 = self._find_any(layer, self._scale_attrs[1])
        if s13 is None or s2 is None:
            raise NotImplementedError("INT4 experts found no group scales on the layer")
        w13, s13 = repack_gptq_int4(w13, s13)
        w2, s2 = repack_gptq_int4(w2, s2)
        ok = (w13.dim() == 3 and w2.dim() == 3 and w13.shape[2] * 2 == w2.shape[1]
              and w2.shape[2] * 2 == w13.shape[1] // 2)
        if not ok:
            raise NotImplementedError(
                f"INT4 experts cannot take w13 {tuple(w13.shape)} / w2 {tuple(w2.shape)}: "
                "expected the byte-packed [E, 2I, H/2] / [E, H, I/2] layout (AWQ's N-packed "
                "layout is not supported)")
        H, I = int(w2.shape[1]), int(w13.shape[1]) // 2
        if s13.shape[-1] * group != H or s2.shape[-1] * group != I:
            raise ValueError(f"INT4 scales {tuple(s13.shape)} / {tuple(s2.shape)} do not match "
                             f"group_size {group} for H={H}, I={I}")
        self._weights = ExpertWeights.from_dense(F.FMT_INT4, w13, s13, w2, s2, device="cpu")
        gpu = torch.cuda.is_available()
        store = HostExpertStore.from_weights(self._weights, pin=gpu)
        pre = int(os.environ.get("XTU_CD_PREALLOC_TOKENS", "512") or 512) if gpu else 0
        self._host = CpuExperts.from_store(
            store, swiglu_limit=float(self.swiglu_limit or 0.0),
            swiglu_alpha=float(self.swiglu_alpha if self.swiglu_alpha is not None else 1.0),
            swiglu_beta=float(self.swiglu_beta or 0.0), max_tokens=pre,
            max_topk=max(int(self.top_k or 1), 1))
        self._store = store

    def _experts(self, x, ids, wts, kw):
        eng = self._host
        T, K = ids.shape
        odt, out = kw.get("out_dtype", torch.float32), kw.get("out")
        if not x.is_cuda:
            res = eng.forward(x, ids.cpu(), wts.cpu())
        elif T <= eng.max_tokens and K <= eng.max_topk:
            res = _scratch("int4_out", (T, eng.H), torch.float32, x.device)
            rc = eng.cpu_decode(torch.cuda.current_stream(x.device).cuda_stream, T, K, x,
                                ids.to(torch.int32).contiguous(),
                                wts.to(torch.float32).contiguous(), res)
            if rc:
                raise RuntimeError(f"INT4 host engine refused the batch (cpu_decode {rc})")
        else:   # beyond the staging: a synchronous host forward (not capturable)
            torch.cuda.current_stream(x.device).synchronize()
            res = eng.forward(x.cpu(), ids.cpu(), wts.cpu()).to(x.device)
        if out is not None:
            out.copy_(res)
            return out
        # the device result sits in a reused buffer: hand out a copy
        return res.to(odt, copy=True) if x.is_cuda else res.to(odt)
