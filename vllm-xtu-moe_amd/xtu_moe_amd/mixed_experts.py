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
1x32, FP8 128x128 (and NVFP4 1x16 with per-expert global scales).

Here the experts run on the HIP library with the layer's weights packed once
into the device layout; vLLM itself is not needed (an ``activation`` of
None or a string name is accepted when vLLM's enum is absent).
"""
from __future__ import annotations

import enum

import torch

from . import formats as F
from .layer import ExpertWeights, _buf as _scratch, moe_forward, route

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
        w13, w2 = layer.w13_weight, layer.w2_weight
        s13 = self._find(layer, self._scale_attrs[0])
        s2 = self._find(layer, self._scale_attrs[1])
        g13 = self._find(layer, self._global_scale_attrs[0])
        g2 = self._find(layer, self._global_scale_attrs[1])
        dev = torch.device("cuda") if not w13.is_cuda else w13.device
        self._weights = ExpertWeights.from_dense(self._fmt, self._weight_view(w13), s13,
                                                 self._weight_view(w2), s2, g13, g2, device=dev)

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
        if self._weights is None:
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
        direct = (output is not None and output.dtype == odt and output.is_contiguous()
                  and tuple(output.shape) == (T, self._weights.H) and output.device == x.device)
        kw = dict(swiglu_limit=float(self.swiglu_limit or 0.0),
                  swiglu_alpha=float(self.swiglu_alpha if self.swiglu_alpha is not None else 1.0),
                  swiglu_beta=float(self.swiglu_beta or 0.0),
                  out=output if direct else None, out_dtype=odt)
        if topk_weights is not None and topk_ids is not None:
            res = moe_forward(x, topk_ids.to(torch.int32).contiguous(),
                              topk_weights.to(torch.float32).contiguous(), self._weights, **kw)
        elif (expert_map is None and self.custom_routing_function is None
              and router_logits is not None):
            # monolithic path: routing (+ segmentation, + the shared experts'
            # gate/up at decode sizes) inside the layer's own launches
            ids = _scratch("hook_ids", (T, int(self.top_k)), torch.int32, x.device)
            wts = _scratch("hook_wts", (T, int(self.top_k)), torch.float32, x.device)
            res = moe_forward(x, ids, wts, self._weights, router=self._router_args(router_logits),
                              **kw)
        else:
            topk_weights, topk_ids = self._select_topk(hidden_states, router_logits)
            if expert_map is not None:
                topk_ids, topk_weights = self._local_ids(expert_map, topk_ids, topk_weights)
            res = moe_forward(x, topk_ids.contiguous(), topk_weights.contiguous(), self._weights,
                              **kw)
        if direct:
            return output
        res = res.to(hidden_states.dtype)
        if output is not None:
            output.copy_(res)
            return output
        return res

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
