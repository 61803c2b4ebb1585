"""One MoE layer's shape, quantization and routing rule, and the C descriptor built from it."""
from __future__ import annotations

import functools
from dataclasses import dataclass, field

from . import formats as F

_ROUTES = {"softmax_topk": 0, "softmax_topk_renorm": 1, "topk_softmax": 2, "sigmoid_topk": 3,
           "sigmoid_topk_renorm": 4}
_ACTS = {"swiglu": 0, "swiglu_clamped": 1, "silu_mlp": 2}
_RDT = {"float32": 0, "bfloat16": 1}
_QMODES = {"affine": 0, "mxfp4": 1, "none": 2}   # BRX_QUANT_*
MAX_WIDTH = 8192   # largest hidden / intermediate width libbrx takes


@dataclass(frozen=True)
class LayerSpec:
    """A routed-expert layer.

    route: how the block turns logits into (indices, weights) -- the rule adapter.py:75-93
    records per model: "softmax_topk" (OLMoE: w = softmax(logits)[idx]),
    "softmax_topk_renorm" (Qwen3 norm_topk_prob: then w /= sum(w)), "topk_softmax"
    (gpt-oss: w = softmax(logits[idx])), "sigmoid_topk" / "sigmoid_topk_renorm" (DeepSeek-V3-style
    scoring: select on sigmoid(logits) + the router bias, weigh sigmoid(logits)[idx], optionally
    renormalised). n_group > 1 makes the selection group-limited (the topk_group best of
    n_group contiguous expert groups stay eligible); route_scale multiplies every weight
    (routed_scaling_factor).
    act: "swiglu" = silu(gate) * up; "swiglu_clamped" = gpt-oss's clamped form with
    alpha/limit; "silu_mlp" = a plain two-layer expert fc2(silu(fc1 x)) (SwitchMLP,
    stream.py:1167-1169).
    """
    hidden: int
    inter: int
    n_experts: int
    top_k: int
    quant: F.QuantSpec = field(default_factory=F.QuantSpec)
    has_bias: bool = False
    act: str = "swiglu"
    alpha: float = 1.702
    limit: float = 7.0
    route: str = "softmax_topk_renorm"
    router_dtype: str = "bfloat16"
    shared_inter: int = 0
    n_group: int = 0
    topk_group: int = 0
    route_scale: float = 1.0

    def __post_init__(self):
        if self.route not in _ROUTES:
            raise ValueError(f"route {self.route!r} not in {sorted(_ROUTES)}")
        if self.act not in _ACTS:
            raise ValueError(f"act {self.act!r} not in {sorted(_ACTS)}")
        if self.router_dtype not in _RDT:
            raise ValueError(f"router_dtype {self.router_dtype!r} not in {sorted(_RDT)}")
        if not 1 <= self.top_k <= self.n_experts:
            raise ValueError(f"top_k {self.top_k} outside [1, {self.n_experts}]")
        if self.n_group > 1:
            G = self.n_experts // self.n_group if self.n_group <= 64 else 0
            if (not G or self.n_experts % self.n_group or
                    not 1 <= self.topk_group <= self.n_group or self.top_k > self.topk_group * G):
                raise ValueError(f"group-limited routing needs n_group <= 64 dividing n_experts, "
                                 f"1 <= topk_group <= n_group and top_k <= topk_group * group size "
                                 f"(n_group {self.n_group}, topk_group {self.topk_group})")
        if not self.route_scale > 0:
            raise ValueError(f"route_scale {self.route_scale} must be positive")
        for name in ("hidden", "inter", "shared_inter"):
            v = getattr(self, name)
            if v % 64 or v > MAX_WIDTH or (v <= 0 and name != "shared_inter") or v < 0:
                raise ValueError(f"{name} {v} must be a multiple of 64 in "
                                 f"[{0 if name == 'shared_inter' else 64}, {MAX_WIDTH}]")

    @property
    def route_mode(self) -> int:
        return _ROUTES[self.route]

    @property
    def route_rule(self) -> dict:
        """The oracle router's keyword arguments for this layer's rule beyond its mode."""
        return {"n_group": self.n_group, "topk_group": self.topk_group, "scale": self.route_scale}

    @property
    def gated(self) -> bool:
        """Gated experts (gate/up/down) unless the activation is the plain two-layer fc1/fc2."""
        return self.act != "silu_mlp"

    def expert_spec(self, shared: bool = False) -> dict:
        inter = self.shared_inter if shared else self.inter
        return F.expert_spec(self.hidden, inter, self.quant, self.has_bias, self.gated)

    @functools.cached_property
    def bytes_per_expert(self) -> int:
        """Packed bytes of one routed expert (computed once: it is read per admission)."""
        return F.spec_bytes(self.expert_spec())

    @property
    def router_bytes(self) -> int:
        return self.n_experts * self.hidden * (4 if self.router_dtype == "float32" else 2)

    def desc(self):
        from .lib import LayerDesc
        q = self.quant
        return LayerDesc(self.hidden, self.inter, self.n_experts, self.top_k,
                         _QMODES[q.mode], q.bits, q.group_size,
                         1 if q.scale_dtype == "float16" else 0, int(self.has_bias),
                         _ACTS[self.act], self.alpha, self.limit, self.route_mode,
                         _RDT[self.router_dtype], self.shared_inter, self.n_group,
                         self.topk_group, self.route_scale)


# The synthetic layer shapes the benchmarks and parity tests run (hidden, experts, top-k,
# intermediate, routing rule, quantization).
OLMOE_1B_7B = LayerSpec(2048, 1024, 64, 8, route="softmax_topk", router_dtype="float32")
QWEN3_30B_A3B = LayerSpec(2048, 768, 128, 8, route="softmax_topk_renorm")
# the layout of the shipped Qwen3-30B-A3B-3bit blob (3-bit affine, group 64, bf16 scale + bias:
# data/blobs/Qwen3-30B-A3B-3bit.experts.manifest.json, 2,064,384 bytes per expert)
QWEN3_30B_A3B_3BIT = LayerSpec(2048, 768, 128, 8, route="softmax_topk_renorm",
                               quant=F.QuantSpec(3, 64, "affine", "bfloat16"))
# unquantized bf16 experts (Qwen3-30B-A3B-bf16, the checkpoint the reference's reader names for
# the no-quant case, direct.py:110-142): 9,437,184 bytes per expert
QWEN3_30B_A3B_BF16 = LayerSpec(2048, 768, 128, 8, route="softmax_topk_renorm",
                               quant=F.QuantSpec(16, 0, "none"))
E256_SHARED = LayerSpec(2048, 512, 256, 8, route="softmax_topk_renorm", shared_inter=512)
GPT_OSS_120B = LayerSpec(2880, 2880, 128, 4, quant=F.QuantSpec(4, 32, "mxfp4"), has_bias=True,
                         act="swiglu_clamped", route="topk_softmax")
