"""Seeded synthetic layers for the tests: packed experts, router weights, activations."""
from __future__ import annotations

from dataclasses import dataclass, replace

import numpy as np

from bigrig_amd import formats as F
from bigrig_amd.spec import LayerSpec


@dataclass
class Layer:
    spec: LayerSpec
    experts: list           # packed bytes per expert id
    router: np.ndarray      # [E, H] float32 or bf16 bits
    bias: np.ndarray | None  # [E] float32 or None
    shared: bytes | None
    sgate_w: np.ndarray | None  # [H] bf16 bits


def make_layer(spec: LayerSpec, seed: int = 0, bank: int | None = None, zipf: float = 0.0,
               router_std: float = 0.02, expert_std: float = 0.02) -> Layer:
    """Experts N(0, expert_std) quantized to spec.quant. With `bank`, only that many distinct
    experts are quantized and expert e reuses bank entry (e * 7 + seed) % bank (different
    neighbours, so a wrong slot still reads different bytes)."""
    rng = np.random.default_rng(seed)
    nq = spec.n_experts if bank is None else min(bank, spec.n_experts)
    made = [F.make_expert(rng, spec.hidden, spec.inter, spec.quant, std=expert_std,
                          has_bias=spec.has_bias, gated=spec.gated) for _ in range(nq)]
    if bank is None:
        experts = made
    else:
        experts = [made[(e * 7 + seed) % nq] for e in range(spec.n_experts)]
    wr = (rng.standard_normal((spec.n_experts, spec.hidden), dtype=np.float32) * router_std)
    router = wr if spec.router_dtype == "float32" else F.f32_to_bf16_bits(wr)
    bias = zipf_bias(spec.n_experts, zipf, rng) if zipf else None
    shared = sgw = None
    if spec.shared_inter:
        shared = F.make_expert(rng, spec.hidden, spec.shared_inter, spec.quant, std=expert_std,
                               has_bias=spec.has_bias, gated=spec.gated)
        sgw = F.f32_to_bf16_bits(rng.standard_normal(spec.hidden, dtype=np.float32) * router_std)
    return Layer(spec, experts, router, bias, shared, sgw)


def zipf_bias(E: int, s: float, rng: np.random.Generator) -> np.ndarray:
    """Per-expert logit bias -s * ln(rank + 1) over a seeded permutation of the experts, so the
    router's choices follow a Zipf(s)-like popularity."""
    perm = rng.permutation(E)
    return (-s * np.log(perm.astype(np.float64) + 1.0)).astype(np.float32)


def make_x(T: int, H: int, seed: int = 1, std: float = 1.0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return F.f32_to_bf16_bits(rng.standard_normal((T, H), dtype=np.float32) * std)


def small(spec: LayerSpec, **kw) -> LayerSpec:
    return replace(spec, **kw)
