"""Synthetic MLX-style checkpoints for the checkpoint-reader tests: stacked expert tensors
(E, ...) per layer and projection component, in safetensors shards, with a config.json."""
from __future__ import annotations

import json
import os
import struct

import numpy as np

from bigrig_amd import formats as F

_ST = {"uint32": "U32", "uint8": "U8", "bfloat16": "BF16", "float16": "F16", "float32": "F32"}


def write_safetensors(path: str, tensors: dict, metadata: dict | None = None) -> None:
    """tensors: {name: (safetensors dtype, shape, raw bytes)}, written in name order."""
    hdr, pos, blobs = {}, 0, []
    if metadata:
        hdr["__metadata__"] = metadata
    for name in sorted(tensors):
        dt, shape, raw = tensors[name]
        hdr[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [pos, pos + len(raw)]}
        blobs.append(raw)
        pos += len(raw)
    body = json.dumps(hdr).encode()
    body += b" " * (-len(body) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(body)))
        f.write(body)
        for b in blobs:
            f.write(b)


def make_checkpoint(d: str, layers: dict, *, infix: str = ".mlp.switch_mlp.", shards: int = 2,
                    config: dict | None = None, seed: int = 0, extra: bool = True) -> dict:
    """Write a checkpoint whose layer li has the experts of layers[li] = (hidden, inter,
    n_experts, QuantSpec, has_bias[, gated]) (gated False: fc1/fc2 experts). Returns {li: (expert spec, quant, [expert bytes])} -- the
    argument formats.pack_blob takes -- so a test can pack the same experts into a blob."""
    os.makedirs(d, exist_ok=True)
    rng = np.random.default_rng(seed)
    out = {}
    files = [dict() for _ in range(shards)]
    for n, li in enumerate(sorted(layers)):
        H, I, E, q, has_bias, *rest = layers[li]
        gated = rest[0] if rest else True
        spec = F.expert_spec(H, I, q, has_bias, gated)
        experts = [F.make_expert(rng, H, I, q, has_bias=has_bias, gated=gated) for _ in range(E)]
        out[li] = (spec, q, experts)
        parts = [F.split_expert(b, spec) for b in experts]
        tens = files[n % shards]
        for proj in spec:
            for comp, m in spec[proj].items():
                stack = np.stack([p[(proj, comp)] for p in parts])
                tens[f"model.layers.{li}{infix}{proj}.{comp}"] = (
                    _ST[m["dtype"]], (E, *m["shape"]), stack.tobytes())
        if extra:   # non-expert tensors the reader must ignore
            tens[f"model.layers.{li}.self_attn.q_proj.weight"] = ("BF16", (4, 8), bytes(64))
            tens[f"model.layers.{li}.mlp.shared_experts.gate_proj.weight"] = ("U32", (4, 2), bytes(32))
    for i, tens in enumerate(files):
        if tens:
            write_safetensors(os.path.join(d, f"model-{i:05d}-of-{shards:05d}.safetensors"), tens,
                              {"format": "mlx"})
    cfg = {"model_type": "qwen3_moe", "num_experts_per_tok": 2, "norm_topk_prob": True,
           "quantization": {"group_size": 64, "bits": 4}}
    if config is not None:
        cfg = config
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(cfg, f)
    return out
