"""Routed experts read straight out of an MLX checkpoint's safetensors shards.

A stacked expert tensor of shape (E, ...) stores expert e's slice contiguously at a computable
offset of its file, so an expert's bytes need no second copy on disk: expert e of a layer is
the concatenation, projection outer and component inner, of slice e of each of its component
tensors -- exactly the bytes a packed blob region holds for it (the reference's direct reader,
bigrig_engine/direct.py:145-240, and its invariant, tests/test_direct.py:39-83). This module
builds that description (`expert_manifest`), reads experts from it (`read_expert`), derives the
layer's shape (`layer_spec`) and the routing rule from config.json (`routing_from_config`);
`pool.HostStore.from_checkpoint` fills the pinned host store with it.

The safetensors format (8-byte little-endian header length, a JSON header mapping tensor names
to dtype, shape and data offsets relative to the end of the header, then the data) is read here
with its bounds checked before any byte is trusted.
"""
from __future__ import annotations

import glob
import json
import os
import struct
from dataclasses import dataclass, field

from . import formats as F

# Where MoE families put their stacked expert tensors (a naming convention, not a property of
# the bytes; direct.py:43-45). `shared_experts` paths are not routed and are not listed.
EXPERT_INFIXES = (".mlp.switch_mlp.", ".mlp.experts.", ".feed_forward.experts.",
                  ".ffn.switch_mlp.", ".ffn.experts.", ".mixer.switch_mlp.",
                  ".block_sparse_moe.switch_mlp.", ".block_sparse_moe.experts.")

# the two-layer MLP expert layout some families use; these kernels compute SwiGLU experts only
MLP_PROJECTIONS = ("fc1", "fc2")

# safetensors dtype -> (dtype name in the expert spec, bytes per element)
ST_DTYPES = {"F64": ("float64", 8), "F32": ("float32", 4), "F16": ("float16", 2),
             "BF16": ("bfloat16", 2), "I64": ("int64", 8), "I32": ("int32", 4),
             "I16": ("int16", 2), "I8": ("int8", 1), "U8": ("uint8", 1), "U32": ("uint32", 4),
             "U16": ("uint16", 2), "BOOL": ("bool_", 1)}

_MAX_HEADER = 1 << 30


@dataclass(frozen=True)
class Tensor:
    """One tensor of a shard: its file, absolute byte offset and length, dtype and shape."""
    path: str
    offset: int
    nbytes: int
    dtype: str
    shape: tuple


def read_header(path: str) -> tuple:
    """(header dict, absolute offset of the data section) of one safetensors file."""
    with open(path, "rb") as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise ValueError(f"{path} is too short to be a safetensors file")
        n = struct.unpack("<Q", raw)[0]
        if not 0 < n < _MAX_HEADER:
            raise ValueError(f"{path}: implausible safetensors header length {n}")
        body = f.read(n)
    if len(body) != n:
        raise ValueError(f"{path}: header of {n} bytes is cut short at {len(body)}")
    hdr = json.loads(body)
    if not isinstance(hdr, dict):
        raise ValueError(f"{path}: safetensors header is not an object")
    return hdr, 8 + n


def scan(model_dir: str) -> dict:
    """{tensor name: Tensor} over every `*.safetensors` shard of a model directory."""
    d = os.path.expanduser(model_dir)
    files = sorted(glob.glob(os.path.join(d, "*.safetensors")))
    if not files:
        raise FileNotFoundError(f"no safetensors in {d}")
    out = {}
    for p in files:
        hdr, base = read_header(p)
        size = os.path.getsize(p)
        for name, ent in hdr.items():
            if name == "__metadata__":
                continue
            a, b = (int(v) for v in ent["data_offsets"])
            if b < a or base + b > size:
                raise ValueError(f"{p}: tensor {name} claims bytes {a}..{b}, which runs past the "
                                 f"file ({size} bytes). Refusing to read past the end.")
            if ent["dtype"] not in ST_DTYPES:
                raise ValueError(f"{p}: tensor {name} has unknown dtype {ent['dtype']}")
            out[name] = Tensor(p, base + a, b - a, ent["dtype"], tuple(int(x) for x in ent["shape"]))
    return out


def quant_for(cfg: dict, module_path: str, spec: dict | None = None) -> dict:
    """A layer's {bits, group_size, mode}, or {} for unquantized weights.

    The tensors decide first: a layer with no `scales` component is not quantized whatever
    config.json says. Then a per-module entry of the config's quantization block, then its
    global bits / group size (direct.py:110-142)."""
    if spec is not None and not any("scales" in comps for comps in spec.values()):
        return {}
    q = cfg.get("quantization") or cfg.get("quantization_config") or {}
    if not q:
        return {}
    v = q.get(module_path)
    if isinstance(v, dict):
        return {"bits": int(v["bits"]), "group_size": int(v["group_size"]),
                "mode": v.get("mode", "affine")}
    return {"bits": int(q.get("bits", 4)), "group_size": int(q.get("group_size", 64)),
            "mode": q.get("mode", "affine")}


@dataclass
class CheckpointManifest:
    """A blob manifest's description of every expert, pointing into the checkpoint's files:
    per layer {n_experts, spec, bytes_per_expert, quant} as a packed blob's manifest records it,
    and per expert "L:e" the (path, offset, length) segments that concatenate to its bytes."""
    model_dir: str
    layers: dict = field(default_factory=dict)
    segments: dict = field(default_factory=dict)
    total_bytes: int = 0
    top_k: int | None = None
    config: dict = field(default_factory=dict)
    version: int = 4

    def expert_segments(self, layer: int, expert: int) -> list:
        key = f"{layer}:{expert}"
        if key not in self.segments:
            raise KeyError((layer, expert))
        return self.segments[key]

    def quant(self, layer) -> F.QuantSpec:
        """The layer's QuantSpec (scale dtype from its spec), as formats.Manifest.quant."""
        return F.Manifest(layers=self.layers).quant(layer)


def expert_manifest(model_dir: str) -> CheckpointManifest:
    """Describe every routed expert of an MLX checkpoint by where its bytes already sit."""
    d = os.path.expanduser(model_dir)
    tensors = scan(d)
    with open(os.path.join(d, "config.json")) as f:
        cfg = json.load(f)
    layers, found_infix, foreign = {}, None, set()
    for name in tensors:
        for infix in EXPERT_INFIXES:
            if infix in name:
                break
        else:
            continue
        head, tail = name.split(infix, 1)
        li = int(head.rsplit(".", 1)[1])
        proj, comp = tail.rsplit(".", 1)
        if proj not in F.PROJECTIONS:
            foreign.add(proj)
            continue
        if comp not in F.COMPONENTS:
            continue
        found_infix = infix
        layers.setdefault(li, {}).setdefault(proj, {})[comp] = name
    if not layers:
        if foreign:
            kind = "a two-layer MLP (fc1/fc2)" if foreign <= set(MLP_PROJECTIONS) else "a"
            raise ValueError(f"{d} is a mixture-of-experts model, but its experts use {kind} "
                             f"{'/'.join(sorted(foreign))} layout; these kernels compute "
                             f"gate/up/down (SwiGLU) experts")
        raise ValueError(f"{d} has no MoE expert tensors (looked for "
                         f"{', '.join('*' + i + '*' for i in EXPERT_INFIXES)})")

    man = CheckpointManifest(model_dir=d, config=cfg)
    tk = cfg.get("num_experts_per_tok") or cfg.get("moe_topk")
    if isinstance(tk, int) and tk > 0:
        man.top_k = tk
    total = 0
    for li in sorted(layers):
        spec, n_experts, per_expert, ordered = {}, None, 0, []
        for proj in F.PROJECTIONS:          # projection outer, component inner: packing order
            comps = layers[li].get(proj)
            if not comps:
                raise ValueError(f"layer {li} is missing {proj}; the checkpoint is incomplete")
            spec[proj] = {}
            for comp in F.COMPONENTS:
                nm = comps.get(comp)
                if nm is None:
                    continue
                t = tensors[nm]
                if len(t.shape) < 2:
                    raise ValueError(f"{nm} has shape {t.shape}; stacked expert tensors lead with E")
                if n_experts is None:
                    n_experts = t.shape[0]
                elif t.shape[0] != n_experts:
                    raise ValueError(f"layer {li}: {nm} has {t.shape[0]} experts but a sibling "
                                     f"has {n_experts}. Refusing to guess which is right.")
                dt, isize = ST_DTYPES[t.dtype]
                stride = isize
                for x in t.shape[1:]:
                    stride *= x
                if stride * n_experts != t.nbytes:
                    raise ValueError(f"{nm}: {n_experts} x {stride} != {t.nbytes} bytes on disk. "
                                     f"The header and the data disagree.")
                spec[proj][comp] = {"shape": list(t.shape[1:]), "dtype": dt, "nbytes": stride}
                ordered.append((t.path, t.offset, stride))
                per_expert += stride
        for e in range(n_experts):
            man.segments[f"{li}:{e}"] = [(p, o + e * s, s) for p, o, s in ordered]
        man.layers[str(li)] = {
            "n_experts": n_experts, "spec": spec, "bytes_per_expert": per_expert,
            "quant": quant_for(cfg, f"model.layers.{li}{found_infix}gate_proj", spec)}
        total += per_expert * n_experts
    man.total_bytes = total
    return man


def read_expert_into(man: CheckpointManifest, layer: int, expert: int, out, fds: dict) -> int:
    """Read expert `expert` of `layer` into the writable buffer `out` (its segments in order);
    `fds` caches open file descriptors by path. Returns the bytes read."""
    mv = memoryview(out).cast("B")
    pos = 0
    for path, off, n in man.expert_segments(layer, expert):
        fd = fds.get(path)
        if fd is None:
            fd = fds[path] = os.open(path, os.O_RDONLY)
        got = 0
        while got < n:
            r = os.preadv(fd, [mv[pos + got:pos + n]], off + got)
            if r <= 0:
                raise OSError(f"{path}: short read at {off + got} ({got} of {n} bytes)")
            got += r
        pos += n
    return pos


def read_expert(man: CheckpointManifest, layer: int, expert: int) -> bytes:
    """Expert `expert` of `layer` as one bytes object, in packed-blob order."""
    buf = bytearray(int(man.layers[str(layer)]["bytes_per_expert"]))
    fds = {}
    try:
        read_expert_into(man, layer, expert, buf, fds)
    finally:
        for fd in fds.values():
            os.close(fd)
    return bytes(buf)


def routing_from_config(cfg: dict) -> dict:
    """The block's routing rule and activation as LayerSpec fields, from config.json: softmax
    top-k, renormalised when `norm_topk_prob` is set (adapter.py:75-93); gpt-oss applies the
    softmax to the top-k logits and a clamped SwiGLU (`swiglu_limit`)."""
    mt = str(cfg.get("model_type", "")).lower()
    fn = str(cfg.get("score_function") or cfg.get("scoring_func") or "softmax").lower()
    if "sigmoid" in fn or cfg.get("n_group") or cfg.get("topk_group"):
        raise ValueError("sigmoid / group-limited routing is not a rule these kernels implement")
    if mt == "gpt_oss":
        return {"route": "topk_softmax", "act": "swiglu_clamped",
                "limit": float(cfg.get("swiglu_limit", 7.0))}
    return {"route": "softmax_topk_renorm" if cfg.get("norm_topk_prob") else "softmax_topk",
            "act": "swiglu"}


def layer_spec(man: CheckpointManifest, layer: int, **overrides):
    """The LayerSpec of one checkpoint layer: shapes from its expert tensors, quantization from
    the manifest, top-k and routing from config.json (any field can be overridden)."""
    from .spec import LayerSpec
    e = man.layers[str(layer)]
    q = man.quant(layer)
    gate = e["spec"]["gate_proj"]
    inter = int(gate["weight"]["shape"][0])
    hidden = int(gate["weight"]["shape"][1]) * 32 // q.bits
    kw = {"hidden": hidden, "inter": inter, "n_experts": int(e["n_experts"]),
          "top_k": int(man.top_k or 1), "quant": q, "has_bias": "bias" in gate}
    kw.update(routing_from_config(man.config))
    kw.update(overrides)
    spec = LayerSpec(**kw)
    if F.spec_bytes(spec.expert_spec()) != int(e["bytes_per_expert"]):
        raise ValueError(f"layer {layer}: the derived shape accounts for "
                         f"{F.spec_bytes(spec.expert_spec())} bytes per expert, the checkpoint "
                         f"holds {e['bytes_per_expert']}")
    return spec
