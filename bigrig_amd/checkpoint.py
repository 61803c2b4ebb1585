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
import re
import struct
from dataclasses import dataclass, field

import numpy as np

from . import formats as F

# Where MoE families put their stacked expert tensors (a naming convention, not a property of
# the bytes; direct.py:43-45). `shared_experts` paths are not routed and are not listed.
EXPERT_INFIXES = (".mlp.switch_mlp.", ".mlp.experts.", ".feed_forward.experts.",
                  ".ffn.switch_mlp.", ".ffn.experts.", ".mixer.switch_mlp.",
                  ".block_sparse_moe.switch_mlp.", ".block_sparse_moe.experts.")

# the two-layer MLP expert layout some families use (fc2(silu(fc1 x)), stream.py:57, 1167-1169)
MLP_PROJECTIONS = F.MLP_PROJECTIONS

# safetensors dtype -> (dtype name in the expert spec, bytes per element)
ST_DTYPES = {"F64": ("float64", 8), "F32": ("float32", 4), "F16": ("float16", 2),
             "BF16": ("bfloat16", 2), "I64": ("int64", 8), "I32": ("int32", 4),
             "I16": ("int16", 2), "I8": ("int8", 1), "U8": ("uint8", 1), "U32": ("uint32", 4),
             "U16": ("uint16", 2), "BOOL": ("bool_", 1)}

_MAX_HEADER = 1 << 30

# <anything>.<layer index><one of the infixes><projection>.<component>
_EXPERT_NAME = re.compile(
    r"^.*\.(?P<layer>\d+)(?P<infix>" + "|".join(re.escape(i) for i in EXPERT_INFIXES) +
    r")(?P<proj>[A-Za-z0-9_]+)\.(?P<comp>[A-Za-z0-9_]+)$")


@dataclass(frozen=True)
class Tensor:
    """One tensor of a shard: its file, absolute byte offset and length, dtype and shape."""
    path: str
    offset: int
    nbytes: int
    dtype: str
    shape: tuple


def read_header(path: str) -> tuple:
    """(header dict, absolute offset of the data section) of one safetensors file: a
    little-endian u64 header length, then that many bytes of JSON object."""
    with open(path, "rb") as f:
        prefix = f.read(8)
        if len(prefix) < 8:
            raise ValueError(f"{path} is too short to be a safetensors file ({len(prefix)} bytes)")
        (hlen,) = struct.unpack("<Q", prefix)
        if hlen == 0 or hlen >= _MAX_HEADER:
            raise ValueError(f"{path}: implausible safetensors header length {hlen}")
        text = f.read(hlen)
    if len(text) < hlen:
        raise ValueError(f"{path}: the {hlen}-byte header is cut short at {len(text)} bytes")
    header = json.loads(text)
    if type(header) is not dict:
        raise ValueError(f"{path}: the safetensors header is not an object")
    return header, 8 + hlen


def _shard_tensors(path: str) -> dict:
    """{name: Tensor} of one shard, every entry's dtype and byte range checked against the
    file before it is trusted."""
    header, start = read_header(path)
    end = os.path.getsize(path)
    found = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        lo, hi = (int(v) for v in meta["data_offsets"])
        if not 0 <= lo <= hi or start + hi > end:
            raise ValueError(f"{path}: tensor {name} claims bytes {lo}..{hi}, which runs past the "
                             f"file ({end} bytes); nothing is read past the end")
        dt = meta["dtype"]
        if dt not in ST_DTYPES:
            raise ValueError(f"{path}: tensor {name} has unknown dtype {dt}")
        found[name] = Tensor(path, start + lo, hi - lo, dt, tuple(int(x) for x in meta["shape"]))
    return found


def scan(model_dir: str) -> dict:
    """{tensor name: Tensor} over every `*.safetensors` shard of a model directory."""
    root = os.path.expanduser(model_dir)
    shards = sorted(glob.glob(os.path.join(root, "*.safetensors")))
    if not shards:
        raise FileNotFoundError(f"no safetensors in {root}")
    index = {}
    for path in shards:
        index.update(_shard_tensors(path))
    return index


def quant_for(cfg: dict, module_path: str, spec: dict | None = None) -> dict:
    """A layer's {bits, group_size, mode}, or {} for unquantized weights (direct.py:110-142):
    weights without `scales` are unquantized whatever config.json says; otherwise the entry for
    the module in the config's quantization block, else the block's global bits / group size."""
    if spec is not None and all("scales" not in comps for comps in spec.values()):
        return {}
    block = cfg.get("quantization") or cfg.get("quantization_config") or {}
    if not block:
        return {}
    src = block[module_path] if isinstance(block.get(module_path), dict) else block
    return {"bits": int(src.get("bits", 4)), "group_size": int(src.get("group_size", 64)),
            "mode": src.get("mode", "affine")}


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


def _expert_tensors(tensors: dict):
    """{layer: {projection: {component: name}}} of the stacked routed-expert tensors (gated
    gate/up/down or two-layer fc1/fc2), the infix they were found under, and the projection
    names seen that are neither."""
    known = set(F.PROJECTIONS) | set(MLP_PROJECTIONS)
    by_layer, infix, other = {}, None, set()
    for name in tensors:
        m = _EXPERT_NAME.match(name)
        if m is None:
            continue
        proj, comp = m.group("proj"), m.group("comp")
        if proj not in known:
            other.add(proj)
        elif comp in F.COMPONENTS:
            by_layer.setdefault(int(m.group("layer")), {}).setdefault(proj, {})[comp] = name
            infix = m.group("infix")
    return by_layer, infix, other


def _layer_layout(li: int, comps_of: dict, tensors: dict):
    """(spec, expert count, [(path, offset of expert 0, bytes per expert)] in packing order) of
    one layer: projections in F.PROJECTIONS (or fc1, fc2) order, components in F.COMPONENTS
    order."""
    projections = MLP_PROJECTIONS if set(comps_of) <= set(MLP_PROJECTIONS) else F.PROJECTIONS
    spec, segs, count = {}, [], None
    for proj in projections:
        if not comps_of.get(proj):
            raise ValueError(f"layer {li} is missing {proj}; the checkpoint is incomplete")
        spec[proj] = {}
        for comp in (c for c in F.COMPONENTS if c in comps_of[proj]):
            name = comps_of[proj][comp]
            t = tensors[name]
            if len(t.shape) < 2:
                raise ValueError(f"{name} has shape {t.shape}; stacked expert tensors lead with E")
            if count is None:
                count = t.shape[0]
            if t.shape[0] != count:
                raise ValueError(f"layer {li}: {name} has {t.shape[0]} experts but a sibling "
                                 f"has {count}; the layer is refused rather than guessed at")
            dtype, isize = ST_DTYPES[t.dtype]
            per = isize * int(np.prod(t.shape[1:], dtype=np.int64))
            if per * count != t.nbytes:
                raise ValueError(f"{name}: {count} x {per} != {t.nbytes} bytes on disk; "
                                 f"the header and the data disagree")
            spec[proj][comp] = {"shape": list(t.shape[1:]), "dtype": dtype, "nbytes": per}
            segs.append((t.path, t.offset, per))
    return spec, count, segs


def expert_manifest(model_dir: str) -> CheckpointManifest:
    """Describe every routed expert of an MLX checkpoint by where its bytes already sit."""
    root = os.path.expanduser(model_dir)
    tensors = scan(root)
    with open(os.path.join(root, "config.json")) as f:
        cfg = json.load(f)
    by_layer, infix, other = _expert_tensors(tensors)
    if not by_layer:
        if other:
            raise ValueError(f"{root} is a mixture-of-experts model, but its experts use a "
                             f"{'/'.join(sorted(other))} layout; these kernels compute gated "
                             f"gate/up/down or two-layer fc1/fc2 experts")
        raise ValueError(f"{root} has no MoE expert tensors (looked for "
                         f"{', '.join('*' + i + '*' for i in EXPERT_INFIXES)})")
    man = CheckpointManifest(model_dir=root, config=cfg)
    top_k = cfg.get("num_experts_per_tok") or cfg.get("moe_topk")
    man.top_k = top_k if isinstance(top_k, int) and top_k > 0 else None
    for li in sorted(by_layer):
        spec, count, segs = _layer_layout(li, by_layer[li], tensors)
        per_expert = sum(n for _, _, n in segs)
        man.segments.update({f"{li}:{e}": [(p, o + e * n, n) for p, o, n in segs]
                             for e in range(count)})
        man.layers[str(li)] = {
            "n_experts": count, "spec": spec, "bytes_per_expert": per_expert,
            "quant": quant_for(cfg, f"model.layers.{li}{infix}{next(iter(spec))}", spec)}
        man.total_bytes += per_expert * count
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
    """The block's routing rule and activation as LayerSpec fields, from config.json, decided as
    adapter.py:75-93 describes it: sigmoid scoring when `score_function` / `scoring_func` names
    it, softmax when it names softmax, and otherwise sigmoid exactly when the config has
    expert groups; group-limited when `n_group` / `topk_group` are set; renormalised when
    `norm_topk_prob` is set; weights scaled by `routed_scaling_factor`. gpt-oss applies the
    softmax to the top-k logits and a clamped SwiGLU (`swiglu_limit`)."""
    mt = str(cfg.get("model_type", "")).lower()
    if mt == "gpt_oss":
        return {"route": "topk_softmax", "act": "swiglu_clamped",
                "limit": float(cfg.get("swiglu_limit", 7.0))}
    fn = str(cfg.get("score_function") or cfg.get("scoring_func") or "").lower()
    grouped = bool(cfg.get("n_group") or cfg.get("topk_group"))
    sigmoid = "sigmoid" in fn or ("softmax" not in fn and grouped)
    norm = bool(cfg.get("norm_topk_prob"))
    out = {"route": ("sigmoid_topk" if sigmoid else "softmax_topk") + ("_renorm" if norm else ""),
           "act": "swiglu"}
    if grouped:
        n_group = int(cfg.get("n_group") or 1)
        out.update(n_group=n_group, topk_group=int(cfg.get("topk_group") or n_group))
    scale = cfg.get("routed_scaling_factor")
    if scale is not None:
        out["route_scale"] = float(scale)
    return out


def layer_spec(man: CheckpointManifest, layer: int, **overrides):
    """The LayerSpec of one checkpoint layer: shapes from its expert tensors, quantization from
    the manifest, top-k and routing from config.json (any field can be overridden)."""
    from .spec import LayerSpec
    e = man.layers[str(layer)]
    q = man.quant(layer)
    two_layer = not F.is_gated(e["spec"])
    first = e["spec"]["fc1" if two_layer else "gate_proj"]
    inter = int(first["weight"]["shape"][0])
    # packed weights hold 32 / bits codes per uint32 word; bf16 weights are [n_out, n_in]
    n_words = int(first["weight"]["shape"][1])
    hidden = n_words if q.mode == "none" else n_words * 32 // q.bits
    kw = {"hidden": hidden, "inter": inter, "n_experts": int(e["n_experts"]),
          "top_k": int(man.top_k or 1), "quant": q, "has_bias": "bias" in first}
    kw.update(routing_from_config(man.config))
    if two_layer:
        kw["act"] = "silu_mlp"
    kw.update(overrides)
    spec = LayerSpec(**kw)
    if F.spec_bytes(spec.expert_spec()) != int(e["bytes_per_expert"]):
        raise ValueError(f"layer {layer}: the derived shape accounts for "
                         f"{F.spec_bytes(spec.expert_spec())} bytes per expert, the checkpoint "
                         f"holds {e['bytes_per_expert']}")
    return spec
