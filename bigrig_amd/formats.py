"""Byte layouts of one routed expert, kept identical to the MLX layouts BigRig packs.

An expert is its projections in order (gate_proj, up_proj, down_proj), and each projection is
its components in order (weight, scales, biases, bias); the bytes of each component follow the
previous one with no padding. This is the layout `pack_experts` writes into a blob region
(bigrig_engine/stream.py:106-186, `PROJECTIONS` stream.py:56, `COMPONENTS` stream.py:81) and the
one `ExpertPool.build_arrays` reinterprets as 1-D uint8 -> view(dtype) -> reshape(shape)
(stream.py:707-755). A pool slot in HBM holds exactly these bytes, so a blob region is copied
into a slot verbatim.

Quantized formats (the arithmetic MLX defines; MLX itself is not importable here):

* affine (MLX `mode="affine"`): weight uint32 [N, K*bits/32] with 32/bits values per word, value
  j of a word in bits [bits*j, bits*j + bits) (least significant first); scales and biases
  [N, K/group] in bf16 (fp16 in some checkpoints). w = scale * q + bias.
* mxfp4 (MLX `mode="mxfp4"`): weight uint32 [N, K/8], e2m1 nibbles least significant first
  (two per byte, low nibble first); scales uint8 [N, K/32] holding an e8m0 exponent; no biases.
  w = e2m1(q) * 2**(e - 127). An optional per-output `bias` [N] bf16 follows (gpt-oss).

Everything bf16 is carried as uint16 bit patterns: numpy has no bfloat16.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass, field

import numpy as np

PROJECTIONS = ("gate_proj", "up_proj", "down_proj")
MLP_PROJECTIONS = ("fc1", "fc2")      # a plain two-layer expert, fc2(silu(fc1 x)) (stream.py:57)
COMPONENTS = ("weight", "scales", "biases", "bias")

# e2m1 code -> value (sign in bit 3). OCP Microscaling spec, element type FP4 E2M1.
E2M1_VALUES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                        -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=np.float32)

DTYPE_SIZE = {"uint32": 4, "uint8": 1, "bfloat16": 2, "float16": 2, "float32": 4}


# --------------------------------------------------------------------------- bf16 helpers
def f32_to_bf16_bits(a) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even; NaN stays NaN."""
    a = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    if nan.any():
        r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r


def bf16_bits_to_f32(b) -> np.ndarray:
    b = np.asarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_bf16(a) -> np.ndarray:
    """float32 values rounded through bf16 and back."""
    return bf16_bits_to_f32(f32_to_bf16_bits(a))


def f16_bits_to_f32(b) -> np.ndarray:
    return np.asarray(b, dtype=np.uint16).view(np.float16).astype(np.float32)


# --------------------------------------------------------------------------- quant descriptor
@dataclass(frozen=True)
class QuantSpec:
    """(bits, group_size, mode) per layer, as the blob manifest records it
    (`entry["quant"]`, stream.py:145-149)."""
    bits: int = 4
    group_size: int = 64
    mode: str = "affine"          # "affine" | "mxfp4" | "none" (unquantized bf16 weights)
    scale_dtype: str = "bfloat16"  # affine only: "bfloat16" | "float16"

    def __post_init__(self):
        if self.mode not in ("affine", "mxfp4", "none"):
            raise ValueError(f"unknown quant mode {self.mode!r}")
        if self.mode == "none" and (self.bits != 16 or self.group_size != 0):
            raise ValueError("unquantized experts are bf16: bits 16, no scale groups")
        if self.mode == "mxfp4" and (self.bits != 4 or self.group_size != 32):
            raise ValueError("mxfp4 is 4-bit with 32-element scale groups")
        if self.mode == "affine" and self.bits not in (2, 3, 4, 5, 6, 8):
            raise ValueError(f"affine bits {self.bits} not supported")


def bytes_per_param(bits: int, group_size: int) -> float:
    """Affine bytes per parameter including a 16-bit scale and bias per group
    (bigrig_engine/precision.py:54-55)."""
    return (bits + 32.0 / group_size) / 8.0


def projection_spec(n_out: int, n_in: int, q: QuantSpec, has_bias: bool = False) -> dict:
    """{component: {shape, dtype, nbytes}} of one projection W [n_out, n_in], in COMPONENTS
    order, as the manifest records it (stream.py:133-138). Unquantized (mode "none"): the bf16
    weight alone (+ bias), no scales -- the tensors an unquantized checkpoint carries
    (direct.py:110-142)."""
    if q.mode == "none":
        spec = {"weight": {"shape": [n_out, n_in], "dtype": "bfloat16"}}
        if has_bias:
            spec["bias"] = {"shape": [n_out], "dtype": "bfloat16"}
        for c in spec.values():
            c["nbytes"] = int(np.prod(c["shape"])) * DTYPE_SIZE[c["dtype"]]
        return spec
    if n_in % q.group_size:
        raise ValueError(f"input dim {n_in} is not a multiple of group size {q.group_size}")
    if (n_in * q.bits) % 32:
        raise ValueError(f"input dim {n_in} at {q.bits} bits does not fill whole uint32 words")
    spec = {"weight": {"shape": [n_out, n_in * q.bits // 32], "dtype": "uint32"}}
    G = n_in // q.group_size
    if q.mode == "affine":
        spec["scales"] = {"shape": [n_out, G], "dtype": q.scale_dtype}
        spec["biases"] = {"shape": [n_out, G], "dtype": q.scale_dtype}
    else:
        spec["scales"] = {"shape": [n_out, G], "dtype": "uint8"}
    if has_bias:
        spec["bias"] = {"shape": [n_out], "dtype": "bfloat16"}
    for c in spec.values():
        c["nbytes"] = int(np.prod(c["shape"])) * DTYPE_SIZE[c["dtype"]]
    return spec


def expert_spec(hidden: int, inter: int, q: QuantSpec, has_bias: bool = False,
                gated: bool = True) -> dict:
    """Manifest `spec` of one expert. Gated: gate/up are [inter, hidden], down is [hidden,
    inter]. Not gated (a plain two-layer expert): fc1 [inter, hidden], fc2 [hidden, inter]."""
    if not gated:
        return {"fc1": projection_spec(inter, hidden, q, has_bias),
                "fc2": projection_spec(hidden, inter, q, has_bias)}
    return {"gate_proj": projection_spec(inter, hidden, q, has_bias),
            "up_proj": projection_spec(inter, hidden, q, has_bias),
            "down_proj": projection_spec(hidden, inter, q, has_bias)}


def is_gated(spec: dict) -> bool:
    """Whether an expert spec is gated (gate/up/down) or a plain two-layer expert (fc1/fc2)."""
    return tuple(spec) != MLP_PROJECTIONS


def spec_bytes(spec: dict) -> int:
    """Bytes of one expert: the sum of its component arrays (stream.py:539-541)."""
    return sum(c["nbytes"] for p in spec.values() for c in p.values())


def spec_offsets(spec: dict) -> dict:
    """{(proj, comp): byte offset within the expert} in packing order."""
    out, pos = {}, 0
    for proj in spec:
        for comp in COMPONENTS:
            if comp in spec[proj]:
                out[(proj, comp)] = pos
                pos += spec[proj][comp]["nbytes"]
    return out


def split_expert(blob, spec: dict) -> dict:
    """One expert's packed bytes as {(proj, comp): ndarray}, the 1-D uint8 -> view -> reshape
    sequence of ExpertPool.build_arrays (stream.py:739-755). bf16/fp16 come back as uint16.
    Raises ValueError if the region is not exactly the manifest's size (stream.py:696-703)."""
    raw = np.frombuffer(blob, dtype=np.uint8)
    want = spec_bytes(spec)
    if raw.nbytes != want:
        raise ValueError(f"the manifest accounts for {want} bytes but the region supplied "
                         f"{raw.nbytes}")
    out, pos = {}, 0
    for proj in spec:
        for comp in COMPONENTS:
            if comp not in spec[proj]:
                continue
            m = spec[proj][comp]
            n = m["nbytes"]
            dt = {"uint32": np.uint32, "uint8": np.uint8, "bfloat16": np.uint16,
                  "float16": np.uint16, "float32": np.float32}[m["dtype"]]
            out[(proj, comp)] = raw[pos:pos + n].view(dt).reshape(m["shape"])
            pos += n
    return out


def join_expert(arrays: dict, spec: dict) -> bytes:
    """Inverse of split_expert: concatenate component bytes in packing order."""
    parts = []
    for proj in spec:
        for comp in COMPONENTS:
            if comp in spec[proj]:
                a = np.ascontiguousarray(arrays[(proj, comp)])
                if a.nbytes != spec[proj][comp]["nbytes"]:
                    raise ValueError(f"{proj}.{comp}: {a.nbytes} bytes, spec says "
                                     f"{spec[proj][comp]['nbytes']}")
                parts.append(a.tobytes())
    return b"".join(parts)


# --------------------------------------------------------------------------- packing
def pack_bits(q: np.ndarray, bits: int) -> np.ndarray:
    """Pack unsigned integer codes [N, K] along K into uint32 words, LSB first.

    bits 2/4/8 divide 32 and pack 32/bits values per word. bits 3/5/6 pack byte-aligned runs
    (8 values in 3 bytes, 8 in 5, 4 in 3), which is how MLX lays out those widths; the result is
    then viewed as uint32 words (K*bits must be a multiple of 32)."""
    q = np.asarray(q, dtype=np.uint64)
    N, K = q.shape
    if (K * bits) % 32:
        raise ValueError("K*bits must be a multiple of 32")
    if 32 % bits == 0:
        per = 32 // bits
        qq = q.reshape(N, K // per, per)
        shifts = (np.arange(per, dtype=np.uint64) * bits)
        return (qq << shifts).sum(axis=-1).astype(np.uint32)
    per, nbytes = {3: (8, 3), 5: (8, 5), 6: (4, 3)}[bits]
    qq = q.reshape(N, K // per, per)
    shifts = (np.arange(per, dtype=np.uint64) * bits)
    word = (qq << shifts).sum(axis=-1)             # up to 40 bits
    by = np.stack([(word >> np.uint64(8 * i)) & np.uint64(0xFF) for i in range(nbytes)], -1)
    return by.astype(np.uint8).reshape(N, -1).view(np.uint32)


def unpack_bits(w: np.ndarray, bits: int, K: int) -> np.ndarray:
    """Inverse of pack_bits: uint32 [N, K*bits/32] -> codes uint8 [N, K]."""
    w = np.ascontiguousarray(np.asarray(w, dtype=np.uint32))
    N = w.shape[0]
    if 32 % bits == 0:
        per = 32 // bits
        shifts = (np.arange(per, dtype=np.uint32) * bits)
        q = (w[:, :, None] >> shifts) & np.uint32((1 << bits) - 1)
        return q.reshape(N, -1)[:, :K].astype(np.uint8)
    per, nbytes = {3: (8, 3), 5: (8, 5), 6: (4, 3)}[bits]
    by = w.view(np.uint8).reshape(N, -1, nbytes).astype(np.uint64)
    word = sum(by[..., i] << np.uint64(8 * i) for i in range(nbytes))
    shifts = (np.arange(per, dtype=np.uint64) * bits)
    q = (word[..., None] >> shifts) & np.uint64((1 << bits) - 1)
    return q.reshape(N, -1)[:, :K].astype(np.uint8)


# --------------------------------------------------------------------------- quantizers
def quantize_affine(w: np.ndarray, group_size: int = 64, bits: int = 4,
                    scale_dtype: str = "bfloat16"):
    """MLX-style affine quantization of W [N, K] along K.

    Per group: the edge of larger magnitude (min or max) is made exactly representable, the
    scale spans max - min over 2**bits - 1 steps, bias = that edge (or 0). Codes are computed
    against the float32 scale/bias, which are then stored rounded to `scale_dtype`. This is the
    build's documented quantizer (MLX's published `mx.quantize` algorithm restated); layer
    parity never depends on it, because the kernels and the oracle dequantize the same bytes.
    Returns (weight uint32, scales uint16 bits, biases uint16 bits)."""
    w = np.asarray(w, dtype=np.float32)
    N, K = w.shape
    n_bins = float((1 << bits) - 1)
    g = w.reshape(N, K // group_size, group_size)
    w_max = g.max(-1)
    w_min = g.min(-1)
    mask = np.abs(w_min) > np.abs(w_max)
    scales = np.maximum((w_max - w_min) / n_bins, 1e-7).astype(np.float32)
    scales = np.where(mask, scales, -scales)
    edge = np.where(mask, w_min, w_max)
    q0 = np.round(edge / scales)
    with np.errstate(divide="ignore", invalid="ignore"):
        scales = np.where(q0 != 0, edge / np.where(q0 != 0, q0, 1), scales).astype(np.float32)
    biases = np.where(q0 == 0, 0.0, edge).astype(np.float32)
    q = np.clip(np.round((g - biases[..., None]) / scales[..., None]), 0, n_bins)
    q = q.reshape(N, K).astype(np.uint32)
    if scale_dtype == "bfloat16":
        s_bits, b_bits = f32_to_bf16_bits(scales), f32_to_bf16_bits(biases)
    elif scale_dtype == "float16":
        s_bits = scales.astype(np.float16).view(np.uint16)
        b_bits = biases.astype(np.float16).view(np.uint16)
    else:
        raise ValueError(scale_dtype)
    return pack_bits(q, bits), s_bits, b_bits


def dequantize_affine(wq, scales, biases, group_size: int = 64, bits: int = 4,
                      scale_dtype: str = "bfloat16") -> np.ndarray:
    """fp32 dequant w = s*q + b. s*q is exact in fp32 (<= 11 + 8 significant bits), so the
    single rounding of the add makes this bit-exact whatever the evaluation order."""
    N = wq.shape[0]
    K = wq.shape[1] * 32 // bits
    q = unpack_bits(wq, bits, K).astype(np.float32).reshape(N, -1, group_size)
    cvt = bf16_bits_to_f32 if scale_dtype == "bfloat16" else f16_bits_to_f32
    s = cvt(scales)[..., None]
    b = cvt(biases)[..., None]
    return (s * q + b).astype(np.float32).reshape(N, K)


def _e2m1_encode(v: np.ndarray) -> np.ndarray:
    """Nearest e2m1 code (ties to even mantissa), saturating at +-6."""
    a = np.minimum(np.abs(v), 6.0)
    mags = E2M1_VALUES[:8]
    # distance to every magnitude; ties resolved toward the even code (codes 0,2,4,6 have an
    # even mantissa bit)
    d = np.abs(a[..., None] - mags)
    best = d.min(-1, keepdims=True)
    cand = (d == best)
    even = (np.arange(8) % 2 == 0)
    code = np.where(cand & even, np.arange(8), 99).min(-1)
    code = np.where(code == 99, np.argmax(cand, axis=-1), code)
    sign = (np.signbit(v) & (code > 0)).astype(np.int64) << 3
    return (code | sign).astype(np.uint8)


def quantize_mxfp4(w: np.ndarray):
    """OCP MXFP4 quantization of W [N, K] along K in groups of 32: shared exponent
    e = floor(log2(amax)) - 2 (e2m1's largest exponent), elements rounded to e2m1.
    Returns (weight uint32 [N, K/8], scales uint8 [N, K/32])."""
    w = np.asarray(w, dtype=np.float32)
    N, K = w.shape
    g = w.reshape(N, K // 32, 32)
    amax = np.abs(g).max(-1)
    with np.errstate(divide="ignore"):
        e = np.where(amax > 0, np.floor(np.log2(np.maximum(amax, 1e-38))) - 2, -127)
    e = np.clip(e, -127, 127).astype(np.int64)
    scaled = g / np.exp2(e.astype(np.float64))[..., None]
    codes = _e2m1_encode(scaled.astype(np.float32)).reshape(N, K)
    return pack_bits(codes, 4), (e + 127).astype(np.uint8)


def dequantize_mxfp4(wq, scales) -> np.ndarray:
    N = wq.shape[0]
    K = wq.shape[1] * 8
    q = unpack_bits(wq, 4, K).reshape(N, -1, 32)
    vals = E2M1_VALUES[q]
    e = np.asarray(scales, dtype=np.int64)
    p = np.where(e == 255, np.nan, np.ldexp(np.float32(1.0), (e - 127).astype(np.int32)))
    return (vals * p[..., None].astype(np.float32)).astype(np.float32).reshape(N, K)


# --------------------------------------------------------------------------- expert factory
def dequantize_projection(arrays: dict, proj: str, q: QuantSpec) -> np.ndarray:
    """fp32 dequantized weight [n_out, n_in] of one projection from split_expert() arrays."""
    if q.mode == "none":
        return bf16_bits_to_f32(arrays[(proj, "weight")])
    if q.mode == "affine":
        return dequantize_affine(arrays[(proj, "weight")], arrays[(proj, "scales")],
                                 arrays[(proj, "biases")], q.group_size, q.bits, q.scale_dtype)
    return dequantize_mxfp4(arrays[(proj, "weight")], arrays[(proj, "scales")])


def make_expert(rng: np.random.Generator, hidden: int, inter: int, q: QuantSpec,
                std: float = 0.02, has_bias: bool = False, bias_std: float = 0.02,
                gated: bool = True) -> bytes:
    """One synthetic expert: N(0, std) weights quantized to `q`, packed in blob layout."""
    spec = expert_spec(hidden, inter, q, has_bias, gated)
    arrays = {}
    for proj in spec:
        n_out, n_in = (inter, hidden) if proj in ("gate_proj", "up_proj", "fc1") else (hidden, inter)
        w = (rng.standard_normal((n_out, n_in), dtype=np.float32) * std).astype(np.float32)
        if q.mode == "none":
            arrays[(proj, "weight")] = f32_to_bf16_bits(w)
        elif q.mode == "affine":
            wq, s, b = quantize_affine(w, q.group_size, q.bits, q.scale_dtype)
            arrays[(proj, "weight")], arrays[(proj, "scales")], arrays[(proj, "biases")] = wq, s, b
        else:
            wq, s = quantize_mxfp4(w)
            arrays[(proj, "weight")], arrays[(proj, "scales")] = wq, s
        if has_bias:
            arrays[(proj, "bias")] = f32_to_bf16_bits(
                rng.standard_normal(n_out, dtype=np.float32) * bias_std)
    return join_expert(arrays, spec)


# --------------------------------------------------------------------------- manifest v4
@dataclass
class Manifest:
    """The blob manifest (version 4): regions "L:e" -> [offset, length], per-layer
    {n_experts, spec, bytes_per_expert, quant}, total_bytes, top_k (stream.py:120-186)."""
    layers: dict = field(default_factory=dict)
    regions: dict = field(default_factory=dict)
    total_bytes: int = 0
    top_k: int | None = None
    version: int = 4

    @classmethod
    def load(cls, blob_path: str) -> "Manifest":
        """Read `<blob>.manifest.json` (stream.py:221-228)."""
        p = os.path.expanduser(blob_path) + ".manifest.json"
        if not os.path.exists(p):
            raise FileNotFoundError(f"{p} not found: a blob without its manifest has no known "
                                    f"byte layout")
        with open(p) as f:
            d = json.load(f)
        return cls.from_dict(d)

    @classmethod
    def from_dict(cls, d: dict) -> "Manifest":
        if int(d.get("version", 0)) < 4:
            raise ValueError(f"manifest version {d.get('version')} < 4 carries no quant record")
        return cls(layers=d["layers"], regions=d["regions"], total_bytes=int(d["total_bytes"]),
                   top_k=d.get("top_k"), version=int(d["version"]))

    def to_dict(self) -> dict:
        d = {"regions": self.regions, "layers": self.layers, "version": self.version,
             "total_bytes": self.total_bytes}
        if self.top_k:
            d["top_k"] = self.top_k
        return d

    def quant(self, layer) -> QuantSpec:
        """The layer's quant record; without one, the tensors decide (direct.py:110-142): no
        `scales` beside the weights is an unquantized (bf16) layer."""
        e = self.layers[str(layer)]
        spec = e["spec"]
        first = next(iter(spec.values()))
        if not e.get("quant") and not any("scales" in comps for comps in spec.values()):
            return QuantSpec(16, 0, "none")
        qd = e.get("quant") or {"bits": 4, "group_size": 64, "mode": "affine"}
        sd = first.get("scales", {}).get("dtype", "bfloat16")
        if qd.get("mode", "affine") != "affine":
            sd = "bfloat16"
        return QuantSpec(int(qd["bits"]), int(qd["group_size"]), qd.get("mode", "affine"), sd)

    def region(self, layer: int, expert: int) -> tuple:
        key = f"{layer}:{expert}"
        if key not in self.regions:
            raise KeyError((layer, expert))
        o, n = self.regions[key]
        return int(o), int(n)

    def check(self) -> None:
        """Regions tile [0, total_bytes) with no gap or overlap, and each layer's
        bytes_per_expert equals the sum of its component arrays (test_stream.py:45-55)."""
        regs = sorted((int(o), int(n)) for o, n in self.regions.values())
        pos = 0
        for o, n in regs:
            if o != pos:
                raise ValueError(f"region at {o} does not follow the previous one ending at {pos}")
            pos = o + n
        if pos != self.total_bytes:
            raise ValueError(f"regions cover {pos} bytes, manifest says {self.total_bytes}")
        for li, e in self.layers.items():
            if spec_bytes(e["spec"]) != int(e["bytes_per_expert"]):
                raise ValueError(f"layer {li}: bytes_per_expert disagrees with its spec")


def pack_blob(path: str, layers: dict, top_k: int | None = None) -> Manifest:
    """Write experts {layer: [bytes per expert]} expert-contiguous, plus a v4 manifest, in the
    format of stream.pack_experts. `layers[l]` is (spec, quant, [expert bytes])."""
    man = Manifest(top_k=top_k)
    off = 0
    with open(path, "wb") as f:
        for li in sorted(layers):
            spec, q, experts = layers[li]
            per = spec_bytes(spec)
            entry = {"n_experts": len(experts), "spec": spec, "bytes_per_expert": per}
            if q.mode != "none":    # an unquantized layer carries no quant record (stream.py:145-149)
                entry["quant"] = {"group_size": q.group_size, "bits": q.bits, "mode": q.mode}
            man.layers[str(li)] = entry
            for e, b in enumerate(experts):
                if len(b) != per:
                    raise ValueError(f"layer {li} expert {e}: {len(b)} bytes, spec says {per}")
                f.write(b)
                man.regions[f"{li}:{e}"] = [off, per]
                off += per
    man.total_bytes = off
    with open(path + ".manifest.json", "w") as f:
        json.dump(man.to_dict(), f)
    return man
