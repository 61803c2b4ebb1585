"""Byte layouts and quantization formats (CPU).

Pins: the reference's own shipped manifests (data/blobs/*.manifest.json, copied to tests/golden)
for shapes, dtypes and per-expert byte counts; bytes_per_param KATs from
tests/test_precision.py:31-47; closed forms for dequantization and the OCP e2m1 table;
torch's round-to-nearest-even for bf16.
"""
import json
import os

import numpy as np
import pytest

from bigrig_amd import formats as F
from bigrig_amd.spec import E256_SHARED, GPT_OSS_120B, OLMOE_1B_7B, QWEN3_30B_A3B

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_bytes_per_param_kats():
    # precision.py:54-55; test_precision.py:31-37
    bpp = F.bytes_per_param
    assert abs(bpp(4, 64) - 4.5 / 8) < 1e-12
    assert abs(bpp(2, 128) - 2.25 / 8) < 1e-12
    assert bpp(4, 128) < bpp(4, 64) < bpp(4, 32)
    assert bpp(2, 64) < bpp(3, 64) < bpp(4, 64) < bpp(8, 64)


@pytest.mark.parametrize("spec,want", [
    (QWEN3_30B_A3B, 2_654_208), (OLMOE_1B_7B, 3_538_944), (E256_SHARED, 1_769_472),
    (GPT_OSS_120B, 13_236_480)])
def test_bytes_per_expert(spec, want):
    assert spec.bytes_per_expert == want
    if spec.quant.mode == "affine":
        # closed form 3 * (I*H/2 + 2*I*(H/64)*2)
        H, I = spec.hidden, spec.inter
        assert want == 3 * (I * H // 2 + 2 * I * (H // 64) * 2)


@pytest.mark.parametrize("name,H,I,q", [
    ("OLMoE-1B-7B-0125-4bit", 2048, 1024, F.QuantSpec(4, 64, "affine", "float16")),
    ("Qwen3-30B-A3B-3bit", 2048, 768, F.QuantSpec(3, 64, "affine", "bfloat16"))])
def test_spec_matches_shipped_manifest(name, H, I, q):
    """Our layout arithmetic reproduces the reference blob manifests exactly (stream.py:133-151)."""
    with open(os.path.join(GOLDEN, f"{name}.experts.manifest.json")) as f:
        man = F.Manifest.from_dict(json.load(f))
    man.check()
    for li, entry in man.layers.items():
        assert entry["spec"] == F.expert_spec(H, I, q)
        assert int(entry["bytes_per_expert"]) == F.spec_bytes(F.expert_spec(H, I, q))
        assert man.quant(li) == q
    # regions are contiguous per layer in expert order (the pack_experts loop, stream.py:152-165)
    per = F.spec_bytes(F.expert_spec(H, I, q))
    o0, n0 = man.region(0, 0)
    o1, _ = man.region(0, 1)
    assert (o0, n0, o1) == (0, per, per)
    with pytest.raises(KeyError):
        man.region(10_000, 0)


def test_manifest_check_catches_gaps_and_wrong_sizes():
    spec = F.expert_spec(128, 64, F.QuantSpec())
    per = F.spec_bytes(spec)
    good = {"version": 4, "total_bytes": 2 * per, "regions": {"0:0": [0, per], "0:1": [per, per]},
            "layers": {"0": {"n_experts": 2, "spec": spec, "bytes_per_expert": per}}}
    F.Manifest.from_dict(good).check()
    gap = json.loads(json.dumps(good))
    gap["regions"]["0:1"] = [per + 16, per]
    gap["total_bytes"] = 2 * per + 16
    with pytest.raises(ValueError):
        F.Manifest.from_dict(gap).check()
    bad = json.loads(json.dumps(good))
    bad["layers"]["0"]["bytes_per_expert"] = per + 1
    with pytest.raises(ValueError):
        F.Manifest.from_dict(bad).check()
    old = json.loads(json.dumps(good))
    old["version"] = 3
    with pytest.raises(ValueError):
        F.Manifest.from_dict(old)


def test_pack_blob_roundtrip(tmp_path):
    rng = np.random.default_rng(0)
    q = F.QuantSpec()
    spec = F.expert_spec(128, 64, q)
    experts = [F.make_expert(rng, 128, 64, q) for _ in range(3)]
    path = str(tmp_path / "t.experts")
    man = F.pack_blob(path, {0: (spec, q, experts), 1: (spec, q, experts[::-1])}, top_k=2)
    man2 = F.Manifest.load(path)
    man2.check()
    assert man2.top_k == 2 and man2.total_bytes == os.path.getsize(path) == 6 * len(experts[0])
    blob = open(path, "rb").read()
    o, n = man2.region(1, 0)
    assert blob[o:o + n] == experts[2]
    assert man.regions == man2.regions


def test_unquantized_layout_and_manifest(tmp_path):
    """Unquantized experts: each projection is its bf16 weight [n_out, n_in] (+ bias), no
    scales; the layer's manifest entry carries no quant record (stream.py:145-149) and reading
    it back, the tensors decide (direct.py:110-142): no scales is the unquantized mode."""
    rng = np.random.default_rng(5)
    q = F.QuantSpec(16, 0, "none")
    spec = F.expert_spec(128, 64, q, has_bias=True)
    assert spec["gate_proj"] == {"weight": {"shape": [64, 128], "dtype": "bfloat16", "nbytes": 64 * 128 * 2},
                                 "bias": {"shape": [64], "dtype": "bfloat16", "nbytes": 128}}
    assert F.spec_bytes(spec) == 3 * 64 * 128 * 2 + 2 * 64 * 2 + 128 * 2
    experts = [F.make_expert(rng, 128, 64, q, has_bias=True) for _ in range(2)]
    arrs = F.split_expert(experts[1], spec)
    w = F.dequantize_projection(arrs, "down_proj", q)
    assert w.shape == (128, 64) and np.array_equal(w, F.bf16_bits_to_f32(arrs[("down_proj", "weight")]))
    path = str(tmp_path / "u.experts")
    F.pack_blob(path, {0: (spec, q, experts)}, top_k=2)
    man = F.Manifest.load(path)
    assert "quant" not in man.layers["0"] and man.quant(0) == q
    # a layer with scales but no quant record keeps the 4-bit default
    q4 = F.QuantSpec()
    F.pack_blob(path, {0: (F.expert_spec(128, 64, q4), q4, [F.make_expert(rng, 128, 64, q4)])})
    d = json.load(open(path + ".manifest.json"))
    del d["layers"]["0"]["quant"]
    assert F.Manifest.from_dict(d).quant(0) == q4
    with pytest.raises(ValueError):
        F.QuantSpec(16, 64, "none")


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_pack_unpack_roundtrip(bits):
    rng = np.random.default_rng(bits)
    K = 64 * 4
    q = rng.integers(0, 1 << bits, size=(5, K)).astype(np.uint8)
    w = F.pack_bits(q, bits)
    assert w.dtype == np.uint32 and w.shape == (5, K * bits // 32)
    assert np.array_equal(F.unpack_bits(w, bits, K), q)


def test_pack_order_kats():
    # 4-bit: value j of a word in bits [4j, 4j+4), least significant first
    q = np.arange(8, dtype=np.uint8)[None, :]
    assert F.pack_bits(q, 4)[0, 0] == 0x76543210
    # 3-bit: 8 values in 3 bytes, value j at bits [3j, 3j+3) of the little-endian 24-bit run
    q3 = np.array([[1, 2, 3, 4, 5, 6, 7, 0] * 4], dtype=np.uint8)
    word = sum(int(v) << (3 * j) for j, v in enumerate([1, 2, 3, 4, 5, 6, 7, 0]))
    by = F.pack_bits(q3, 3).view(np.uint8)[0]
    assert list(by[:3]) == [word & 0xFF, (word >> 8) & 0xFF, (word >> 16) & 0xFF]


def test_bf16_rounding_matches_torch():
    import torch
    rng = np.random.default_rng(1)
    a = np.concatenate([(rng.standard_normal(10000) * 10.0 ** rng.integers(-30, 30, 10000)).astype(np.float32),
                        np.array([0.0, -0.0, np.inf, -np.inf, 1.0, 3.0], np.float32),
                        np.array([0x3F808000, 0x3F818000, 0x3F80FFFF], np.uint32).view(np.float32)])
    ours = F.f32_to_bf16_bits(a)
    theirs = torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    # ties go to even
    assert F.f32_to_bf16_bits(np.array([0x3F808000], np.uint32).view(np.float32))[0] == 0x3F80
    assert F.f32_to_bf16_bits(np.array([0x3F818000], np.uint32).view(np.float32))[0] == 0x3F82
    assert np.isnan(F.bf16_bits_to_f32(F.f32_to_bf16_bits(np.array([np.nan], np.float32))))[0]


@pytest.mark.parametrize("scale_dtype", ["bfloat16", "float16"])
def test_affine_dequant_single_rounding(scale_dtype):
    """w = fl32(s*q + b): s*q is exact, so the fp32 result equals the float64 value rounded once."""
    rng = np.random.default_rng(2)
    w = rng.standard_normal((16, 256)).astype(np.float32) * 0.02
    wq, s, b = F.quantize_affine(w, 64, 4, scale_dtype)
    got = F.dequantize_affine(wq, s, b, 64, 4, scale_dtype)
    cvt = F.bf16_bits_to_f32 if scale_dtype == "bfloat16" else F.f16_bits_to_f32
    q = F.unpack_bits(wq, 4, 256).astype(np.float64).reshape(16, 4, 64)
    want = (cvt(s).astype(np.float64)[..., None] * q + cvt(b).astype(np.float64)[..., None])
    assert np.array_equal(got, want.astype(np.float32).reshape(16, 256))
    # error bound of the MLX-style quantizer: half a step inside the covered range, plus the
    # shortfall 15*|s - s0| at the far end, where s0 = (max - min)/15 is the unsnapped step and
    # s = edge/round(edge/s0) the step after snapping the zero point onto the group edge,
    # plus the 16-bit rounding of s (x15) and of the bias
    g = w.reshape(16, 4, 64)
    s0 = (g.max(-1) - g.min(-1)) / 15.0
    step = np.abs(cvt(s))
    ulp = 2.0 ** -8 if scale_dtype == "bfloat16" else 2.0 ** -11
    bound = 0.5 * step + 15 * np.abs(step - s0) + ulp * (16 * step + np.abs(g).max(-1)) + 1e-7
    err = np.abs(got - w).reshape(16, 4, 64).max(-1)
    assert (err <= bound).all()
    # a plausible slip (bias applied with the wrong sign) breaks the bound
    bad = F.dequantize_affine(wq, s, b ^ np.uint16(0x8000), 64, 4, scale_dtype)
    assert not (np.abs(bad - w).reshape(16, 4, 64).max(-1) <= bound).all()


def test_affine_quantizer_special_groups():
    # a constant group: bias = the value, scale irrelevant, dequant exact up to bf16 rounding
    w = np.full((1, 64), 0.25, np.float32)
    wq, s, b = F.quantize_affine(w)
    assert np.allclose(F.dequantize_affine(wq, s, b), 0.25)
    # zero weights dequantize to exact zero
    wq, s, b = F.quantize_affine(np.zeros((2, 128), np.float32))
    assert not np.any(F.dequantize_affine(wq, s, b))


def test_e2m1_table_is_the_ocp_definition():
    for c in range(16):
        sign = -1.0 if c & 8 else 1.0
        e, m = (c >> 1) & 3, c & 1
        v = sign * (0.5 * m if e == 0 else 2.0 ** (e - 1) * (1 + 0.5 * m))
        assert F.E2M1_VALUES[c] == np.float32(v)


def test_mxfp4_roundtrip_and_scales():
    rng = np.random.default_rng(3)
    w = rng.standard_normal((8, 128)).astype(np.float32) * 0.02
    wq, sc = F.quantize_mxfp4(w)
    assert wq.shape == (8, 16) and sc.shape == (8, 4) and sc.dtype == np.uint8
    d = F.dequantize_mxfp4(wq, sc)
    # |w| / 2^e lies in [0, 8); e2m1 steps are at most 2 (rounding error <= 1 unit) and values in
    # [6, 8) saturate to 6 (error < 2 units), so |err| < 2 * 2^e with 2^e = 2^(e8m0 - 127)
    scale = np.ldexp(1.0, sc.astype(np.int64) - 127)
    err = np.abs(d - w).reshape(8, 4, 32).max(-1)
    assert (err <= 2 * scale + 1e-12).all()
    # exact values survive: a group of e2m1 values times 2^-3
    g = (F.E2M1_VALUES[np.arange(32) % 16] * 0.125).astype(np.float32)[None, :]
    gq, gs = F.quantize_mxfp4(g)
    assert np.array_equal(F.dequantize_mxfp4(gq, gs), g)
    # e8m0 special values
    one = F.dequantize_mxfp4(np.full((1, 4), 0x22222222, np.uint32), np.full((1, 1), 127, np.uint8))
    assert np.all(one == 1.0)
    nan = F.dequantize_mxfp4(np.full((1, 4), 0x22222222, np.uint32), np.full((1, 1), 255, np.uint8))
    assert np.all(np.isnan(nan))


def test_split_join_and_short_region():
    rng = np.random.default_rng(4)
    q = F.QuantSpec(4, 32, "mxfp4")
    spec = F.expert_spec(128, 64, q, has_bias=True)
    blob = F.make_expert(rng, 128, 64, q, has_bias=True)
    arrs = F.split_expert(blob, spec)
    assert list(arrs) == [(p, c) for p in F.PROJECTIONS for c in ("weight", "scales", "bias")]
    assert F.join_expert(arrs, spec) == blob
    with pytest.raises(ValueError, match="manifest accounts"):
        F.split_expert(blob[:-4], spec)
    offs = F.spec_offsets(spec)
    assert offs[("gate_proj", "weight")] == 0
    assert offs[("down_proj", "bias")] == len(blob) - 128 * 2
