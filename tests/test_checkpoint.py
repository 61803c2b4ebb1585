"""Reading routed experts straight out of an MLX checkpoint's safetensors shards.

The central assertion is the reference's (tests/test_direct.py:39-83): expert e read from the
checkpoint is EXACTLY the bytes a packed blob holds for expert e, and the checkpoint manifest
describes the same layers (spec, bytes per expert, quantization, top-k) as the blob's. The
parser refuses malformed files before trusting any byte (test_direct.py:85-116).
"""
import json
import os
import struct

import numpy as np
import pytest

from bigrig_amd import checkpoint as CK
from bigrig_amd import formats as F
from bigrig_amd.spec import QWEN3_30B_A3B
from tests.ckpt_util import make_checkpoint, write_safetensors
from tests.helpers import small

Q4 = F.QuantSpec(4, 64, "affine")
Q3 = F.QuantSpec(3, 64, "affine")
Q4F16 = F.QuantSpec(4, 64, "affine", "float16")
MX = F.QuantSpec(4, 32, "mxfp4")


def _pack(tmp_path, made, top_k=2):
    blob = str(tmp_path / "b.experts")
    return blob, F.pack_blob(blob, made, top_k=top_k)


def test_checkpoint_experts_are_the_packed_blob_bytes(tmp_path):
    d = str(tmp_path / "model")
    made = make_checkpoint(d, {0: (128, 64, 4, Q4, False), 1: (128, 64, 4, Q4, False),
                               2: (128, 64, 4, Q4, False)}, shards=2)
    blob, bm = _pack(tmp_path, made)
    cm = CK.expert_manifest(d)
    assert cm.total_bytes == bm.total_bytes
    assert cm.top_k == bm.top_k == 2
    assert set(cm.segments) == set(bm.regions)
    for li in bm.layers:
        a, b = cm.layers[li], bm.layers[li]
        assert a["n_experts"] == b["n_experts"] and a["bytes_per_expert"] == b["bytes_per_expert"]
        assert a["spec"] == b["spec"], "shapes, dtypes and component order must match the blob"
        assert a["quant"] == b["quant"]
    raw = np.fromfile(blob, dtype=np.uint8)
    for li in (0, 1, 2):
        for e in range(4):
            o, n = bm.region(li, e)
            got = CK.read_expert(cm, li, e)
            assert got == raw[o:o + n].tobytes(), (li, e)
            assert len(cm.expert_segments(li, e)) == 9    # 3 projections x weight/scales/biases
    assert CK.read_expert(cm, 0, 0) != CK.read_expert(cm, 0, 1)


def test_three_bit_and_f16_and_mxfp4_layers(tmp_path):
    """Other layouts the manifest records: a 3-bit layer (uint32 words straddled by the
    codes), fp16 scales, and gpt-oss-style MXFP4 experts with per-output biases under
    `.mlp.experts.`; the bytes still match the blob and dequantize to the same weights."""
    cfg = {"model_type": "qwen3_moe", "num_experts_per_tok": 2,
           "quantization": {"group_size": 64, "bits": 4,
                            "model.layers.1.mlp.switch_mlp.gate_proj": {"group_size": 64, "bits": 3}}}
    d = str(tmp_path / "m3")
    made = make_checkpoint(d, {0: (128, 64, 3, Q4F16, False), 1: (128, 64, 3, Q3, False)}, config=cfg)
    blob, bm = _pack(tmp_path, made)
    cm = CK.expert_manifest(d)
    assert cm.layers["1"]["quant"] == {"bits": 3, "group_size": 64, "mode": "affine"}
    assert cm.quant(0).scale_dtype == "float16" and cm.quant(1).bits == 3
    raw = np.fromfile(blob, dtype=np.uint8)
    for li in (0, 1):
        for e in range(3):
            o, n = bm.region(li, e)
            got = CK.read_expert(cm, li, e)
            assert got == raw[o:o + n].tobytes()
            spec, q, experts = made[li]
            w = F.dequantize_projection(F.split_expert(got, spec), "down_proj", cm.quant(li))
            w0 = F.dequantize_projection(F.split_expert(experts[e], spec), "down_proj", q)
            assert np.array_equal(w.view(np.uint32), w0.view(np.uint32))

    cfg = {"model_type": "gpt_oss", "num_experts_per_tok": 4, "swiglu_limit": 7.0,
           "quantization": {"group_size": 32, "bits": 4, "mode": "mxfp4"}}
    d = str(tmp_path / "gptoss")
    made = make_checkpoint(d, {0: (128, 64, 4, MX, True)}, infix=".mlp.experts.", config=cfg, shards=1)
    blob, bm = _pack(tmp_path, made, top_k=4)
    cm = CK.expert_manifest(d)
    raw = np.fromfile(blob, dtype=np.uint8)
    for e in range(4):
        o, n = bm.region(0, e)
        assert CK.read_expert(cm, 0, e) == raw[o:o + n].tobytes()
    spec = CK.layer_spec(cm, 0)
    assert (spec.hidden, spec.inter, spec.n_experts, spec.top_k) == (128, 64, 4, 4)
    assert spec.quant.mode == "mxfp4" and spec.has_bias
    assert spec.route == "topk_softmax" and spec.act == "swiglu_clamped" and spec.limit == 7.0


def test_layer_spec_and_routing_from_config(tmp_path):
    d = str(tmp_path / "q")
    make_checkpoint(d, {0: (256, 128, 8, Q4, False)})
    cm = CK.expert_manifest(d)
    s = CK.layer_spec(cm, 0)
    assert (s.hidden, s.inter, s.n_experts, s.top_k) == (256, 128, 8, 2)
    assert s.route == "softmax_topk_renorm" and s.act == "swiglu" and not s.has_bias
    assert s.bytes_per_expert == cm.layers["0"]["bytes_per_expert"]
    assert CK.layer_spec(cm, 0, top_k=4).top_k == 4
    assert CK.routing_from_config({"norm_topk_prob": False})["route"] == "softmax_topk"


def test_routing_rule_follows_the_adapter():
    """adapter.py:75-93: the named score function wins; with none named, expert groups mean
    sigmoid; groups make the selection group-limited; norm_topk_prob renormalises;
    routed_scaling_factor scales the weights."""
    r = CK.routing_from_config({"scoring_func": "sigmoid", "n_group": 8, "topk_group": 4,
                                "norm_topk_prob": True, "routed_scaling_factor": 2.5})
    assert r == {"route": "sigmoid_topk_renorm", "act": "swiglu", "n_group": 8, "topk_group": 4,
                 "route_scale": 2.5}
    assert CK.routing_from_config({"n_group": 8, "topk_group": 3})["route"] == "sigmoid_topk"
    v2 = CK.routing_from_config({"scoring_func": "softmax", "n_group": 8, "topk_group": 3,
                                 "routed_scaling_factor": 16.0})
    assert v2["route"] == "softmax_topk" and v2["n_group"] == 8 and v2["route_scale"] == 16.0
    assert CK.routing_from_config({"score_function": "sigmoid"})["route"] == "sigmoid_topk"
    assert "n_group" not in CK.routing_from_config({"norm_topk_prob": True})
    spec = small(QWEN3_30B_A3B, n_experts=256, **{k: v for k, v in r.items() if k != "act"})
    assert (spec.route_mode, spec.n_group, spec.topk_group, spec.route_scale) == (4, 8, 4, 2.5)
    d = spec.desc()
    assert (d.route_mode, d.n_group, d.topk_group, d.route_scale) == (4, 8, 4, 2.5)
    with pytest.raises(ValueError, match="group-limited"):
        small(QWEN3_30B_A3B, n_experts=256, top_k=8, n_group=8, topk_group=0)
    with pytest.raises(ValueError, match="group-limited"):
        small(QWEN3_30B_A3B, n_experts=100, n_group=8, topk_group=2)


def test_unquantized_checkpoint_layer(tmp_path):
    """A bf16 checkpoint (expert weights with no scales, config.json with or without a
    quantization block): the layer is unquantized, its shape comes from the bf16 weight and each
    expert reads back as the bytes a blob holds."""
    q = F.QuantSpec(16, 0, "none")
    for cfg in ({"model_type": "qwen3_moe", "num_experts_per_tok": 2},
                {"model_type": "qwen3_moe", "num_experts_per_tok": 2, "quantization": {"bits": 4, "group_size": 64}}):
        d = str(tmp_path / f"bf16_{len(cfg)}")
        made = make_checkpoint(d, {0: (256, 128, 4, q, False)}, config=cfg, seed=3)
        man = CK.expert_manifest(d)
        spec = CK.layer_spec(man, 0)
        assert spec.quant == q and (spec.hidden, spec.inter, spec.n_experts) == (256, 128, 4)
        assert spec.bytes_per_expert == 3 * 256 * 128 * 2
        for e in range(4):
            assert CK.read_expert(man, 0, e) == made[0][2][e]


def test_quantisation_is_decided_by_the_tensors(tmp_path):
    spec = {"gate_proj": {"weight": {}}}
    assert CK.quant_for({"quantization": {"bits": 4, "group_size": 64}}, "x", spec) == {}
    spec = {"gate_proj": {"weight": {}, "scales": {}}}
    assert CK.quant_for({}, "x", spec) == {}
    assert CK.quant_for({"quantization": {"bits": 8}}, "x", spec) == {
        "bits": 8, "group_size": 64, "mode": "affine"}
    assert CK.quant_for({"quantization_config": {"x": {"bits": 2, "group_size": 32}}}, "x", spec) == {
        "bits": 2, "group_size": 32, "mode": "affine"}


def test_reader_agrees_with_an_independent_safetensors_writer(tmp_path):
    """A file written by the safetensors library itself: offsets, dtypes and shapes read here
    address exactly the bytes it stored (bf16 and uint8 tensors)."""
    torch = pytest.importorskip("torch")
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(0)
    a = torch.randn((3, 5, 16), generator=g).to(torch.bfloat16)
    b = torch.randint(0, 255, (3, 7), generator=g, dtype=torch.uint8)
    d = tmp_path / "st"
    d.mkdir()
    save_file({"model.layers.0.mlp.switch_mlp.gate_proj.scales": a, "other.b": b},
              str(d / "model.safetensors"))
    t = CK.scan(str(d))
    ta = t["model.layers.0.mlp.switch_mlp.gate_proj.scales"]
    assert ta.dtype == "BF16" and ta.shape == (3, 5, 16) and ta.nbytes == a.numel() * 2
    with open(ta.path, "rb") as f:
        f.seek(ta.offset)
        assert f.read(ta.nbytes) == a.view(torch.int16).numpy().tobytes()
    tb = t["other.b"]
    with open(tb.path, "rb") as f:
        f.seek(tb.offset)
        assert f.read(tb.nbytes) == b.numpy().tobytes()


# ------------------------------------------------------------------ malformed input
def _one(tmp_path, name, payload) -> str:
    d = tmp_path / name
    d.mkdir()
    p = d / "x.safetensors"
    p.write_bytes(payload)
    return str(p)


def test_parser_refuses_nonsense(tmp_path):
    with pytest.raises(ValueError, match="too short"):
        CK.read_header(_one(tmp_path, "short", b"\x01\x02"))
    with pytest.raises(ValueError, match="implausible"):
        CK.read_header(_one(tmp_path, "huge", struct.pack("<Q", 1 << 40) + b"{}"))
    with pytest.raises(ValueError, match="cut short"):
        CK.read_header(_one(tmp_path, "cut", struct.pack("<Q", 64) + b"{}"))
    with pytest.raises(ValueError, match="not an object"):
        CK.read_header(_one(tmp_path, "list", struct.pack("<Q", 2) + b"[]"))
    hdr = json.dumps({"t": {"dtype": "F16", "shape": [4, 8], "data_offsets": [0, 999999]}}).encode()
    p = _one(tmp_path, "past", struct.pack("<Q", len(hdr)) + hdr + b"\x00" * 16)
    with pytest.raises(ValueError, match="past the file"):
        CK.scan(os.path.dirname(p))
    with pytest.raises(FileNotFoundError):
        CK.expert_manifest(str(tmp_path / "no-such-model"))


def test_checkpoint_errors_name_the_problem(tmp_path):
    # a dense model: no expert tensors at all
    d = tmp_path / "dense"
    d.mkdir()
    write_safetensors(str(d / "model.safetensors"),
                      {"model.layers.0.self_attn.q_proj.weight": ("F16", (2, 2), bytes(8))})
    (d / "config.json").write_text("{}")
    with pytest.raises(ValueError, match="no MoE expert tensors"):
        CK.expert_manifest(str(d))
    # an expert layout that is neither gated nor fc1/fc2 is recognised as MoE and refused by name
    d = tmp_path / "odd"
    d.mkdir()
    write_safetensors(str(d / "model.safetensors"),
                      {"model.layers.0.mlp.switch_mlp.w_in.weight": ("U32", (2, 4, 4), bytes(128))})
    (d / "config.json").write_text("{}")
    with pytest.raises(ValueError, match="w_in"):
        CK.expert_manifest(str(d))
    # siblings disagreeing on the expert count
    d = str(tmp_path / "mism")
    make_checkpoint(d, {0: (128, 64, 4, Q4, False)}, shards=1, extra=False)
    p = os.path.join(d, "model-00000-of-00001.safetensors")
    hdr, base = CK.read_header(p)
    data = open(p, "rb").read()[base:]
    name = "model.layers.0.mlp.switch_mlp.up_proj.biases"
    ent = hdr[name]
    a, b = ent["data_offsets"]
    tens = {}
    for nm, e in hdr.items():
        if nm == "__metadata__":
            continue
        lo, hi = e["data_offsets"]
        raw = data[lo:hi]
        shape = list(e["shape"])
        if nm == name:
            shape[0] = 3
            raw = raw[:len(raw) * 3 // 4]
        tens[nm] = (e["dtype"], shape, raw)
    os.remove(p)
    write_safetensors(p, tens)
    with pytest.raises(ValueError, match="3 experts but a sibling has 4"):
        CK.expert_manifest(d)
    # a layer missing a projection
    d = str(tmp_path / "missing")
    make_checkpoint(d, {0: (128, 64, 2, Q4, False)}, shards=1, extra=False)
    p = os.path.join(d, "model-00000-of-00001.safetensors")
    hdr, base = CK.read_header(p)
    data = open(p, "rb").read()[base:]
    tens = {nm: (e["dtype"], e["shape"], data[e["data_offsets"][0]:e["data_offsets"][1]])
            for nm, e in hdr.items() if nm != "__metadata__" and ".down_proj." not in nm}
    os.remove(p)
    write_safetensors(p, tens)
    with pytest.raises(ValueError, match="missing down_proj"):
        CK.expert_manifest(d)
    # header and data disagreeing on a tensor's size
    d = str(tmp_path / "size")
    make_checkpoint(d, {0: (128, 64, 2, Q4, False)}, shards=1, extra=False)
    p = os.path.join(d, "model-00000-of-00001.safetensors")
    hdr, base = CK.read_header(p)
    data = open(p, "rb").read()[base:]
    tens = {}
    for nm, e in hdr.items():
        if nm == "__metadata__":
            continue
        raw = data[e["data_offsets"][0]:e["data_offsets"][1]]
        tens[nm] = (e["dtype"], e["shape"], raw[:-4] if nm.endswith("gate_proj.scales") else raw)
    os.remove(p)
    write_safetensors(p, tens)
    with pytest.raises(ValueError, match="header and the data disagree"):
        CK.expert_manifest(d)
    with pytest.raises(KeyError):
        CK.CheckpointManifest("x").expert_segments(9, 9)


def test_two_layer_experts_read_as_the_blob_holds_them(tmp_path):
    """fc1/fc2 experts (SwitchMLP): the reader describes them projection by projection as a
    packed blob lays them out, and layer_spec gives the two-layer activation."""
    d = str(tmp_path / "mlp")
    q = F.QuantSpec(4, 64, "affine", "bfloat16")
    layers = make_checkpoint(d, {0: (256, 128, 6, q, False, False), 3: (256, 128, 6, q, True, False)},
                             config={"num_experts_per_tok": 2})
    cm = CK.expert_manifest(d)
    for li, (spec, _, experts) in layers.items():
        assert list(cm.layers[str(li)]["spec"]) == ["fc1", "fc2"]
        for e in range(6):
            assert CK.read_expert(cm, li, e) == experts[e]
    s = CK.layer_spec(cm, 0)
    assert s.act == "silu_mlp" and (s.hidden, s.inter, s.top_k) == (256, 128, 2)
    assert s.bytes_per_expert == len(layers[0][2][0])
    assert CK.layer_spec(cm, 3).has_bias
