"""libbrx.so without a GPU: it loads, exports every entry point include/brx.h declares, and
its host-side validation and layout arithmetic behave (no kernel is launched here)."""
import ctypes as C
import os
import re

import pytest

from bigrig_amd import formats as F
from bigrig_amd import lib as L
from bigrig_amd.spec import E256_SHARED, GPT_OSS_120B, OLMOE_1B_7B, QWEN3_30B_A3B, QWEN3_30B_A3B_BF16

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "brx.h")
SPECS = [OLMOE_1B_7B, QWEN3_30B_A3B, E256_SHARED, GPT_OSS_120B, QWEN3_30B_A3B_BF16]


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(brx_\w+)\s*\(", src, flags=re.M)))


def test_header_declarations_match_binding():
    names = _declared()
    assert len(names) >= 19
    assert sorted(L.EXPORTS) == names
    assert set(L._SIGS) == set(names)


def test_library_loads_and_exports_every_symbol():
    lib = L.load()
    raw = C.CDLL(L.LIB)
    for name in _declared():
        assert hasattr(raw, name), name
    assert lib.brx_abi_version() == L.ABI_VERSION == 2
    src = open(HEADER).read()
    assert int(re.search(r"#define BRX_ABI_VERSION (\d+)", src).group(1)) == L.ABI_VERSION


def test_header_enums_match_binding():
    src = open(HEADER).read()
    for cname, val in (("BRX_EINVAL", L.BRX_EINVAL), ("BRX_ESTATE", L.BRX_ESTATE),
                       ("BRX_ERANGE", L.BRX_ERANGE), ("BRX_QUANT_MXFP4", L.QUANT_MXFP4),
                       ("BRX_ACT_SWIGLU_CLAMPED", L.ACT_SWIGLU_CLAMPED),
                       ("BRX_ROUTE_TOPK_SOFTMAX", L.ROUTE_TOPK_SOFTMAX),
                       ("BRX_ROUTE_SIGMOID_TOPK_RENORM", L.ROUTE_SIGMOID_TOPK_RENORM),
                       ("BRX_DT_BF16", L.DT_BF16),
                       ("BRX_FWD_FORCE_PREFILL", L.FWD_FORCE_PREFILL),
                       ("BRX_FWD_PHASE_B", L.FWD_PHASE_B), ("BRX_FWD_PHASE_R", L.FWD_PHASE_R)):
        m = re.search(rf"\b{cname}\s*=\s*(-?\d+)", src) or \
            re.search(rf"#define {cname}\s+\(?(-?\d+)u?", src)
        assert m, cname
        assert int(m.group(1)) == val, cname
    assert C.sizeof(L.LayerDesc) == 80 and C.sizeof(L.ExpertLayout) == 13 * 8


@pytest.mark.parametrize("spec", SPECS, ids=lambda s: f"H{s.hidden}I{s.inter}{s.quant.mode}")
def test_expert_layout_matches_formats(spec):
    lib = L.load()
    d = spec.desc()
    out = L.ExpertLayout()
    L.check(lib.brx_expert_layout_get(C.byref(d), 0, C.byref(out)))
    es = spec.expert_spec()
    offs = F.spec_offsets(es)
    assert out.bytes_per_expert == F.spec_bytes(es) == spec.bytes_per_expert
    for p, proj in enumerate(F.PROJECTIONS):
        assert out.weight[p] == offs[(proj, "weight")]
        assert out.scales[p] == offs.get((proj, "scales"), -1)
        assert out.biases[p] == offs.get((proj, "biases"), -1)
        assert out.bias[p] == offs.get((proj, "bias"), -1)
    if spec.shared_inter:
        L.check(lib.brx_expert_layout_get(C.byref(d), 1, C.byref(out)))
        assert out.bytes_per_expert == F.spec_bytes(spec.expert_spec(True))
    else:
        assert lib.brx_expert_layout_get(C.byref(d), 1, C.byref(out)) == L.BRX_EINVAL


BAD = [("hidden", 100, "hidden"), ("inter", 0, "inter"), ("n_experts", 513, "n_experts"),
       ("top_k", 0, "top_k"), ("bits", 5, "affine"), ("bits", 7, "affine"), ("group_size", 32, "affine"),
       ("group_size", 256, "affine"),
       ("quant_mode", 7, "quant_mode"), ("act", 5, "act"), ("route_mode", 5, "route_mode"),
       ("n_group", 65, "n_group"), ("n_group", 3, "divide"), ("n_group", 4, "topk_group 0 outside"),
       ("route_scale", -1.0, "route_scale"), ("router_dtype", 9, "router_dtype"), ("shared_inter", 96, "shared_inter"),
       ("hidden", 8256, "at most 8192"), ("inter", 8256, "at most 8192"),
       ("shared_inter", 8256, "at most 8192")]


@pytest.mark.parametrize("field,value,msg", BAD, ids=[f"{b[0]}={b[1]}" for b in BAD])
def test_descriptor_validation(field, value, msg):
    """Every entry point validates the descriptor before anything touches the device."""
    lib = L.load()
    d = QWEN3_30B_A3B.desc()
    setattr(d, field, value)
    out = L.ExpertLayout()
    assert lib.brx_expert_layout_get(C.byref(d), 0, C.byref(out)) == L.BRX_EINVAL
    assert msg in lib.brx_last_error().decode()
    assert lib.brx_router_topk(C.byref(d), None, None, None, None, 1, None, None, None,
                               None) == L.BRX_EINVAL
    assert lib.brx_sort_pairs(C.byref(d), None, 1, None, None, None) == L.BRX_EINVAL
    h = C.c_void_p()
    assert lib.brx_pool_create(C.byref(d), 4, C.byref(h)) == L.BRX_EINVAL and not h.value


# the reference's per-layer precision candidates (bigrig_engine/precision.py:58), plus 6- and
# 8-bit at group 128 (MLX writes those too)
WIDTHS = [(2, 128), (2, 64), (3, 128), (3, 64), (4, 128), (4, 64), (6, 64), (8, 64), (6, 128), (8, 128)]


@pytest.mark.parametrize("bits,group", WIDTHS, ids=[f"{b}bit-g{g}" for b, g in WIDTHS])
def test_every_affine_width_is_accepted_with_the_packed_layout(bits, group):
    """Each width validates and its expert layout is the one formats packs (weight words of
    32 / bits codes or byte-aligned runs, then K / group scales and biases per row)."""
    from dataclasses import replace
    lib = L.load()
    for fp16 in (False, True):
        spec = replace(QWEN3_30B_A3B, quant=F.QuantSpec(bits, group, "affine", "float16" if fp16 else "bfloat16"))
        d = spec.desc()
        out = L.ExpertLayout()
        L.check(lib.brx_expert_layout_get(C.byref(d), 0, C.byref(out)))
        offs = F.spec_offsets(spec.expert_spec())
        assert out.bytes_per_expert == F.spec_bytes(spec.expert_spec())
        for p, proj in enumerate(F.PROJECTIONS):
            assert out.weight[p] == offs[(proj, "weight")]
            assert out.scales[p] == offs[(proj, "scales")]
            assert out.biases[p] == offs[(proj, "biases")]


def test_unquantized_descriptor_rules():
    """Unquantized experts are bf16 with no scale groups: bits 16 and group_size 0, nothing else."""
    lib = L.load()
    out = L.ExpertLayout()
    d = QWEN3_30B_A3B_BF16.desc()
    assert (d.quant_mode, d.bits, d.group_size) == (L.QUANT_NONE, 16, 0)
    L.check(lib.brx_expert_layout_get(C.byref(d), 0, C.byref(out)))
    assert out.bytes_per_expert == 3 * 2048 * 768 * 2 and out.scales[0] == out.biases[0] == -1
    for field, value in (("bits", 4), ("group_size", 64)):
        d = QWEN3_30B_A3B_BF16.desc()
        setattr(d, field, value)
        assert lib.brx_expert_layout_get(C.byref(d), 0, C.byref(out)) == L.BRX_EINVAL
        assert "unquantized experts are bf16" in lib.brx_last_error().decode()


def test_group_of_128_needs_widths_it_divides():
    lib = L.load()
    for field in ("hidden", "inter", "shared_inter"):
        d = E256_SHARED.desc()
        d.group_size = 128
        setattr(d, field, 704)          # a multiple of 64, not of 128
        out = L.ExpertLayout()
        assert lib.brx_expert_layout_get(C.byref(d), 0, C.byref(out)) == L.BRX_EINVAL
        assert "multiples of the group size" in lib.brx_last_error().decode()


def test_calls_before_init_fail_cleanly():
    lib = L.load()
    d = QWEN3_30B_A3B.desc()
    assert lib.brx_router_topk(C.byref(d), None, None, None, None, 1, None, None, None,
                               None) == L.BRX_ESTATE
    assert "brx_init" in lib.brx_last_error().decode()
    assert lib.brx_pool_destroy(None) == L.BRX_OK          # like free(NULL)
    assert lib.brx_pool_capacity(None) < 0
    with pytest.raises(L.BrxError):
        L.check(lib.brx_pool_sync(None))


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        L.load(str(tmp_path / "nope.so"))


def test_shared_expert_width_is_independent_of_the_routed_width():
    """A shared expert wider than the routed ones (a different shared intermediate) is a layout
    of its own, equal to what formats packs."""
    from dataclasses import replace
    lib = L.load()
    for sh in (256, 1024, 1536):
        spec = replace(E256_SHARED, shared_inter=sh)
        d = spec.desc()
        out = L.ExpertLayout()
        L.check(lib.brx_expert_layout_get(C.byref(d), 1, C.byref(out)))
        assert out.bytes_per_expert == F.spec_bytes(spec.expert_spec(True))
        L.check(lib.brx_expert_layout_get(C.byref(d), 0, C.byref(out)))
        assert out.bytes_per_expert == spec.bytes_per_expert


def test_layer_spec_refuses_widths_the_kernels_do_not_take():
    from dataclasses import replace
    for kw in ({"hidden": 8256}, {"inter": 100}, {"shared_inter": 96}, {"hidden": 0}):
        with pytest.raises(ValueError):
            replace(QWEN3_30B_A3B, **kw)
    assert replace(QWEN3_30B_A3B, hidden=8192).hidden == 8192


def test_two_layer_expert_layout_matches_formats():
    """act BRX_ACT_SILU_MLP: fc1 in slot 0, fc2 in slot 2, slot 1 absent -- the offsets of the
    fc1/fc2 blob layout."""
    from dataclasses import replace
    lib = L.load()
    for base in (QWEN3_30B_A3B, GPT_OSS_120B):
        spec = replace(base, act="silu_mlp")
        d = spec.desc()
        out = L.ExpertLayout()
        L.check(lib.brx_expert_layout_get(C.byref(d), 0, C.byref(out)))
        es = spec.expert_spec()
        offs = F.spec_offsets(es)
        assert list(es) == ["fc1", "fc2"] and out.bytes_per_expert == F.spec_bytes(es)
        for slot, proj in ((0, "fc1"), (2, "fc2")):
            assert out.weight[slot] == offs[(proj, "weight")]
            assert out.scales[slot] == offs[(proj, "scales")]
            assert out.biases[slot] == offs.get((proj, "biases"), -1)
            assert out.bias[slot] == offs.get((proj, "bias"), -1)
        assert out.weight[1] == out.scales[1] == out.biases[1] == out.bias[1] == -1
