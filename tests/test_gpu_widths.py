"""Affine code widths besides 3- and 4-bit at group 64: the reference's per-layer precision
candidates (bigrig_engine/precision.py:58: 2, 3 and 4 bits at groups of 128, 2 bits at 64, 6 and
8 bits at 64) and 6/8 bits at 128, which MLX checkpoints also use. requantize_blob writes such
layers and records `quant` per layer (precision.py:136-229, 219); the streaming path takes that
record as the authority (stream.py:1876-1881).

For each width: every projection dequantized bit-exact by the hook (fp32, bf16 and fp16
scales); decode and prefill layers against the oracle and the float64 truth; the whole block with
its routing bit-exact and the same bits as router + operator; and a stack of layers of mixed
widths, each served by a bounded pool with misses refilled from pinned host memory, against the
oracle layer by layer and bit-identical to full residency."""
import numpy as np
import pytest

import oracle
from bigrig_amd import formats as F
from bigrig_amd import layer as ops
from bigrig_amd.spec import QWEN3_30B_A3B
from tests.gpu_util import bits, build_gpu_layer, bytes_dev, to_dev_bits
from tests.helpers import make_layer, make_x, small

pytestmark = pytest.mark.gpu

TOL = 1e-2
WIDTHS = [(2, 128), (2, 64), (3, 128), (4, 128), (6, 64), (8, 64), (6, 128), (8, 128)]
WIDS = [f"{b}bit-g{g}" for b, g in WIDTHS]


def _spec(bits_, group, scale="bfloat16", **kw):
    # inter 320 leaves a partial 128-feature prefill tile; groups of 128 need a multiple of 128
    kw.setdefault("inter", 320 if group == 64 else 384)
    return small(QWEN3_30B_A3B, hidden=512, n_experts=16, top_k=4,
                 quant=F.QuantSpec(bits_, group, "affine", scale), **kw)


@pytest.mark.parametrize("scale", ["bfloat16", "float16"])
@pytest.mark.parametrize("bits_,group", WIDTHS, ids=WIDS)
def test_width_dequant_bit_exact(gpu, bits_, group, scale):
    spec = _spec(bits_, group, scale)
    lay = make_layer(spec, seed=800 + bits_)
    for e in (0, spec.n_experts - 1):
        dev = bytes_dev(lay.experts[e], gpu)
        for p in range(3):
            got = ops.dequant(spec, dev, p).cpu().numpy()
            want = oracle.dequant(spec, lay.experts[e], p)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (e, p)


def _check(lay, moe, T, seed, f64=True):
    import torch
    spec = lay.spec
    x = make_x(T, spec.hidden, seed=seed)
    out = moe(to_dev_bits(x, moe.router_w.device))
    torch.cuda.synchronize()
    _, idx, w, sg = oracle.router(x, lay.router, spec.router_dtype == "float32", lay.bias,
                                  spec.top_k, spec.route_mode, lay.sgate_w)
    ref, _ = oracle.moe_forward(spec, lay.experts, x, idx, w, lay.shared, sg)
    got = F.bf16_bits_to_f32(bits(out))
    r = oracle.rel_l2(got, F.bf16_bits_to_f32(ref))
    assert r < TOL, f"rel L2 vs C oracle {r:.3e}"
    if f64:
        truth, _ = oracle.moe_forward_f64(spec, lay.experts, x, idx, w, lay.shared, sg)
        assert oracle.rel_l2(got, truth) < TOL
    return bits(out)


@pytest.mark.parametrize("bits_,group", WIDTHS, ids=WIDS)
@pytest.mark.parametrize("T", [1, 3, 8, 9, 64, 300])
def test_width_layer(gpu, bits_, group, T):
    """Decode (1-8 tokens: one-token, one-launch and per-entry kernels) and prefill (9+)."""
    spec = _spec(bits_, group)
    lay = make_layer(spec, seed=810 + bits_, zipf=0.9)
    moe, _, pool, _ = build_gpu_layer(lay, gpu)
    print(f"[widths] layer {bits_}-bit g{group} T={T}", flush=True)
    _check(lay, moe, T, seed=8100 + T, f64=T <= 64)
    pool.close()


@pytest.mark.parametrize("bits_,group", [(2, 128), (6, 64), (8, 64)], ids=["2bit-g128", "6bit-g64", "8bit-g64"])
@pytest.mark.parametrize("T", [1, 8, 40])
def test_width_block(gpu, bits_, group, T):
    """The whole block with fp16 scales and a shared expert: routing bit-exact, output within
    tolerance, and the same bits as router + operator through the separate entry points."""
    import torch
    spec = _spec(bits_, group, "float16", shared_inter=256 if group == 64 else 384)
    lay = make_layer(spec, seed=820 + bits_, zipf=0.9)
    _, sw, pool, _ = build_gpu_layer(lay, gpu)
    pool.g2s_device(torch.cuda.current_stream().cuda_stream)
    x = make_x(T, spec.hidden, seed=8200 + T)
    xd = to_dev_bits(x, gpu)
    router = to_dev_bits(lay.router, gpu)
    bias = None if lay.bias is None else to_dev_bits(lay.bias, gpu)
    sgw = to_dev_bits(lay.sgate_w, gpu)
    print(f"[widths] block {bits_}-bit g{group} T={T}", flush=True)
    gi = torch.full((T, spec.top_k), -1, dtype=torch.int32, device=gpu)
    out = ops.moe_block(spec, pool, xd, router, bias, sgw, sw.shared, out_idx=gi,
                        flags=ops.path_flag(T, spec.top_k))
    torch.cuda.synchronize()
    _, idx, w, sg = oracle.router(x, lay.router, False, lay.bias, spec.top_k, spec.route_mode,
                                  lay.sgate_w)
    assert np.array_equal(gi.cpu().numpy(), idx)
    ref, _ = oracle.moe_forward(spec, lay.experts, x, idx, w, lay.shared, sg)
    assert oracle.rel_l2(F.bf16_bits_to_f32(bits(out)), F.bf16_bits_to_f32(ref)) < TOL
    moe = ops.MoELayer(spec, router, sw, router_bias=bias, shared_gate_w=sgw)
    sw._sync_free = False
    out2 = moe(xd)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out2), bits(out))
    pool.close()


# a requantized stack: every layer at its own width (precision.py:219), the same shape
MIXED = [(2, 128), (4, 64), (8, 64), (3, 128), (6, 64), (4, 128), (2, 64)]


@pytest.mark.parametrize("T,C,steps", [(1, 6, 12), (40, 8, 3)], ids=["decode-C6", "prefill-C8"])
def test_mixed_width_stack_bounded_pool(gpu, T, C, steps):
    """Seven layers of different widths, each through a bounded pool of C of 16 slots with
    misses refilled from pinned host memory, a fresh input per layer and step: every layer's
    output within 1e-2 of the oracle on its own experts, and the same bits as with every expert
    resident."""
    import torch
    lays = [make_layer(_spec(b, g, inter=384), seed=830 + i, zipf=0.6) for i, (b, g) in enumerate(MIXED)]
    res = {}
    for cap in (16, C):
        built = [build_gpu_layer(lay, gpu, capacity=cap) for lay in lays]
        outs = []
        for step in range(steps):
            for li, (lay, (moe, _, pool, _)) in enumerate(zip(lays, built)):
                b_, g_ = MIXED[li]
                print(f"[widths] mixed C={cap} step {step} layer {li} ({b_}-bit g{g_}) T={T}", flush=True)
                x = make_x(T, 512, seed=8300 + 97 * step + li)
                out = moe(to_dev_bits(x, gpu))
                torch.cuda.synchronize()
                outs.append(bits(out))
                if cap == C:
                    _, idx, w, _ = oracle.router(x, lay.router, False, lay.bias, lay.spec.top_k,
                                                 lay.spec.route_mode)
                    ref, _ = oracle.moe_forward(lay.spec, lay.experts, x, idx, w)
                    r = oracle.rel_l2(F.bf16_bits_to_f32(outs[-1]), F.bf16_bits_to_f32(ref))
                    assert r < TOL, f"layer {li} ({b_}-bit g{g_}) step {step}: rel L2 {r:.3e}"
        if cap == C:
            assert sum(p.evicts for _, _, p, _ in built) > 0
        for _, _, pool, _ in built:
            pool.close()
        res[cap] = outs
    for i, (a, b) in enumerate(zip(res[16], res[C])):
        assert np.array_equal(a, b), f"call {i} differs between the bounded and resident pools"
