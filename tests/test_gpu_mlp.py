"""Plain two-layer experts (SwitchMLP, `fc2(silu(fc1 x))`, stream.py:1167-1169) on the GPU: fc1 /
fc2 dequantized bit-exact, decode and prefill layers against the oracle and the float64 truth
(affine and MXFP4 with biases, a shared two-layer expert of its own width, an intermediate width
that leaves a partial 256-feature tile), the whole block with routing bit-exact, and a bounded
pool bit-identical to full residency on the decode and span paths."""
import numpy as np
import pytest

import oracle
from bigrig_amd import formats as F
from bigrig_amd import layer as ops
from bigrig_amd.spec import E256_SHARED, GPT_OSS_120B, QWEN3_30B_A3B
from tests.gpu_util import bits, build_gpu_layer, bytes_dev, to_dev_bits
from tests.helpers import make_layer, make_x, small

pytestmark = pytest.mark.gpu

TOL = 1e-2

MLP_AFFINE = small(QWEN3_30B_A3B, hidden=512, inter=320, n_experts=32, top_k=8, act="silu_mlp")
MLP_MXFP4 = small(GPT_OSS_120B, hidden=576, inter=320, n_experts=16, top_k=4, act="silu_mlp")
MLP_SHARED = small(E256_SHARED, hidden=512, inter=256, n_experts=32, top_k=8, shared_inter=640,
                   act="silu_mlp")
SPECS = [MLP_AFFINE, MLP_MXFP4, MLP_SHARED]
IDS = ["affine", "mxfp4-bias", "shared"]


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


@pytest.mark.parametrize("spec", [MLP_AFFINE, MLP_MXFP4], ids=["affine", "mxfp4-bias"])
def test_fc1_fc2_dequant_bit_exact(gpu, spec):
    lay = make_layer(spec, seed=601)
    dev = bytes_dev(lay.experts[3], gpu)
    for p in (0, 2):
        got = ops.dequant(spec, dev, p).cpu().numpy()
        want = oracle.dequant(spec, lay.experts[3], p)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), p


@pytest.mark.parametrize("spec", SPECS, ids=IDS)
@pytest.mark.parametrize("T", [1, 3, 8, 9, 64, 300])
def test_two_layer_expert_layer(gpu, spec, T):
    lay = make_layer(spec, seed=602, zipf=0.9)
    moe, sw, pool, _ = build_gpu_layer(lay, gpu)
    print(f"[mlp] {spec.quant.mode} I={spec.inter} shared={spec.shared_inter} T={T}", flush=True)
    _check(lay, moe, T, seed=6020 + T, f64=T <= 64)
    pool.close()


@pytest.mark.parametrize("spec", SPECS, ids=IDS)
@pytest.mark.parametrize("T", [1, 8, 40])
def test_two_layer_block(gpu, spec, T):
    """The whole block (routing ranked in the decode kernel): routing bit-exact, output within
    tolerance, and the same bits as router + operator through the separate entry points."""
    import torch
    lay = make_layer(spec, seed=603, zipf=0.9)
    _, sw, pool, _ = build_gpu_layer(lay, gpu)
    pool.g2s_device(torch.cuda.current_stream().cuda_stream)
    x = make_x(T, spec.hidden, seed=6030 + T)
    xd = to_dev_bits(x, gpu)
    router = to_dev_bits(lay.router, gpu)
    bias = to_dev_bits(lay.bias, gpu)
    sgw = None if lay.sgate_w is None else to_dev_bits(lay.sgate_w, gpu)
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


@pytest.mark.parametrize("T,C,steps", [(1, 10, 24), (64, 12, 3)], ids=["decode-C10", "spans-C12"])
def test_two_layer_bounded_pool_bit_identical(gpu, T, C, steps):
    import torch
    spec = MLP_AFFINE
    lay = make_layer(spec, seed=604, zipf=0.8)
    xs = [make_x(T, spec.hidden, seed=6040 + i) for i in range(steps)]
    res = {}
    for cap in (spec.n_experts, C):
        moe, sw, pool, _ = build_gpu_layer(lay, gpu, capacity=cap)
        outs = [moe(to_dev_bits(x, gpu)) for x in xs]
        torch.cuda.synchronize()
        res[cap] = [bits(o) for o in outs]
        if cap == C:
            assert pool.evicts > 0
        pool.close()
    for a, b in zip(res[spec.n_experts], res[C]):
        assert np.array_equal(a, b)
