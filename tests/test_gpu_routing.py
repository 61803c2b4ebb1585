"""Sigmoid and group-limited routing on the GPU (the rule adapter.py:75-93 describes: sigmoid
scoring with a selection bias, group-limited top-k, normalisation, routed scaling): the router
kernel and the decode kernels' in-launch ranking give the oracle's indices bit for bit and its
weights to 1e-5, and whole blocks match the oracle's layer output."""
import numpy as np
import pytest

import oracle
from bigrig_amd import formats as F
from bigrig_amd import layer as ops
from bigrig_amd.spec import QWEN3_30B_A3B
from tests.gpu_util import bits, build_gpu_layer, to_dev_bits
from tests.helpers import make_layer, make_x, small

pytestmark = pytest.mark.gpu

RULES = {
    # DeepSeek-V3 routing: 256 experts in 8 groups, 4 kept, sigmoid + bias, renormalised, x2.5
    "v3-e256": small(QWEN3_30B_A3B, n_experts=256, top_k=8, route="sigmoid_topk_renorm",
                     n_group=8, topk_group=4, route_scale=2.5),
    "sigmoid-e128": small(QWEN3_30B_A3B, n_experts=128, top_k=8, route="sigmoid_topk"),
    "softmax-groups-e64": small(QWEN3_30B_A3B, n_experts=64, top_k=6, route="softmax_topk",
                                n_group=8, topk_group=3, route_scale=16.0),
    "renorm-groups-e160": small(QWEN3_30B_A3B, n_experts=160, top_k=6,
                                route="softmax_topk_renorm", n_group=5, topk_group=2),
}


@pytest.mark.parametrize("name", list(RULES))
@pytest.mark.parametrize("T", [1, 8, 65, 300])
def test_rule_router_bit_exact(gpu, name, T):
    spec = RULES[name]
    rng = np.random.default_rng(T + 11)
    w = F.f32_to_bf16_bits(rng.standard_normal((spec.n_experts, spec.hidden),
                                               dtype=np.float32) * 0.02)
    bias = rng.standard_normal(spec.n_experts).astype(np.float32) * 0.05
    x = make_x(T, spec.hidden, seed=T + 12)
    print(f"[routing] {name} T={T}", flush=True)
    idx, wt, _ = ops.router_topk(spec, to_dev_bits(x, gpu), to_dev_bits(w, gpu),
                                 to_dev_bits(bias, gpu))
    _, oidx, ow, _ = oracle.router(x, w, False, bias, spec.top_k, spec.route_mode,
                                   **spec.route_rule)
    assert np.array_equal(idx.cpu().numpy(), oidx)
    np.testing.assert_allclose(wt.cpu().numpy(), ow, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("name", ["v3-e256", "softmax-groups-e64", "sigmoid-e128"])
@pytest.mark.parametrize("T", [1, 8, 40])
def test_rule_block(gpu, name, T):
    """Whole blocks: T <= 8 ranks inside the decode kernel, 40 routes first and runs the
    grouped GEMM; indices bit-exact, output within 1e-2 of the oracle, and the same bits
    through the separate router and operator."""
    import torch
    spec = small(RULES[name], hidden=512, inter=256)
    lay = make_layer(spec, seed=801, zipf=0.05)
    _, sw, pool, _ = build_gpu_layer(lay, gpu)
    pool.g2s_device(torch.cuda.current_stream().cuda_stream)
    x = make_x(T, spec.hidden, seed=8010 + T)
    xd = to_dev_bits(x, gpu)
    router = to_dev_bits(lay.router, gpu)
    bias = to_dev_bits(lay.bias, gpu)
    gi = torch.full((T, spec.top_k), -1, dtype=torch.int32, device=gpu)
    gw = torch.zeros((T, spec.top_k), dtype=torch.float32, device=gpu)
    print(f"[routing block] {name} T={T}", flush=True)
    out = ops.moe_block(spec, pool, xd, router, bias, None, None, out_idx=gi, out_w=gw,
                        flags=ops.path_flag(T, spec.top_k))
    torch.cuda.synchronize()
    _, idx, w, _ = oracle.router(x, lay.router, False, lay.bias, spec.top_k, spec.route_mode,
                                 **spec.route_rule)
    assert np.array_equal(gi.cpu().numpy(), idx)
    np.testing.assert_allclose(gw.cpu().numpy(), w, rtol=1e-5, atol=1e-7)
    ref, _ = oracle.moe_forward(spec, lay.experts, x, idx, w)
    assert oracle.rel_l2(F.bf16_bits_to_f32(bits(out)), F.bf16_bits_to_f32(ref)) < 1e-2
    moe = ops.MoELayer(spec, router, sw, router_bias=bias)
    sw._sync_free = False
    out2 = moe(xd)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out2), bits(out))
    pool.close()
