"""Unquantized bf16 experts (the mx.gather_mm branch of StreamingSwitchGLU._proj,
bigrig_engine/stream.py:1626-1628; layers whose tensors carry no scales, direct.py:110-142) on
the GPU: the dequant hook returns the weights bit for bit; decode and prefill layers against the
oracle and the float64 truth (a shared expert, biases, a two-layer expert, a partial feature
tile); the whole block with its routing bit-exact and the same bits as router + operator; a
bounded pool bit-identical to full residency; a bf16 checkpoint served through a bounded pool.
The full-size Qwen3-30B-A3B-bf16 layer runs in test_gpu_full_size.py."""
import numpy as np
import pytest

import oracle
from bigrig_amd import formats as F
from bigrig_amd import layer as ops
from bigrig_amd.spec import E256_SHARED, QWEN3_30B_A3B
from tests.gpu_util import bits, build_gpu_layer, bytes_dev, to_dev_bits
from tests.helpers import make_layer, make_x, small

pytestmark = pytest.mark.gpu

TOL = 1e-2
QN = F.QuantSpec(16, 0, "none")
SPECS = {
    "qwen3": small(QWEN3_30B_A3B, hidden=512, inter=320, n_experts=16, top_k=4, quant=QN),
    "shared-bias": small(E256_SHARED, hidden=576, inter=256, n_experts=16, top_k=4, shared_inter=384,
                         quant=QN, has_bias=True),
    "mlp": small(QWEN3_30B_A3B, hidden=512, inter=320, n_experts=16, top_k=4, quant=QN, act="silu_mlp"),
}


@pytest.mark.parametrize("name", list(SPECS))
def test_bf16_dequant_is_the_weights(gpu, name):
    spec = SPECS[name]
    lay = make_layer(spec, seed=850)
    for e in (0, spec.n_experts - 1):
        dev = bytes_dev(lay.experts[e], gpu)
        for p in (0, 2) if spec.act == "silu_mlp" else (0, 1, 2):
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


@pytest.mark.parametrize("name", list(SPECS))
@pytest.mark.parametrize("T", [1, 3, 8, 9, 64, 300])
def test_bf16_layer(gpu, name, T):
    spec = SPECS[name]
    lay = make_layer(spec, seed=860, zipf=0.9)
    moe, _, pool, _ = build_gpu_layer(lay, gpu)
    print(f"[bf16] layer {name} T={T}", flush=True)
    _check(lay, moe, T, seed=8600 + T, f64=T <= 64)
    pool.close()


@pytest.mark.parametrize("T", [1, 8, 40])
def test_bf16_block(gpu, T):
    """The whole block (routing ranked in the decode kernel): routing bit-exact, output within
    tolerance, and the same bits as router + operator through the separate entry points."""
    import torch
    spec = SPECS["shared-bias"]
    lay = make_layer(spec, seed=870, zipf=0.9)
    _, sw, pool, _ = build_gpu_layer(lay, gpu)
    pool.g2s_device(torch.cuda.current_stream().cuda_stream)
    x = make_x(T, spec.hidden, seed=8700 + T)
    xd = to_dev_bits(x, gpu)
    router = to_dev_bits(lay.router, gpu)
    bias = None if lay.bias is None else to_dev_bits(lay.bias, gpu)
    sgw = to_dev_bits(lay.sgate_w, gpu)
    print(f"[bf16] block T={T}", flush=True)
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


@pytest.mark.parametrize("T,C,steps", [(1, 6, 16), (40, 8, 3)], ids=["decode-C6", "spans-C8"])
def test_bf16_bounded_pool_bit_identical(gpu, T, C, steps):
    import torch
    spec = SPECS["qwen3"]
    lay = make_layer(spec, seed=880, zipf=0.8)
    xs = [make_x(T, spec.hidden, seed=8800 + i) for i in range(steps)]
    res = {}
    for cap in (spec.n_experts, C):
        moe, sw, pool, _ = build_gpu_layer(lay, gpu, capacity=cap)
        print(f"[bf16] bounded pool C={cap} T={T}", flush=True)
        outs = [moe(to_dev_bits(x, gpu)) for x in xs]
        torch.cuda.synchronize()
        res[cap] = [bits(o) for o in outs]
        if cap == C:
            assert pool.evicts > 0
        pool.close()
    for a, b in zip(res[spec.n_experts], res[C]):
        assert np.array_equal(a, b)


def test_bf16_checkpoint_bounded_pool(gpu, tmp_path):
    """A bf16 MLX checkpoint (weights without scales) read into the pinned host store and
    served by a 6-slot pool: routing bit-exact and outputs within 1e-2 of the oracle on the
    experts read back from the shards."""
    from bigrig_amd import checkpoint as CK
    from bigrig_amd.layer import MoELayer, StreamingSwitchGLU
    from bigrig_amd.pool import ExpertPool, HostStore, PinnedFetcher
    from tests.ckpt_util import make_checkpoint
    H, I, E, C = 512, 256, 16, 6
    cfg = {"model_type": "qwen3_moe", "num_experts_per_tok": 4, "norm_topk_prob": True}
    d = str(tmp_path / "ckpt_bf16")
    make_checkpoint(d, {0: (H, I, E, QN, False)}, config=cfg, shards=2, seed=9)
    man = CK.expert_manifest(d)
    spec = CK.layer_spec(man, 0)
    assert spec.quant == QN and spec.bytes_per_expert == 3 * H * I * 2
    store = HostStore.from_checkpoint(man)
    experts = [CK.read_expert(man, 0, e) for e in range(E)]
    rng = np.random.default_rng(19)
    router = F.f32_to_bf16_bits(rng.standard_normal((E, H), dtype=np.float32) * 0.02)
    pool = ExpertPool(0, spec, C).build()
    moe = MoELayer(spec, to_dev_bits(router, gpu), StreamingSwitchGLU(pool, PinnedFetcher(store)))
    for T in (1, 7, 40):
        print(f"[bf16 checkpoint] H={H} I={I} E={E} C={C} T={T}", flush=True)
        x = make_x(T, H, seed=410 + T)
        _, idx, w, _ = oracle.router(x, router, False, None, spec.top_k, spec.route_mode)
        out = moe(to_dev_bits(x, gpu))
        ref, _ = oracle.moe_forward(spec, experts, x, idx, w)
        r = oracle.rel_l2(F.bf16_bits_to_f32(bits(out)), F.bf16_bits_to_f32(ref))
        assert r < TOL, f"T={T}: rel L2 {r:.3e}"
    assert pool.admits > C
    pool.close()
