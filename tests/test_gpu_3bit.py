"""3-bit affine experts (group 64, 8 codes in 3 bytes, the layout of the shipped
Qwen3-30B-A3B-3bit blob: data/blobs/Qwen3-30B-A3B-3bit.experts.manifest.json) on the GPU:
every projection dequantized bit-exact against the oracle, decode and prefill layers against the
oracle and the float64 truth (bf16 and fp16 scales, a shared expert, an intermediate width that
leaves a partial feature tile), the whole block with routing bit-exact, a bounded pool
bit-identical to full residency, a 3-bit checkpoint served through a bounded pool, and the
full-size 128-expert layer at batch 1 and a 2048-token chunk."""
import numpy as np
import pytest

import oracle
from bigrig_amd import formats as F
from bigrig_amd import layer as ops
from bigrig_amd.spec import E256_SHARED, OLMOE_1B_7B, QWEN3_30B_A3B, QWEN3_30B_A3B_3BIT
from tests.gpu_util import (bits, build_gpu_layer, bytes_dev, per_token_rel_l2, tile_edge_tokens,
                            to_dev_bits)
from tests.helpers import make_layer, make_x, small

pytestmark = pytest.mark.gpu

TOL = 1e-2
Q3_BF16 = F.QuantSpec(3, 64, "affine", "bfloat16")
Q3_F16 = F.QuantSpec(3, 64, "affine", "float16")

Q3_QWEN = small(QWEN3_30B_A3B, hidden=512, inter=320, n_experts=32, top_k=8, quant=Q3_BF16)
Q3_OLMOE = small(OLMOE_1B_7B, hidden=640, inter=384, n_experts=16, top_k=8, quant=Q3_F16)
Q3_SHARED = small(E256_SHARED, hidden=512, inter=256, n_experts=32, top_k=8, shared_inter=576,
                  quant=Q3_BF16)
SPECS = [Q3_QWEN, Q3_OLMOE, Q3_SHARED]
IDS = ["qwen3-bf16", "olmoe-f16", "shared"]


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


@pytest.mark.parametrize("spec", [Q3_QWEN, Q3_OLMOE], ids=["bf16", "f16"])
def test_3bit_dequant_bit_exact(gpu, spec):
    lay = make_layer(spec, seed=701)
    for e in (0, 5):
        dev = bytes_dev(lay.experts[e], gpu)
        for p in range(3):
            got = ops.dequant(spec, dev, p).cpu().numpy()
            want = oracle.dequant(spec, lay.experts[e], p)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (e, p)


@pytest.mark.parametrize("spec", SPECS, ids=IDS)
@pytest.mark.parametrize("T", [1, 3, 8, 9, 64, 300])
def test_3bit_layer(gpu, spec, T):
    lay = make_layer(spec, seed=702, zipf=0.9)
    moe, sw, pool, _ = build_gpu_layer(lay, gpu)
    print(f"[3bit] {spec.quant.scale_dtype} H={spec.hidden} I={spec.inter} "
          f"shared={spec.shared_inter} T={T}", flush=True)
    _check(lay, moe, T, seed=7020 + T, f64=T <= 64)
    pool.close()


@pytest.mark.parametrize("spec", SPECS, ids=IDS)
@pytest.mark.parametrize("T", [1, 8, 40])
def test_3bit_block(gpu, spec, T):
    """The whole block (routing ranked in the decode kernel): routing bit-exact, output within
    tolerance, and the same bits as router + operator through the separate entry points."""
    import torch
    lay = make_layer(spec, seed=703, zipf=0.9)
    _, sw, pool, _ = build_gpu_layer(lay, gpu)
    pool.g2s_device(torch.cuda.current_stream().cuda_stream)
    x = make_x(T, spec.hidden, seed=7030 + T)
    xd = to_dev_bits(x, gpu)
    f32 = spec.router_dtype == "float32"
    router = to_dev_bits(lay.router, gpu)
    bias = None if lay.bias is None else to_dev_bits(lay.bias, gpu)
    sgw = None if lay.sgate_w is None else to_dev_bits(lay.sgate_w, gpu)
    gi = torch.full((T, spec.top_k), -1, dtype=torch.int32, device=gpu)
    out = ops.moe_block(spec, pool, xd, router, bias, sgw, sw.shared, out_idx=gi,
                        flags=ops.path_flag(T, spec.top_k))
    torch.cuda.synchronize()
    _, idx, w, sg = oracle.router(x, lay.router, f32, lay.bias, spec.top_k, spec.route_mode,
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
def test_3bit_bounded_pool_bit_identical(gpu, T, C, steps):
    import torch
    spec = Q3_QWEN
    lay = make_layer(spec, seed=704, zipf=0.8)
    xs = [make_x(T, spec.hidden, seed=7040 + i) for i in range(steps)]
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


def test_3bit_checkpoint_bounded_pool(gpu, tmp_path):
    """A 3-bit MLX checkpoint (uint32 words straddled by 3-bit codes) read into the pinned host
    store and served by a 6-slot pool: routing bit-exact and outputs within 1e-2 of the oracle on
    the experts read back from the shards."""
    from bigrig_amd import checkpoint as CK
    from bigrig_amd.layer import MoELayer, StreamingSwitchGLU
    from bigrig_amd.pool import ExpertPool, HostStore, PinnedFetcher
    from tests.ckpt_util import make_checkpoint
    H, I, E, C = 512, 256, 16, 6
    cfg = {"model_type": "qwen3_moe", "num_experts_per_tok": 4, "norm_topk_prob": True,
           "quantization": {"group_size": 64, "bits": 3}}
    d = str(tmp_path / "ckpt3")
    make_checkpoint(d, {0: (H, I, E, Q3_BF16, False)}, config=cfg, shards=2, seed=7)
    man = CK.expert_manifest(d)
    spec = CK.layer_spec(man, 0)
    assert spec.quant.bits == 3 and spec.bytes_per_expert == 3 * (I * H * 3 // 8 + I * H // 16)
    store = HostStore.from_checkpoint(man)
    experts = [CK.read_expert(man, 0, e) for e in range(E)]
    rng = np.random.default_rng(13)
    router = F.f32_to_bf16_bits(rng.standard_normal((E, H), dtype=np.float32) * 0.02)
    pool = ExpertPool(0, spec, C).build()
    moe = MoELayer(spec, to_dev_bits(router, gpu), StreamingSwitchGLU(pool, PinnedFetcher(store)))
    for T in (1, 7, 40):
        print(f"[3bit checkpoint] H={H} I={I} E={E} C={C} T={T}", flush=True)
        x = make_x(T, H, seed=310 + T)
        _, idx, w, _ = oracle.router(x, router, False, None, spec.top_k, spec.route_mode)
        out = moe(to_dev_bits(x, gpu))
        ref, _ = oracle.moe_forward(spec, experts, x, idx, w)
        r = oracle.rel_l2(F.bf16_bits_to_f32(bits(out)), F.bf16_bits_to_f32(ref))
        assert r < TOL, f"T={T}: rel L2 {r:.3e}"
    assert pool.admits > C
    pool.close()


@pytest.mark.parametrize("T", [1, 2048], ids=["decode1", "prefill2048"])
def test_3bit_full_size_layer(gpu, T):
    """The Qwen3-30B-A3B-3bit layer at full size (hidden 2048, 128 experts, top-8, inter 768,
    Zipf(1.1) router bias), every expert resident: outputs finite, the whole call's routing
    bit-exact, and the tokens of every expert's 64-row run edges (every M tile's first and last
    row) within 1e-2 of the oracle, as a whole and token by token."""
    import torch

    from bigrig_amd import synth
    from bigrig_amd.pool import ExpertPool
    spec = QWEN3_30B_A3B_3BIT
    print(f"[3bit full-size] T={T}", flush=True)
    experts = synth.make_layer_experts(spec, seed=720 + T)
    assert experts.shape[1] == spec.bytes_per_expert == 2064384
    pool = ExpertPool(0, spec, spec.n_experts).build()
    for e in range(spec.n_experts):
        pool.touch([e], [0])
        pool.admit_device(e, experts[e].data_ptr())
    pool.g2s_device(torch.cuda.current_stream().cuda_stream)
    pool.device.sync()
    wr = synth.router_weights(spec, seed=721 + T)
    bias = synth.zipf_bias_torch(spec.n_experts, 1.1, seed=722 + T)
    x = synth.activations(T, spec.hidden, seed=723 + T)
    idx = torch.empty((T, spec.top_k), dtype=torch.int32, device=gpu)
    w = torch.empty((T, spec.top_k), dtype=torch.float32, device=gpu)
    out = ops.moe_block(spec, pool, x, wr, bias, None, None, out_idx=idx, out_w=w,
                        flags=ops.path_flag(T, spec.top_k))
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out.float()).all())
    xb_all = bits(x)
    _, oidx_all, ow_all, _ = oracle.router(xb_all, bits(wr), False, bias.cpu().numpy(), spec.top_k,
                                           spec.route_mode)
    assert np.array_equal(idx.cpu().numpy(), oidx_all)
    np.testing.assert_allclose(w.cpu().numpy(), ow_all, rtol=1e-5, atol=1e-7)
    toks = tile_edge_tokens(oidx_all, spec.n_experts) if T > 8 else list(range(T))
    oidx, ow = oidx_all[toks], ow_all[toks]
    need = sorted(set(int(e) for e in oidx.reshape(-1)))
    host = {e: experts[e].cpu().numpy().tobytes() for e in need}
    elist = [host.get(e, host[need[0]]) for e in range(spec.n_experts)]
    ref, _ = oracle.moe_forward(spec, elist, xb_all[toks], oidx, ow)
    got = F.bf16_bits_to_f32(bits(out)[toks])
    want = F.bf16_bits_to_f32(ref)
    assert np.abs(want).max() > 1e-3
    r = oracle.rel_l2(got, want)
    rt = per_token_rel_l2(got, want)
    worst = int(np.argmax(rt))
    print(f"[3bit full-size] {len(toks)} tokens: rel L2 {r:.2e}, worst token {toks[worst]} "
          f"{rt[worst]:.2e}", flush=True)
    assert r < TOL
    assert rt[worst] < TOL
    pool.close()
    del experts
    torch.cuda.empty_cache()
