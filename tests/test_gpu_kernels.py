"""GPU parity of libbrx's kernels against the oracle (all calls go through the C-ABI).

Bars: dequantized weights bit-exact in fp32; routing indices bit-exact; routing weights to
1e-5 relative; layer outputs (fp32 accumulate, bf16 out) within 1e-2 relative L2 of the
oracle, which is the tolerance the layer is specified to. The float64 truth is checked too, so
the kernels and the C oracle cannot agree by being wrong the same way.
"""
import numpy as np
import pytest

import oracle
from bigrig_amd import formats as F
from bigrig_amd import layer as ops
from bigrig_amd.spec import E256_SHARED, GPT_OSS_120B, OLMOE_1B_7B, QWEN3_30B_A3B, LayerSpec
from tests.gpu_util import bits, build_gpu_layer, bytes_dev, to_dev_bits
from tests.helpers import make_layer, make_x, small

pytestmark = pytest.mark.gpu

TOL = 1e-2

SMALL_AFFINE = small(QWEN3_30B_A3B, hidden=512, inter=256, n_experts=32, top_k=8)
SMALL_F16 = small(OLMOE_1B_7B, hidden=512, inter=384, n_experts=16, top_k=4,
                  quant=F.QuantSpec(4, 64, "affine", "float16"))
SMALL_MXFP4 = small(GPT_OSS_120B, hidden=576, inter=320, n_experts=16, top_k=4)
SMALL_SHARED = small(E256_SHARED, hidden=512, inter=256, n_experts=64, top_k=8,
                     shared_inter=256)


@pytest.mark.parametrize("spec", [SMALL_AFFINE, SMALL_F16, SMALL_MXFP4], ids=["bf16", "f16", "mxfp4"])
def test_dequant_bit_exact(gpu, spec):
    lay = make_layer(spec, seed=3)
    for e in (0, spec.n_experts - 1):
        dev = bytes_dev(lay.experts[e], gpu)
        for p in range(3):
            got = ops.dequant(spec, dev, p).cpu().numpy()
            want = oracle.dequant(spec, lay.experts[e], p)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (e, p)


@pytest.mark.parametrize("spec", [OLMOE_1B_7B, QWEN3_30B_A3B, E256_SHARED, GPT_OSS_120B],
                         ids=["olmoe", "qwen3", "e256", "gptoss"])
@pytest.mark.parametrize("T", [1, 8, 65, 300])
def test_router_bit_exact(gpu, spec, T):
    rng = np.random.default_rng(T)
    wr = rng.standard_normal((spec.n_experts, spec.hidden), dtype=np.float32) * 0.02
    w = wr if spec.router_dtype == "float32" else F.f32_to_bf16_bits(wr)
    bias = (rng.standard_normal(spec.n_experts).astype(np.float32) if spec.n_experts != 64 else None)
    sgw = F.f32_to_bf16_bits(rng.standard_normal(spec.hidden, dtype=np.float32) * 0.02) \
        if spec.shared_inter else None
    x = make_x(T, spec.hidden, seed=T + 5)
    idx, wt, sg = ops.router_topk(spec, to_dev_bits(x, gpu), to_dev_bits(w, gpu),
                                  None if bias is None else to_dev_bits(bias, gpu),
                                  None if sgw is None else to_dev_bits(sgw, gpu))
    _, oidx, ow, osg = oracle.router(x, w, spec.router_dtype == "float32", bias, spec.top_k,
                                     spec.route_mode, sgw)
    assert np.array_equal(idx.cpu().numpy(), oidx)
    np.testing.assert_allclose(wt.cpu().numpy(), ow, rtol=1e-5, atol=1e-7)
    if sgw is not None:
        np.testing.assert_allclose(sg.cpu().numpy(), osg, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("T", [1, 8, 65])
def test_router_summation_order_kat(gpu, T):
    """The kernels sum a logit in the oracle's lane-tree order: expert 0's row is built so that
    this order gives exactly 0 (element order would give 1), expert 1's row gives 0.5 and every
    other row -1, so the top-2 is [1, 0] only under the specified order."""
    import torch
    spec = small(OLMOE_1B_7B, hidden=1024, n_experts=64, top_k=2)
    H = spec.hidden
    w = np.full((64, H), -1.0 / H, np.float32)
    w[0] = 0.0
    w[0, 0], w[0, 8 * 32], w[0, 8] = 2.0 ** 24, 1.0, -(2.0 ** 24)
    w[1] = 0.5 / H
    x = np.full((T, H), 0x3F80, np.uint16)
    lg, oidx, _, _ = oracle.router(x, w, True, None, 2, spec.route_mode)
    assert (lg[:, 0] == 0.0).all() and (lg[:, 1] == 0.5).all() and (oidx == [1, 0]).all()
    idx, _, _ = ops.router_topk(spec, to_dev_bits(x, gpu), torch.from_numpy(w).to(gpu))
    assert (idx.cpu().numpy() == [1, 0]).all()


def _layer_check(lay, moe, T, seed, check_f64=True):
    import torch
    spec = lay.spec
    x = make_x(T, spec.hidden, seed=seed)
    xd = to_dev_bits(x, moe.router_w.device)
    out = moe(xd)
    torch.cuda.synchronize()
    _, idx, w, sg = oracle.router(x, lay.router, spec.router_dtype == "float32", lay.bias,
                                  spec.top_k, spec.route_mode, lay.sgate_w)
    ref, _ = oracle.moe_forward(spec, lay.experts, x, idx, w, lay.shared, sg)
    got = F.bf16_bits_to_f32(bits(out))
    r = oracle.rel_l2(got, F.bf16_bits_to_f32(ref))
    assert r < TOL, f"rel L2 vs C oracle {r:.3e}"
    if check_f64:
        truth, _ = oracle.moe_forward_f64(spec, lay.experts, x, idx, w, lay.shared, sg)
        r64 = oracle.rel_l2(got, truth)
        assert r64 < TOL, f"rel L2 vs float64 truth {r64:.3e}"
    return r


@pytest.mark.parametrize("spec", [SMALL_AFFINE, SMALL_F16, SMALL_MXFP4, SMALL_SHARED],
                         ids=["bf16", "f16", "mxfp4", "shared"])
@pytest.mark.parametrize("T", [1, 3, 8])
def test_decode_layer(gpu, spec, T):
    lay = make_layer(spec, seed=11)
    moe, sw, pool, _ = build_gpu_layer(lay, gpu)
    assert sw._sync_free
    _layer_check(lay, moe, T, seed=100 + T)
    pool.close()


@pytest.mark.parametrize("spec", [small(QWEN3_30B_A3B, hidden=512, inter=768, n_experts=64, top_k=8),
                                  small(GPT_OSS_120B, hidden=512, inter=1536, n_experts=32, top_k=4)],
                         ids=["affine-I768", "mxfp4-I1536"])
def test_decode_layer_staged_in_batches(gpu, spec):
    """8 tokens whose h rows do not all fit in LDS: the down kernel stages them entry batch by
    entry batch."""
    lay = make_layer(spec, seed=17, bank=8)
    moe, sw, pool, _ = build_gpu_layer(lay, gpu)
    pairs = 8 * spec.top_k
    assert pairs * (spec.inter // 64) * 148 > 96 * 1024
    _layer_check(lay, moe, 8, seed=170, check_f64=False)
    pool.close()


@pytest.mark.parametrize("spec", [SMALL_AFFINE, SMALL_F16, SMALL_MXFP4, SMALL_SHARED],
                         ids=["bf16", "f16", "mxfp4", "shared"])
@pytest.mark.parametrize("T", [9, 64, 257])
def test_prefill_layer(gpu, spec, T):
    lay = make_layer(spec, seed=12, zipf=1.1)
    moe, sw, pool, _ = build_gpu_layer(lay, gpu)
    _layer_check(lay, moe, T, seed=200 + T, check_f64=T < 100)
    pool.close()


@pytest.mark.parametrize("spec", [SMALL_AFFINE, SMALL_F16, SMALL_MXFP4, SMALL_SHARED],
                         ids=["bf16", "f16", "mxfp4", "shared"])
@pytest.mark.parametrize("T", [1, 5, 8, 40])
def test_block_forward(gpu, spec, T):
    """brx_moe_block_forward (routing ranked inside the decode kernel for T <= 8): the routing
    it reports is the oracle's bit for bit, and the block output matches the oracle layer."""
    import torch
    lay = make_layer(spec, seed=13, zipf=0.9)
    _, sw, pool, _ = build_gpu_layer(lay, gpu)
    x = make_x(T, spec.hidden, seed=300 + T)
    xd = to_dev_bits(x, gpu)
    router = to_dev_bits(lay.router, gpu)
    bias = None if lay.bias is None else to_dev_bits(lay.bias, gpu)
    sgw = None if lay.sgate_w is None else to_dev_bits(lay.sgate_w, gpu)
    gi = torch.full((T, spec.top_k), -1, dtype=torch.int32, device=gpu)
    gw = torch.zeros((T, spec.top_k), dtype=torch.float32, device=gpu)
    pool.g2s_device(torch.cuda.current_stream().cuda_stream)
    out = ops.moe_block(spec, pool, xd, router, bias, sgw, sw.shared, out_idx=gi, out_w=gw,
                        flags=ops.path_flag(T, spec.top_k))
    torch.cuda.synchronize()
    _, idx, w, sg = oracle.router(x, lay.router, spec.router_dtype == "float32", lay.bias,
                                  spec.top_k, spec.route_mode, lay.sgate_w)
    assert np.array_equal(gi.cpu().numpy(), idx)
    np.testing.assert_allclose(gw.cpu().numpy(), w, rtol=1e-5, atol=1e-7)
    ref, _ = oracle.moe_forward(spec, lay.experts, x, idx, w, lay.shared, sg)
    r = oracle.rel_l2(F.bf16_bits_to_f32(bits(out)), F.bf16_bits_to_f32(ref))
    assert r < TOL, f"rel L2 vs C oracle {r:.3e}"
    # the same block through the separate router + expert entry points gives the same bits
    moe = ops.MoELayer(spec, router, sw, router_bias=bias, shared_gate_w=sgw)
    sw._sync_free = False
    out2 = moe(xd)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out2), bits(out))
    pool.close()


@pytest.mark.parametrize("spec", [SMALL_AFFINE, SMALL_MXFP4], ids=["affine", "mxfp4"])
def test_one_token_repeated_experts(gpu, spec):
    """One token whose given pairs repeat experts. brx_moe_forward takes the one-token kernels
    (every pair its own entry, then the one-pair down kernel); brx_moe_forward_pairs in decode
    mode, with the pairs' tokens given, merges a repeated expert into one entry of several pairs
    (the down kernel for several pairs an entry). Both against the oracle pair by pair, and the
    same bits, since one token fixes one row split."""
    import torch
    lay = make_layer(spec, seed=23)
    _, sw, pool, _ = build_gpu_layer(lay, gpu)
    pool.g2s_device(torch.cuda.current_stream().cuda_stream)
    k = spec.top_k
    x = make_x(1, spec.hidden, seed=41)
    xd = to_dev_bits(x, gpu)
    e = [5, 5, 2, 9, 5, 1, 0, 3][:k] if k == 8 else [7, 2, 7, 7][:k]
    idx = np.array([e], np.int32)
    print(f"[repeat] {spec.quant.mode} experts {e}", flush=True)
    w = np.full((1, k), 1.0 / k, np.float32)
    y1 = torch.empty((1, k, spec.hidden), dtype=torch.bfloat16, device=gpu)
    ops.moe_forward(spec, pool, xd, torch.from_numpy(idx).to(gpu), torch.from_numpy(w).to(gpu),
                    y_unreduced=y1, flags=ops.path_flag(1, k))
    y2 = torch.full((k, spec.hidden), float("nan"), dtype=torch.bfloat16, device=gpu)
    ops.forward_pairs(spec, pool, xd, torch.zeros(k, dtype=torch.int32, device=gpu),
                      torch.from_numpy(idx[0]).to(gpu), torch.arange(k, dtype=torch.int32, device=gpu), y2,
                      ops.path_flag(1, k))
    torch.cuda.synchronize()
    _, yref = oracle.moe_forward(spec, lay.experts, x, idx, w, want_unreduced=True)
    ref = F.bf16_bits_to_f32(yref)[0]
    got1 = F.bf16_bits_to_f32(bits(y1))[0]
    for j in range(k):
        assert oracle.rel_l2(got1[j], ref[j]) < TOL, j
    assert np.array_equal(bits(y1).reshape(k, -1), bits(y2))
    pool.close()


@pytest.mark.parametrize("T", [1, 16])
def test_unreduced_rows(gpu, T):
    """The operator's unreduced [T, k, H] rows (the reference boundary) against the oracle."""
    import torch
    spec = SMALL_AFFINE
    lay = make_layer(spec, seed=21)
    moe, sw, pool, _ = build_gpu_layer(lay, gpu)
    x = make_x(T, spec.hidden, seed=31)
    _, idx, w, _ = oracle.router(x, lay.router, False, None, spec.top_k, spec.route_mode)
    y = sw(to_dev_bits(x, gpu), torch.from_numpy(idx).to(gpu))
    torch.cuda.synchronize()
    _, yref = oracle.moe_forward(spec, lay.experts, x, idx, w, want_unreduced=True)
    got = F.bf16_bits_to_f32(bits(y))
    ref = F.bf16_bits_to_f32(yref)
    assert got.shape == ref.shape == (T, spec.top_k, spec.hidden)
    for t in range(T):
        for j in range(spec.top_k):
            assert oracle.rel_l2(got[t, j], ref[t, j]) < TOL, (t, j)
    pool.close()


@pytest.mark.parametrize("case", ["uniform", "crowded"])
def test_sort_pairs_matches_stable_argsort(gpu, case):
    """uniform: 333 tokens over 32 experts; crowded: 2600 tokens where expert 5 takes 10,400
    pairs, more than a block lists in LDS, so its block compacts in a second pass."""
    import torch
    spec = SMALL_AFFINE
    rng = np.random.default_rng(4)
    if case == "uniform":
        idx = rng.integers(0, spec.n_experts, size=(333, spec.top_k)).astype(np.int32)
    else:
        idx = rng.integers(0, spec.n_experts, size=(2600, spec.top_k)).astype(np.int32)
        idx[:, : spec.top_k // 2] = 5
        assert (idx == 5).sum() > 8192
    order, offsets = ops.sort_pairs(spec, torch.from_numpy(idx).to(gpu))
    o_ref, off_ref = oracle.sort_pairs(idx, spec.n_experts)
    assert np.array_equal(order.cpu().numpy(), o_ref)
    assert np.array_equal(offsets.cpu().numpy(), off_ref)
    assert np.array_equal(o_ref, np.argsort(idx.reshape(-1), kind="stable"))
