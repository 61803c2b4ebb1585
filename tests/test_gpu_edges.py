"""Edge cases of the path on the GPU, through the C-ABI: empty inputs, router ties (also across a
lane's registers and at the top-k boundary), -inf logits, the largest expert count the library
takes (512, the in-kernel ranking's widest case), and top-1 routing.

Bars as elsewhere: routing indices bit-exact against the oracle (ties to the lower expert id,
the rule of the reference's argsort over -logits, pool.py:333), outputs within 1e-2 relative
L2 of the oracle, and nothing written for an empty call.
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from bigrig_amd import formats as F
from bigrig_amd import layer as ops
from bigrig_amd import lib as L
from bigrig_amd.spec import QWEN3_30B_A3B
from tests.gpu_util import bits, build_gpu_layer, to_dev_bits
from tests.helpers import make_layer, make_x, small

pytestmark = pytest.mark.gpu

TOL = 1e-2
E512 = small(QWEN3_30B_A3B, hidden=512, inter=256, n_experts=512, top_k=8)
TOP1 = small(QWEN3_30B_A3B, hidden=512, inter=256, n_experts=16, top_k=1)


def test_empty_inputs_write_nothing(gpu):
    import torch
    spec = small(QWEN3_30B_A3B, hidden=512, inter=256, n_experts=16, top_k=4)
    lay = make_layer(spec, seed=90)
    _, sw, pool, _ = build_gpu_layer(lay, gpu)
    d = spec.desc()
    lib = L.load()
    x = torch.zeros((1, spec.hidden), dtype=torch.bfloat16, device=gpu)
    router = to_dev_bits(lay.router, gpu)
    out = torch.full((1, spec.hidden), 7.0, dtype=torch.bfloat16, device=gpu)
    idx = torch.full((1, spec.top_k), -5, dtype=torch.int32, device=gpu)
    w = torch.full((1, spec.top_k), 3.0, dtype=torch.float32, device=gpu)
    s = torch.cuda.current_stream().cuda_stream
    assert lib.brx_router_topk(C.byref(d), x.data_ptr(), router.data_ptr(), None, None, 0,
                               idx.data_ptr(), w.data_ptr(), None, s) == 0
    for flags in (L.FWD_FORCE_DECODE, L.FWD_FORCE_PREFILL, 0):
        assert lib.brx_moe_forward(C.byref(d), pool.device.handle, x.data_ptr(), idx.data_ptr(),
                                   w.data_ptr(), None, None, 0, out.data_ptr(), None, flags, s) == 0
        assert lib.brx_moe_block_forward(C.byref(d), pool.device.handle, x.data_ptr(),
                                         router.data_ptr(), None, None, None, 0, out.data_ptr(),
                                         idx.data_ptr(), w.data_ptr(), flags, s) == 0
    assert lib.brx_moe_forward(C.byref(d), pool.device.handle, x.data_ptr(), idx.data_ptr(),
                               w.data_ptr(), None, None, -1, out.data_ptr(), None, 0, s) != 0
    torch.cuda.synchronize()
    assert (out.float() == 7.0).all() and (idx == -5).all() and (w == 3.0).all()
    pool.close()


def test_router_ties_go_to_the_lower_id(gpu):
    """Duplicated router rows give exactly equal logits: the lower expert id ranks first, on the
    decode (in-kernel) and the chunk router alike."""
    import torch
    spec = small(QWEN3_30B_A3B, hidden=512, inter=256, n_experts=32, top_k=8)
    lay = make_layer(spec, seed=91)
    r = F.bf16_bits_to_f32(lay.router).copy()
    for a, b in ((3, 17), (5, 6), (30, 2), (11, 12)):
        r[b] = r[a]
    lay.router = F.f32_to_bf16_bits(r)
    _, sw, pool, _ = build_gpu_layer(lay, gpu)
    pool.g2s_device(torch.cuda.current_stream().cuda_stream)
    router = to_dev_bits(lay.router, gpu)
    ties = 0
    for T in (1, 8, 64):
        x = make_x(T, spec.hidden, seed=910 + T)
        _, idx, wref, _ = oracle.router(x, lay.router, False, None, spec.top_k, spec.route_mode)
        gi = torch.full((T, spec.top_k), -1, dtype=torch.int32, device=gpu)
        gw = torch.zeros((T, spec.top_k), dtype=torch.float32, device=gpu)
        ops.moe_block(spec, pool, to_dev_bits(x, gpu), router, out_idx=gi, out_w=gw,
                      flags=ops.path_flag(T, spec.top_k))
        i2, w2, _ = ops.router_topk(spec, to_dev_bits(x, gpu), router)
        torch.cuda.synchronize()
        assert np.array_equal(gi.cpu().numpy(), idx)
        assert np.array_equal(i2.cpu().numpy(), idx)
        for row in idx:
            for a, b in ((3, 17), (5, 6), (2, 30), (11, 12)):
                if a in row and b in row:
                    ties += 1
                    assert list(row).index(a) < list(row).index(b)
    assert ties > 0, "no token routed to both experts of a tied pair"
    pool.close()


@pytest.mark.parametrize("T", [1, 8, 40])
def test_512_experts(gpu, T):
    """The widest in-kernel ranking (8 logits a lane) and the table staged for 512 experts."""
    import torch
    spec = E512
    lay = make_layer(spec, seed=92, bank=16)
    moe, sw, pool, _ = build_gpu_layer(lay, gpu)
    pool.g2s_device(torch.cuda.current_stream().cuda_stream)
    x = make_x(T, spec.hidden, seed=920 + T)
    router = to_dev_bits(lay.router, gpu)
    gi = torch.full((T, spec.top_k), -1, dtype=torch.int32, device=gpu)
    gw = torch.zeros((T, spec.top_k), dtype=torch.float32, device=gpu)
    out = ops.moe_block(spec, pool, to_dev_bits(x, gpu), router, out_idx=gi, out_w=gw,
                        flags=ops.path_flag(T, spec.top_k))
    torch.cuda.synchronize()
    _, idx, w, _ = oracle.router(x, lay.router, False, None, spec.top_k, spec.route_mode)
    assert np.array_equal(gi.cpu().numpy(), idx)
    np.testing.assert_allclose(gw.cpu().numpy(), w, rtol=1e-5, atol=1e-7)
    ref, _ = oracle.moe_forward(spec, lay.experts, x, idx, w)
    r = oracle.rel_l2(F.bf16_bits_to_f32(bits(out)), F.bf16_bits_to_f32(ref))
    assert r < TOL, f"rel L2 {r:.3e}"
    pool.close()


@pytest.mark.parametrize("T", [1, 3, 33])
def test_top1_routing(gpu, T):
    """k = 1: one pair a token (renormalised weight exactly 1)."""
    import torch
    spec = TOP1
    lay = make_layer(spec, seed=93)
    moe, sw, pool, _ = build_gpu_layer(lay, gpu)
    x = make_x(T, spec.hidden, seed=930 + T)
    out = moe(to_dev_bits(x, gpu))
    torch.cuda.synchronize()
    _, idx, w, _ = oracle.router(x, lay.router, False, None, 1, spec.route_mode)
    assert np.all(w == 1.0)
    ref, _ = oracle.moe_forward(spec, lay.experts, x, idx, w)
    r = oracle.rel_l2(F.bf16_bits_to_f32(bits(out)), F.bf16_bits_to_f32(ref))
    assert r < TOL, f"rel L2 {r:.3e}"
    pool.close()


@pytest.mark.parametrize("case", ["ties", "neg_inf"])
def test_router_ties_across_registers_and_infinities(gpu, case):
    """Exact logits from a one-hot token: ties between experts held in different registers of
    one lane (6 and 70 at E = 128) and at the top-k boundary go to the lower id, and -inf ranks
    below every number (taken lowest id first when fewer than k logits are finite), in the
    in-kernel ranking and the chunk router alike; the expected order is written out by hand."""
    import torch
    spec = small(QWEN3_30B_A3B, hidden=512, inter=256, n_experts=128, top_k=8)
    lay = make_layer(spec, seed=94)
    col = 5
    lg = np.full(spec.n_experts, -np.inf, np.float32)
    if case == "ties":
        for e, v in ((70, 2.0), (6, 2.0), (100, 2.0), (3, 1.5), (127, 0.0), (64, 0.0), (0, 0.0),
                     (90, 0.0), (10, -1.0), (11, -1.0)):
            lg[e] = v
        want = [6, 70, 100, 3, 0, 64, 90, 127]
    else:
        for e, v in ((70, 2.0), (6, 2.0), (3, 1.5), (64, 0.0), (0, 0.0)):
            lg[e] = v
        want = [6, 70, 3, 0, 64, 1, 2, 4]
    r = F.bf16_bits_to_f32(lay.router).copy()
    r[:, col] = lg
    lay.router = F.f32_to_bf16_bits(r)
    _, sw, pool, _ = build_gpu_layer(lay, gpu)
    pool.g2s_device(torch.cuda.current_stream().cuda_stream)
    router = to_dev_bits(lay.router, gpu)
    x = np.zeros((1, spec.hidden), np.uint16)
    x[0, col] = 0x3F80   # bf16 1.0: logit e is the router's entry (e, col) exactly
    _, idx, wref, _ = oracle.router(x, lay.router, False, None, spec.top_k, spec.route_mode)
    assert list(idx[0]) == want
    gi = torch.full((1, spec.top_k), -1, dtype=torch.int32, device=gpu)
    gw = torch.zeros((1, spec.top_k), dtype=torch.float32, device=gpu)
    ops.moe_block(spec, pool, to_dev_bits(x, gpu), router, out_idx=gi, out_w=gw,
                  flags=ops.path_flag(1, spec.top_k))
    i2, w2, _ = ops.router_topk(spec, to_dev_bits(x, gpu), router)
    torch.cuda.synchronize()
    assert list(gi.cpu().numpy()[0]) == want
    assert list(i2.cpu().numpy()[0]) == want
    np.testing.assert_allclose(gw.cpu().numpy(), wref, rtol=1e-6, atol=0)
    np.testing.assert_allclose(w2.cpu().numpy(), wref, rtol=1e-6, atol=0)
    if case == "neg_inf":
        assert np.all(wref[0, 5:] == 0.0)
    pool.close()
