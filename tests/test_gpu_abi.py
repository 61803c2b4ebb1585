"""C-ABI guarantees on the GPU, called through the raw library:

* a whole-block forward refuses a pool that is neither fully resident nor host-backed, before it
  launches anything (the reference raises KeyError for a non-resident expert,
  stream.py:608-615), and writes nothing;
* an expert that routing names but the pool neither holds nor can read from host memory is never
  computed from another expert's slot: every row it touches is NaN, every other row equals the
  oracle's, and brx_pool_check reports it (then clears);
* top-k above 8 at up to 8 tokens (more than 64 pairs) takes the grouped GEMM, not the decode
  kernels, and matches the oracle;
* hidden widths past one router pass (4096: two passes of 3072) route bit-exactly and match the
  oracle through decode and prefill;
* a shared expert whose intermediate width differs from the routed experts' matches the oracle.
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from bigrig_amd import formats as F
from bigrig_amd import layer as ops
from bigrig_amd import lib as L
from bigrig_amd.pool import ExpertPool, HostStore
from bigrig_amd.spec import E256_SHARED, QWEN3_30B_A3B
from tests.gpu_util import bits, build_gpu_layer, to_dev_bits
from tests.helpers import make_layer, make_x, small

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _stream():
    import torch
    return torch.cuda.current_stream().cuda_stream


def _bounded(lay, capacity, admit):
    store = HostStore()
    store.add_layer(0, lay.experts)
    pool = ExpertPool(0, lay.spec, capacity).build()
    for e in admit:
        pool.touch([e], [0])
        pool.admit(e, store.region(0, e))
    pool.g2s_device(_stream())
    pool.device.sync()
    return pool


@pytest.mark.parametrize("capacity", [16, 32], ids=["bounded", "full-capacity-one-missing"])
def test_block_forward_refuses_a_pool_that_is_not_fully_resident(gpu, capacity):
    import torch
    spec = small(QWEN3_30B_A3B, hidden=512, inter=256, n_experts=32, top_k=8)
    lay = make_layer(spec, seed=401)
    pool = _bounded(lay, capacity, range(min(capacity, spec.n_experts - 1)))
    router = to_dev_bits(lay.router, gpu)
    lib = L.load()
    for T in (1, 40):
        print(f"[abi] refuse C={capacity} T={T}", flush=True)
        x = to_dev_bits(make_x(T, spec.hidden, seed=4010 + T), gpu)
        out = torch.full((T, spec.hidden), 7.0, dtype=torch.bfloat16, device=gpu)
        idx = torch.full((T, spec.top_k), -5, dtype=torch.int32, device=gpu)
        d = spec.desc()
        rc = lib.brx_moe_block_forward(C.byref(d), pool.device.handle, x.data_ptr(),
                                       router.data_ptr(), None, None, None, T, out.data_ptr(),
                                       idx.data_ptr(), None, ops.path_flag(T, spec.top_k),
                                       _stream())
        assert rc == L.BRX_ESTATE
        assert "resident" in lib.brx_last_error().decode()
        torch.cuda.synchronize()
        assert bool((out.float() == 7.0).all()) and bool((idx == -5).all()), "wrote outputs"
    pool.close()


@pytest.mark.parametrize("T", [2, 40], ids=["decode", "prefill"])
def test_absent_expert_is_reported_and_its_rows_are_nan(gpu, T):
    import torch
    spec = small(QWEN3_30B_A3B, hidden=512, inter=256, n_experts=32, top_k=4)
    lay = make_layer(spec, seed=402)
    pool = _bounded(lay, 16, range(16))
    rng = np.random.default_rng(T)
    idx = np.stack([rng.permutation(16)[:spec.top_k] for _ in range(T)]).astype(np.int32)
    idx[0, 1] = 20                       # absent: not in a slot, no host backing
    w = np.full((T, spec.top_k), 1.0 / spec.top_k, np.float32)
    x = make_x(T, spec.hidden, seed=4020 + T)
    out = torch.zeros((T, spec.hidden), dtype=torch.bfloat16, device=gpu)
    y = torch.zeros((T, spec.top_k, spec.hidden), dtype=torch.bfloat16, device=gpu)
    print(f"[abi] absent expert T={T}", flush=True)
    ops.moe_forward(spec, pool, to_dev_bits(x, gpu), to_dev_bits(idx, gpu), to_dev_bits(w, gpu),
                    out=out, y_unreduced=y)
    lib = L.load()
    rc = lib.brx_pool_check(pool.device.handle)
    assert rc == L.BRX_ERANGE
    assert "expert 20" in lib.brx_last_error().decode()
    assert lib.brx_pool_check(pool.device.handle) == L.BRX_OK, "the report clears the error"
    yb = F.bf16_bits_to_f32(bits(y))
    ob = F.bf16_bits_to_f32(bits(out))
    assert np.isnan(yb[0, 1]).all() and np.isnan(ob[0]).all()
    ref, yref = oracle.moe_forward(spec, lay.experts, x, idx, w, want_unreduced=True)
    keep = np.ones((T, spec.top_k), bool)
    keep[0, 1] = False
    got, want = yb[keep], F.bf16_bits_to_f32(yref)[keep]
    assert np.isfinite(got).all()
    assert oracle.rel_l2(got, want) < TOL
    if T > 1:
        assert oracle.rel_l2(ob[1:], F.bf16_bits_to_f32(ref)[1:]) < TOL
    pool.close()


@pytest.mark.parametrize("T", [4, 8], ids=["pairs64-decode", "pairs128-gemm"])
def test_top_k_16_block(gpu, T):
    """T x top-16: 64 pairs still decode, 128 take the grouped GEMM; both match the oracle."""
    import torch
    spec = small(QWEN3_30B_A3B, hidden=512, inter=256, n_experts=64, top_k=16)
    lay = make_layer(spec, seed=403, zipf=0.8)
    moe, sw, pool, _ = build_gpu_layer(lay, gpu)
    pool.g2s_device(_stream())
    x = make_x(T, spec.hidden, seed=4030 + T)
    gi = torch.full((T, spec.top_k), -1, dtype=torch.int32, device=gpu)
    gw = torch.zeros((T, spec.top_k), dtype=torch.float32, device=gpu)
    print(f"[abi] top-16 T={T} flag={ops.path_flag(T, spec.top_k)}", flush=True)
    out = ops.moe_block(spec, pool, to_dev_bits(x, gpu), to_dev_bits(lay.router, gpu),
                        to_dev_bits(lay.bias, gpu), out_idx=gi, out_w=gw,
                        flags=ops.path_flag(T, spec.top_k))
    torch.cuda.synchronize()
    _, idx, w, _ = oracle.router(x, lay.router, False, lay.bias, spec.top_k, spec.route_mode)
    assert np.array_equal(gi.cpu().numpy(), idx)
    ref, _ = oracle.moe_forward(spec, lay.experts, x, idx, w)
    r = oracle.rel_l2(F.bf16_bits_to_f32(bits(out)), F.bf16_bits_to_f32(ref))
    assert r < TOL, f"rel L2 {r:.3e}"
    # without a flag the library makes the same choice
    d = spec.desc()
    out2 = torch.empty_like(out)
    xd, rd, bd = (to_dev_bits(x, gpu), to_dev_bits(lay.router, gpu),
                  to_dev_bits(lay.bias, gpu))     # held: a temporary's memory is reused at once
    L.check(L.load().brx_moe_block_forward(
        C.byref(d), pool.device.handle, xd.data_ptr(), rd.data_ptr(), bd.data_ptr(), None,
        None, T, out2.data_ptr(), None, None, 0, _stream()))
    torch.cuda.synchronize()
    assert np.array_equal(bits(out2), bits(out))
    pool.close()


@pytest.mark.parametrize("H,T", [(4096, 1), (4096, 8), (4096, 40), (4096, 80), (8192, 1), (8192, 8),
                                 (8192, 80)])
def test_wide_hidden(gpu, H, T):
    """Several router passes per lane (4096 and 8192 > 3072): routing bit-exact, layer within
    tolerance. At 8192 the prefill router's LDS token tiles (32 H bytes) would exceed a block's
    160 KB, so its token tiles take the register path; the decode kernels stage 8 rows of 8192."""
    import torch
    spec = small(QWEN3_30B_A3B, hidden=H, inter=256, n_experts=16, top_k=4)
    lay = make_layer(spec, seed=404, zipf=0.5)
    moe, sw, pool, _ = build_gpu_layer(lay, gpu)
    x = make_x(T, spec.hidden, seed=4040 + T)
    print(f"[abi] hidden {H} T={T}", flush=True)
    gidx, gw, _ = moe.route(to_dev_bits(x, gpu))
    out = moe(to_dev_bits(x, gpu))
    torch.cuda.synchronize()
    _, idx, w, _ = oracle.router(x, lay.router, False, lay.bias, spec.top_k, spec.route_mode)
    assert np.array_equal(gidx.cpu().numpy(), idx)
    np.testing.assert_allclose(gw.cpu().numpy(), w, rtol=1e-5, atol=1e-7)
    ref, _ = oracle.moe_forward(spec, lay.experts, x, idx, w)
    r = oracle.rel_l2(F.bf16_bits_to_f32(bits(out)), F.bf16_bits_to_f32(ref))
    assert r < TOL, f"rel L2 {r:.3e}"
    pool.close()


@pytest.mark.parametrize("T", [1, 8, 40])
def test_shared_expert_of_its_own_width(gpu, T):
    """Routed inter 256, shared inter 768 (the decode kernels size their h rows for the wider)."""
    import torch
    spec = small(E256_SHARED, hidden=512, inter=256, n_experts=32, top_k=8, shared_inter=768)
    lay = make_layer(spec, seed=405)
    moe, sw, pool, _ = build_gpu_layer(lay, gpu)
    x = make_x(T, spec.hidden, seed=4050 + T)
    print(f"[abi] shared inter 768, routed 256, T={T}", flush=True)
    out = moe(to_dev_bits(x, gpu))
    torch.cuda.synchronize()
    _, idx, w, sg = oracle.router(x, lay.router, False, lay.bias, spec.top_k, spec.route_mode,
                                  lay.sgate_w)
    ref, _ = oracle.moe_forward(spec, lay.experts, x, idx, w, lay.shared, sg)
    got = F.bf16_bits_to_f32(bits(out))
    r = oracle.rel_l2(got, F.bf16_bits_to_f32(ref))
    assert r < TOL, f"rel L2 {r:.3e}"
    truth, _ = oracle.moe_forward_f64(spec, lay.experts, x, idx, w, lay.shared, sg)
    assert oracle.rel_l2(got, truth) < TOL
    pool.close()
