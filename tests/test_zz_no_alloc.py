"""brx_moe_block_forward_noalloc: the whole-block forward over the library's static per-GPU
scratch. Called through the raw C-ABI, it returns exactly what brx_moe_block_forward returns (the
same kernels), for two calls in a row of which the second is smaller (the scratch keeps the first
call's contents and nothing in it may be read before it is written), in the decode and the
grouped-GEMM regimes; a call whose scratch exceeds the maximum is refused before anything runs.
"""
import ctypes as C

import numpy as np
import pytest

from bigrig_amd import lib as L
from bigrig_amd.spec import E256_SHARED, QWEN3_30B_A3B
from tests.gpu_util import bits, build_gpu_layer, to_dev_bits
from tests.helpers import make_layer, make_x, small

pytestmark = pytest.mark.gpu


def _call(fn, spec, pool, x, router, bias, sgw, shared, flags):
    import torch
    T = x.shape[0]
    out = torch.full((T, spec.hidden), 3.0, dtype=torch.bfloat16, device=x.device)
    idx = torch.full((T, spec.top_k), -1, dtype=torch.int32, device=x.device)
    w = torch.zeros((T, spec.top_k), dtype=torch.float32, device=x.device)
    d = spec.desc()
    p = lambda t: None if t is None else t.data_ptr()   # noqa: E731
    rc = fn(C.byref(d), pool.device.handle, x.data_ptr(), router.data_ptr(), p(bias), p(sgw),
            p(shared), T, out.data_ptr(), idx.data_ptr(), w.data_ptr(), flags,
            torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return rc, out, idx, w


@pytest.mark.parametrize("spec", [small(QWEN3_30B_A3B, n_experts=32),
                                  small(E256_SHARED, n_experts=32)], ids=["qwen3", "shared"])
@pytest.mark.parametrize("sizes", [(8, 1), (200, 40)], ids=["decode", "prefill"])
def test_noalloc_block_forward_equals_block_forward(gpu, spec, sizes):
    import torch
    lib = L.load()
    lay = make_layer(spec, seed=501, bank=4, zipf=1.1)
    moe, sw, pool, _ = build_gpu_layer(lay, gpu)
    pool.g2s_device(torch.cuda.current_stream().cuda_stream)
    router = to_dev_bits(lay.router, gpu)
    bias = to_dev_bits(lay.bias, gpu)
    sgw = None if lay.sgate_w is None else to_dev_bits(lay.sgate_w, gpu)
    shared = sw.shared
    for T in sizes:
        flags = 0
        print(f"[noalloc] {spec.n_experts}x{spec.inter} shared={spec.shared_inter} T={T}",
              flush=True)
        x = to_dev_bits(make_x(T, spec.hidden, seed=5010 + T), gpu)
        rc0, out0, idx0, w0 = _call(lib.brx_moe_block_forward, spec, pool, x, router, bias, sgw,
                                    shared, flags)
        rc1, out1, idx1, w1 = _call(lib.brx_moe_block_forward_noalloc, spec, pool, x, router,
                                    bias, sgw, shared, flags)
        assert rc0 == 0 and rc1 == 0, lib.brx_last_error().decode()
        assert np.array_equal(idx1.cpu().numpy(), idx0.cpu().numpy())
        assert np.array_equal(w1.cpu().numpy().view(np.uint32), w0.cpu().numpy().view(np.uint32))
        assert np.array_equal(bits(out1), bits(out0))
    pool.close()


def test_noalloc_refuses_a_call_beyond_its_scratch(gpu):
    import torch
    lib = L.load()
    spec = small(QWEN3_30B_A3B, n_experts=16)
    lay = make_layer(spec, seed=502, bank=2)
    moe, sw, pool, _ = build_gpu_layer(lay, gpu)
    pool.g2s_device(torch.cuda.current_stream().cuda_stream)
    T = 2048
    print(f"[noalloc] refuse T={T}", flush=True)
    x = torch.zeros((T, spec.hidden), dtype=torch.bfloat16, device=gpu)
    rc, out, idx, _ = _call(lib.brx_moe_block_forward_noalloc, spec, pool, x,
                            to_dev_bits(lay.router, gpu), None, None, None, 0)
    assert rc == L.BRX_EINVAL
    assert "scratch" in lib.brx_last_error().decode()
    assert bool((out.float() == 3.0).all()) and bool((idx == -1).all())
    pool.close()
