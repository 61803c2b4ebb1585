"""Host-served misses: a bounded pool with host backing stays on the sync-free path, the kernels
reading every absent expert from the pinned host store, while residency is updated behind the
forwards from routing copied back asynchronously.

The bar is the pool invariant of the reference (stream.py:25-30; tests/test_stream.py:530-545):
where the bytes live never changes the arithmetic, so every output equals the fully resident
layer's bit for bit -- here while admissions race the forwards, since steps are issued back to
back with no host synchronisation. After the copies drain, the device table and every slot's
bytes must agree with the host's bookkeeping.
"""
import ctypes as C

import numpy as np
import pytest

from bigrig_amd import formats as F
from bigrig_amd import lib as L
from bigrig_amd.layer import MoELayer, StreamingSwitchGLU
from bigrig_amd.pool import ExpertPool, HostStore, PinnedFetcher
from bigrig_amd.spec import E256_SHARED, GPT_OSS_120B, OLMOE_1B_7B, QWEN3_30B_A3B
from tests.gpu_util import bits, build_gpu_layer, bytes_dev, to_dev_bits
from tests.helpers import make_layer, make_x, small

pytestmark = pytest.mark.gpu

AFFINE = small(QWEN3_30B_A3B, hidden=512, inter=256, n_experts=32, top_k=8)
SHARED = small(E256_SHARED, hidden=512, inter=256, n_experts=32, top_k=8, shared_inter=256)
MXFP4 = small(GPT_OSS_120B, hidden=576, inter=320, n_experts=16, top_k=4)
F16 = small(OLMOE_1B_7B, hidden=512, inter=256, n_experts=16, top_k=4,
            quant=F.QuantSpec(4, 64, "affine", "float16"))


def _host_served(lay, gpu, C_):
    spec = lay.spec
    store = HostStore()
    store.add_layer(0, lay.experts)
    pool = ExpertPool(0, spec, C_).build()
    shared = bytes_dev(lay.shared, gpu) if lay.shared is not None else None
    sw = StreamingSwitchGLU(pool, PinnedFetcher(store), shared=shared, host_served=True)
    router = to_dev_bits(lay.router, gpu)
    bias = None if lay.bias is None else to_dev_bits(lay.bias, gpu)
    sgw = None if lay.sgate_w is None else to_dev_bits(lay.sgate_w, gpu)
    return MoELayer(spec, router, sw, router_bias=bias, shared_gate_w=sgw), sw, pool, store


def _hip():
    return C.CDLL("libamdhip64.so")


def _d2h(ptr: int, n: int) -> bytes:
    out = (C.c_uint8 * n)()
    hip = _hip()
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    assert hip.hipMemcpy(out, C.c_void_p(ptr), n, 2) == 0     # hipMemcpyDeviceToHost
    return bytes(out)


def _check_settled(sw, pool, store):
    """Device table == host bookkeeping; each resident expert's slot holds its bytes."""
    import torch
    sw._serve.drain()
    pool.device.sync()
    torch.cuda.synchronize()
    g = C.c_void_p()
    L.check(L.load().brx_pool_g2s_ptr(pool.device.handle, C.byref(g)))
    dev = np.frombuffer(_d2h(g.value, 4 * pool.n_experts), dtype=np.int32)
    assert np.array_equal(dev, pool.g2s), (dev, pool.g2s)
    for slot in range(pool.capacity):
        e = int(pool.s2g[slot])
        if e < 0:
            continue
        r = store.region(0, e)
        want = bytes(np.ctypeslib.as_array((C.c_uint8 * r.nbytes).from_address(r.ptr)))
        assert _d2h(pool.device.slot_ptr(slot), r.nbytes) == want, f"slot {slot} (expert {e})"


def _same(a, b):
    assert len(a) == len(b)
    for i, (u, v) in enumerate(zip(a, b)):
        assert u.shape == v.shape
        assert np.array_equal(u, v), f"step {i}: {int((u != v).sum())} of {u.size} differ"


@pytest.mark.parametrize("spec,C_", [(AFFINE, 10), (MXFP4, 5), (F16, 6), (SHARED, 12)],
                         ids=["affine-C10", "mxfp4-C5", "f16-C6", "shared-C12"])
def test_host_served_steps_bit_identical(gpu, spec, C_):
    import torch
    lay = make_layer(spec, seed=70, zipf=0.8)
    # decode steps of 1, 3 and 8 tokens, then prefill chunks (grouped GEMM tiles reading
    # absent experts from the host store)
    xs = [make_x(T, spec.hidden, seed=700 + i)
          for i, T in enumerate([1] * 20 + [3, 8, 1, 40, 1, 1, 77, 1])]
    print(f"[hostserve] {spec.quant.mode} E={spec.n_experts} C={C_} steps={len(xs)}", flush=True)
    moe_f, _, pool_f, _ = build_gpu_layer(lay, gpu)
    full = [moe_f(to_dev_bits(x, gpu)) for x in xs]
    torch.cuda.synchronize()
    full = [bits(o) for o in full]
    pool_f.close()
    moe, sw, pool, store = _host_served(lay, gpu, C_)
    outs = [moe(to_dev_bits(x, gpu)) for x in xs]
    torch.cuda.synchronize()
    _same([bits(o) for o in outs], full)
    _check_settled(sw, pool, store)
    assert pool.admits > 0 and pool.evicts > 0, pool.stats()
    assert sw.sync_seconds == 0.0, "the host never waited for the routing"
    # more steps on the settled pool
    more = [make_x(1, spec.hidden, seed=800 + i) for i in range(6)]
    outs = [moe(to_dev_bits(x, gpu)) for x in more]
    torch.cuda.synchronize()
    moe_f, _, pool_f, _ = build_gpu_layer(lay, gpu)
    ref = [moe_f(to_dev_bits(x, gpu)) for x in more]
    torch.cuda.synchronize()
    _same([bits(o) for o in outs], [bits(o) for o in ref])
    pool_f.close()
    pool.close()


def test_host_served_unreduced_rows_bit_identical(gpu):
    """The operator's own call (explicit routing, unreduced rows) on the host-served path."""
    import torch

    import oracle
    spec = AFFINE
    lay = make_layer(spec, seed=71)
    _, sw_f, pool_f, _ = build_gpu_layer(lay, gpu)
    _, sw, pool, store = _host_served(lay, gpu, 9)
    got, ref = [], []
    for T, seed in ((1, 1), (8, 2), (1, 3), (64, 4), (1, 5), (2, 6)):
        x = make_x(T, spec.hidden, seed=900 + seed)
        _, idx, _, _ = oracle.router(x, lay.router, False, None, spec.top_k, spec.route_mode)
        ti = torch.from_numpy(idx).to(gpu)
        got.append(sw(to_dev_bits(x, gpu), ti))
        ref.append(sw_f(to_dev_bits(x, gpu), ti))
    torch.cuda.synchronize()
    _same([bits(y) for y in got], [bits(y) for y in ref])
    _check_settled(sw, pool, store)
    pool_f.close()
    pool.close()


def test_host_backing_refusals(gpu):
    """Pageable memory, a short region, a used pool and calls without backing are refused
    before anything reaches a kernel."""
    import torch
    spec = F16
    lib = L.load()
    per = spec.bytes_per_expert
    E = spec.n_experts
    pool = ExpertPool(0, spec, 4).build()
    h = pool.device.handle
    pageable = np.zeros(E * per + 256, dtype=np.uint8)
    base = (pageable.ctypes.data + 255) & ~255
    assert lib.brx_pool_set_host_backing(h, base, per, E * per) != 0
    assert b"pinned" in L.load().brx_last_error() or b"runtime" in L.load().brx_last_error()
    pinned = torch.empty((E, per), dtype=torch.uint8, pin_memory=True)
    assert lib.brx_pool_set_host_backing(h, pinned.data_ptr(), per, per * (E - 1)) != 0
    assert lib.brx_pool_set_host_backing(h, pinned.data_ptr(), per - 256, per * E) != 0
    one = (C.c_int32 * 1)(0)
    assert lib.brx_pool_publish_async(h, 1, one, one, None) != 0          # no backing yet
    assert lib.brx_pool_admit_async(h, 0, 0, pinned.data_ptr(), per, None) != 0
    L.check(lib.brx_pool_set_host_backing(h, pinned.data_ptr(), per, pinned.numel()))
    assert lib.brx_pool_set_host_backing(h, pinned.data_ptr(), per, pinned.numel()) != 0
    bad = (C.c_int32 * 1)(E)
    assert lib.brx_pool_publish_async(h, 1, bad, one, None) != 0         # expert out of range
    assert lib.brx_pool_admit_async(h, 0, 4, pinned.data_ptr(), per, None) != 0   # slot
    assert lib.brx_pool_admit_async(h, 0, 0, pinned.data_ptr(), per - 1, None) != 0  # size
    torch.cuda.synchronize()
    pool.close()
    used = ExpertPool(0, spec, 4).build()
    used.device.set_table(np.full(E, -1, np.int32), torch.cuda.current_stream().cuda_stream)
    assert lib.brx_pool_set_host_backing(used.device.handle, pinned.data_ptr(), per,
                                         pinned.numel()) != 0
    torch.cuda.synchronize()
    used.close()
