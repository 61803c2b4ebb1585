"""The bounded HBM pool on the GPU: outputs at capacity C < E are bit-identical to C = E.

The reference's central invariant (bigrig_engine/stream.py:25-30; tests/test_stream.py:530-545):
streaming experts through a pool smaller than the layer changes where the bytes live, never
the arithmetic. Covered here for decode (one token a step, evicting and refilling between
steps), batched decode and prefill chunks that route to more experts than the pool holds (the
expert-sorted span path, stream.py:1521-1561), the shared expert, MXFP4 with biases, and the
operator's unreduced rows. Refills run on the pool's own copy stream; every step is issued
back to back with no host synchronisation other than the routing read the path itself makes.
"""
import numpy as np
import pytest

from bigrig_amd import formats as F
from bigrig_amd.spec import E256_SHARED, GPT_OSS_120B, OLMOE_1B_7B, QWEN3_30B_A3B
from tests.gpu_util import bits, build_gpu_layer, to_dev_bits
from tests.helpers import make_layer, make_x, small

pytestmark = pytest.mark.gpu

AFFINE = small(QWEN3_30B_A3B, hidden=512, inter=256, n_experts=32, top_k=8)
SHARED = small(E256_SHARED, hidden=512, inter=256, n_experts=32, top_k=8, shared_inter=256)
MXFP4 = small(GPT_OSS_120B, hidden=576, inter=320, n_experts=16, top_k=4)
F16 = small(OLMOE_1B_7B, hidden=512, inter=256, n_experts=16, top_k=4,
            quant=F.QuantSpec(4, 64, "affine", "float16"))


def _run(lay, gpu, C, xs):
    import torch
    moe, sw, pool, _ = build_gpu_layer(lay, gpu, capacity=C)
    outs = [moe(to_dev_bits(x, gpu)) for x in xs]
    torch.cuda.synchronize()
    res = [bits(o) for o in outs]
    st = pool.stats()
    st["chunked"] = sw.chunked_calls
    pool.close()
    return res, st


def _same(a, b):
    assert len(a) == len(b)
    for i, (u, v) in enumerate(zip(a, b)):
        assert u.shape == v.shape
        assert np.array_equal(u, v), f"step {i}: {int((u != v).sum())} of {u.size} differ"


@pytest.mark.parametrize("spec,C", [(AFFINE, 10), (AFFINE, 8), (MXFP4, 5), (F16, 6)],
                         ids=["affine-C10", "affine-C8", "mxfp4-C5", "f16-C6"])
def test_decode_steps_bit_identical(gpu, spec, C):
    lay = make_layer(spec, seed=40, zipf=0.8)
    xs = [make_x(1, spec.hidden, seed=400 + i) for i in range(24)]
    full, _ = _run(lay, gpu, spec.n_experts, xs)
    bounded, st = _run(lay, gpu, C, xs)
    _same(bounded, full)
    assert st["evicts"] > 0 and st["chunked"] == 0


@pytest.mark.parametrize("spec,C,T", [(AFFINE, 10, 8), (AFFINE, 12, 64), (AFFINE, 9, 257),
                                      (SHARED, 12, 8), (SHARED, 12, 40), (MXFP4, 5, 33)],
                         ids=["dec8-C10", "pf64-C12", "pf257-C9", "shared-dec8", "shared-pf40",
                              "mxfp4-pf33"])
def test_span_path_bit_identical(gpu, spec, C, T):
    """A chunk routing to more than C experts is split into expert-sorted spans."""
    lay = make_layer(spec, seed=41)
    xs = [make_x(T, spec.hidden, seed=500 + T + i) for i in range(3)]
    full, _ = _run(lay, gpu, spec.n_experts, xs)
    bounded, st = _run(lay, gpu, C, xs)
    assert st["chunked"] == len(xs), "the chunk should have needed more experts than C"
    _same(bounded, full)


def test_unreduced_rows_bit_identical(gpu):
    import torch

    import oracle
    spec = AFFINE
    lay = make_layer(spec, seed=42)
    rows = {}
    for C in (spec.n_experts, 11):
        _, sw, pool, _ = build_gpu_layer(lay, gpu, capacity=C)
        got = []
        for T, seed in ((1, 1), (8, 2), (64, 3)):
            x = make_x(T, spec.hidden, seed=600 + seed)
            _, idx, _, _ = oracle.router(x, lay.router, False, None, spec.top_k,
                                         spec.route_mode)
            y = sw(to_dev_bits(x, gpu), torch.from_numpy(idx).to(gpu))
            got.append(bits(y))
        torch.cuda.synchronize()
        rows[C] = got
        pool.close()
    _same(rows[11], rows[spec.n_experts])


def test_pool_slots_hold_the_admitted_bytes(gpu):
    """After a churn of admissions each slot holds the expert the host table says lives there
    (no refill lost, none written to the wrong slot): the slot's bytes, dequantized in place
    by the library, equal that expert's weights from the oracle bit for bit."""
    import ctypes as C

    import torch

    import oracle
    from bigrig_amd import lib as L
    spec = F16
    lay = make_layer(spec, seed=43)
    _, sw, pool, _ = build_gpu_layer(lay, gpu, capacity=5)
    rng = np.random.default_rng(0)
    for _ in range(40):
        want = np.sort(rng.choice(spec.n_experts, size=4, replace=False))
        sw.ensure(want[None, :])
    assert pool.evicts > 0
    d = spec.desc()
    stream = torch.cuda.current_stream()
    pool.device.sync()
    for slot in range(pool.capacity):
        e = int(pool.s2g[slot])
        assert e >= 0 and pool.g2s[e] == slot
        for p in (0, 2):
            n_out, n_in = (spec.inter, spec.hidden) if p == 0 else (spec.hidden, spec.inter)
            out = torch.empty((n_out, n_in), dtype=torch.float32, device=gpu)
            L.check(L.load().brx_dequant(C.byref(d), pool.device.slot_ptr(slot), p, 0,
                                         out.data_ptr(), stream.cuda_stream))
            want = oracle.dequant(spec, lay.experts[e], p)
            got = out.cpu().numpy()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (slot, e, p)
    pool.close()


def test_refill_range_lands_every_expert(gpu):
    """brx_pool_refill_range_async: one transfer when the experts are back to back on both
    sides, one copy per expert otherwise (a padded host stride); every slot then holds its
    expert's bytes, and a bad range is refused before anything is copied."""
    import ctypes as C

    import torch

    from bigrig_amd import lib as L
    from bigrig_amd.pool import ExpertPool
    spec = F16
    per = spec.bytes_per_expert
    E = spec.n_experts
    rng = np.random.default_rng(5)
    src = rng.integers(0, 256, (E, per), dtype=np.uint8)
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    for pad in (0, 512):
        host = torch.empty((E, per + pad), dtype=torch.uint8, pin_memory=True)
        host.numpy()[:, :per] = src
        pool = ExpertPool(0, spec, E).build()
        n = pool.device.write_range(0, host.data_ptr(), E, per + pad, per)
        assert n == E * per
        pool.device.sync()
        for e in (0, 1, E // 2, E - 1):
            out = (C.c_uint8 * per)()
            assert hip.hipMemcpy(out, C.c_void_p(pool.device.slot_ptr(e)), per, 2) == 0
            assert bytes(out) == src[e].tobytes(), (pad, e)
        lib = L.load()
        s = torch.cuda.current_stream().cuda_stream
        assert lib.brx_pool_refill_range_async(pool.device.handle, 1, E, host.data_ptr(),
                                               per + pad, per, s) != 0       # past the pool
        assert lib.brx_pool_refill_range_async(pool.device.handle, 0, 2, host.data_ptr(),
                                               per + pad, per - 1, s) != 0   # wrong size
        pool.close()
