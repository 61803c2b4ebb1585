"""Layer-major prefill over a ring of whole layers (bigrig_amd/layered.py): the next layer's
experts are copied from pinned host memory while this layer's chunks run, and every row comes
out bit-identical to a token-major pass (each chunk through every layer before the next chunk,
every expert resident), with or without the read-ahead. The first layer is checked against the
oracle at 1e-2 relative L2."""
import numpy as np
import pytest

import oracle
from bigrig_amd import formats as F
from bigrig_amd import layer as ops
from bigrig_amd import layered
from bigrig_amd.pool import ExpertPool, HostStore
from bigrig_amd.spec import QWEN3_30B_A3B
from tests.gpu_util import bits, to_dev_bits
from tests.helpers import make_layer, make_x, small

pytestmark = pytest.mark.gpu


def test_layer_major_prefill_matches_token_major(gpu):
    import torch
    spec = small(QWEN3_30B_A3B, hidden=512, inter=256, n_experts=16, top_k=8)
    nl = 4
    lays = [make_layer(spec, seed=40 + l, zipf=1.1) for l in range(nl)]
    store = HostStore()
    for l, lay in enumerate(lays):
        store.add_layer(10 + l, lay.experts)           # store ids need not be 0..n-1
    ws = [layered.MoEWeights(10 + l, to_dev_bits(lay.router, gpu), to_dev_bits(lay.bias, gpu))
          for l, lay in enumerate(lays)]
    sizes = (40, 33, 5, 70)
    xs = [to_dev_bits(make_x(T, spec.hidden, seed=90 + T), gpu) for T in sizes]
    print(f"[layered] H={spec.hidden} E={spec.n_experts} layers={nl} chunks={sizes}", flush=True)

    ring = layered.LayerRing(spec, depth=2)
    got = layered.prefill(spec, ws, store, [x.clone() for x in xs], ring)
    ring.reset()
    serial = layered.prefill(spec, ws, store, [x.clone() for x in xs], ring, read_ahead=False)
    torch.cuda.synchronize()
    assert ring.bytes_loaded == 2 * nl * spec.n_experts * spec.bytes_per_expert

    # token-major: each chunk through every layer, each layer fully resident in its own pool
    pools = []
    for l in range(nl):
        pool = ExpertPool(10 + l, spec, spec.n_experts).build()
        for e in range(spec.n_experts):
            pool.touch([e], [0])
            pool.admit(e, store.region(10 + l, e))
        pool.g2s_device(torch.cuda.current_stream().cuda_stream)
        pools.append(pool)
    for j, x in enumerate(xs):
        h = x.clone()
        for l in range(nl):
            out = ops.moe_block(spec, pools[l], h, ws[l].router, ws[l].router_bias,
                                flags=ops.path_flag(h.shape[0], spec.top_k))
            if l == 0:
                xb = bits(h)
                _, idx, w, _ = oracle.router(xb, lays[0].router, False, lays[0].bias, spec.top_k,
                                             spec.route_mode)
                ref, _ = oracle.moe_forward(spec, lays[0].experts, xb, idx, w)
                r = oracle.rel_l2(F.bf16_bits_to_f32(bits(out)), F.bf16_bits_to_f32(ref))
                assert r < 1e-2, f"chunk {j} layer 0: rel L2 {r:.3e}"
            h = out + h
        torch.cuda.synchronize()
        assert np.array_equal(bits(got[j]), bits(h)), f"chunk {j}: layer-major differs"
        assert np.array_equal(bits(serial[j]), bits(h)), f"chunk {j}: serial schedule differs"
    for p in pools:
        p.close()
    ring.close()
