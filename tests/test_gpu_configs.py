"""The workload's configurations as specified, at their real shapes on the GPU:

* the OLMoE-1B-7B layer (hidden 2048, 64 experts, inter 1024, fp32 router, softmax top-8 without
  renormalisation, no router bias) over 256 seeded decode steps: every step's routing bit-exact
  against the oracle, every output finite, sampled steps within 1e-2 of the oracle;
* the Qwen3-30B-A3B layer through a 32-of-128-slot pool and the 256-expert + shared layer
  through a 38-of-256-slot pool (Zipf(1.1) router bias), on both bounded paths -- the host
  routing read with refills from pinned memory, and host-served misses -- each bit-identical to
  the fully resident layer over 96 decode steps with fresh inputs, enough for both pools to
  evict (the reference's central invariant, stream.py:25-30), with routing bit-exact against
  the oracle on every step and sampled steps within 1e-2.

Weights are generated and quantized on the GPU (`synth`); the pinned host store the bounded
pools refill from is a copy of the same bytes.
"""
import numpy as np
import pytest

import oracle
from bigrig_amd import formats as F
from bigrig_amd import synth
from bigrig_amd.layer import MoELayer, StreamingSwitchGLU
from bigrig_amd.pool import ExpertPool, HostStore, PinnedFetcher
from bigrig_amd.spec import E256_SHARED, OLMOE_1B_7B, QWEN3_30B_A3B

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _bits(t):
    import torch
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


class _Full:
    """A full-shape synthetic layer: experts on the GPU and in pinned host memory."""

    def __init__(self, spec, seed, zipf):
        import torch
        self.spec = spec
        self.experts = synth.make_layer_experts(spec, seed=seed)
        self.router = synth.router_weights(spec, seed=seed + 1)
        self.bias = synth.zipf_bias_torch(spec.n_experts, zipf, seed=seed + 2) if zipf else None
        self.shared = self.sgw = None
        if spec.shared_inter:
            self.shared = synth.make_layer_experts(spec, seed=seed + 3, shared=True)[0].contiguous()
            g = torch.Generator(device="cuda")
            g.manual_seed(seed + 4)
            self.sgw = (torch.randn(spec.hidden, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
        pinned = torch.empty(tuple(self.experts.shape), dtype=torch.uint8, pin_memory=True)
        pinned.copy_(self.experts)
        self.store = HostStore()
        self.store.add_layer_tensor(0, pinned)

    def moe(self, capacity, host_served=False):
        import torch
        spec = self.spec
        pool = ExpertPool(0, spec, capacity).build()
        if capacity == spec.n_experts:
            for e in range(spec.n_experts):
                pool.touch([e], [0])
                pool.admit_device(e, self.experts[e].data_ptr())
            pool.g2s_device(torch.cuda.current_stream().cuda_stream)
        sw = StreamingSwitchGLU(pool, PinnedFetcher(self.store), shared=self.shared,
                                host_served=host_served)
        sw.refresh()
        return MoELayer(spec, self.router, sw, router_bias=self.bias,
                        shared_gate_w=self.sgw if self.shared is not None else None), pool, sw

    def oracle_check(self, x, out, idx_dev=None):
        """Routing of x bit-exact against the oracle (when idx_dev given) and out within TOL."""
        spec = self.spec
        xb = _bits(x)
        wr = (self.router.cpu().numpy() if spec.router_dtype == "float32" else _bits(self.router))
        bias = None if self.bias is None else self.bias.cpu().numpy()
        sgw = None if self.sgw is None else _bits(self.sgw)
        _, oidx, ow, osg = oracle.router(xb, wr, spec.router_dtype == "float32", bias,
                                         spec.top_k, spec.route_mode, sgw)
        if idx_dev is not None:
            assert np.array_equal(idx_dev, oidx), "routing indices differ from the oracle"
        need = sorted({int(e) for e in oidx.reshape(-1)})
        host = {e: self.experts[e].cpu().numpy().tobytes() for e in need}
        elist = [host.get(e, host[need[0]]) for e in range(spec.n_experts)]
        sh = None if self.shared is None else self.shared.cpu().numpy().tobytes()
        ref, _ = oracle.moe_forward(spec, elist, xb, oidx, ow, sh, osg)
        want = F.bf16_bits_to_f32(ref)
        assert np.abs(want).max() > 1e-3, "degenerate layer: the oracle output is (near) zero"
        r = oracle.rel_l2(F.bf16_bits_to_f32(_bits(out)), want)
        assert r < TOL, f"rel L2 {r:.3e} against the oracle"
        return oidx


def test_olmoe_layer_256_seeded_steps(gpu):
    import torch
    spec = OLMOE_1B_7B
    lay = _Full(spec, seed=700, zipf=0.0)
    moe, pool, _ = lay.moe(spec.n_experts)
    steps = 256
    xs = [synth.activations(1, spec.hidden, seed=7000 + i) for i in range(steps)]
    print(f"[configs] OLMoE layer, {steps} decode steps", flush=True)
    outs, idxs = [], []
    for x in xs:
        idx, _, _ = moe.route(x)
        idxs.append(idx)
        outs.append(moe(x))
    torch.cuda.synchronize()
    gidx = np.concatenate([i.cpu().numpy() for i in idxs])
    xb = np.concatenate([_bits(x) for x in xs])
    _, oidx, _, _ = oracle.router(xb, lay.router.cpu().numpy(), True, None, spec.top_k,
                                  spec.route_mode)
    assert np.array_equal(gidx, oidx), "routing indices differ from the oracle"
    assert all(bool(torch.isfinite(o.float()).all()) for o in outs), "non-finite outputs"
    for i in (0, 97, 255):
        lay.oracle_check(xs[i], outs[i])
    print(f"[configs] OLMoE: {len(np.unique(oidx))} of 64 experts used", flush=True)
    pool.close()


@pytest.mark.parametrize("spec,C", [(QWEN3_30B_A3B, 32), (E256_SHARED, 38)],
                         ids=["qwen3-C32", "e256shared-C38"])
def test_bounded_pool_full_shape_bit_identical(gpu, spec, C):
    import torch
    lay = _Full(spec, seed=710 + C, zipf=1.1)
    steps = 96
    xs = [synth.activations(1, spec.hidden, seed=7100 + i) for i in range(steps)]
    print(f"[configs] H={spec.hidden} E={spec.n_experts} I={spec.inter} C={C}: resident", flush=True)
    full, fpool, _ = lay.moe(spec.n_experts)
    ref, ridx = [], []
    for x in xs:
        idx, _, _ = full.route(x)
        ridx.append(idx.cpu().numpy())
        ref.append(_bits(full(x)))
    torch.cuda.synchronize()
    fpool.close()
    for hs in (False, True):
        print(f"[configs] C={C} {'host-served' if hs else 'host routing read'}", flush=True)
        moe, pool, sw = lay.moe(C, host_served=hs)
        outs = [moe(x) for x in xs]
        torch.cuda.synchronize()
        for i, o in enumerate(outs):
            b = _bits(o)
            assert np.array_equal(b, ref[i]), f"step {i}: {int((b != ref[i]).sum())} differ"
        st = pool.stats()
        print(f"[configs] C={C} hs={hs}: misses {st['misses']} evicts {st['evicts']}", flush=True)
        assert st["evicts"] > 0 and sw.chunked_calls == 0
        pool.close()
    for i in range(steps):
        if i in (0, steps - 1):
            lay.oracle_check(xs[i], torch.from_numpy(ref[i].view(np.int16)).view(torch.bfloat16),
                             ridx[i])
        else:
            xb = _bits(xs[i])
            sgw = None if lay.sgw is None else _bits(lay.sgw)
            _, oidx, _, _ = oracle.router(xb, _bits(lay.router), False, lay.bias.cpu().numpy(),
                                          spec.top_k, spec.route_mode, sgw)
            assert np.array_equal(ridx[i], oidx), f"step {i}: routing differs from the oracle"
