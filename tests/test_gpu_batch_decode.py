"""Batched decode (8 tokens at top-8) when the tokens share experts.

The step's pairs are planned once and merged per expert into entries of at most 4 pairs, so an
expert chosen by all 8 tokens is read by two entries, and the shared expert's 8 tokens are two
groups of 4. Outputs are checked against the oracle, and a token's row must not depend on which
other tokens share the step: the same tokens in another order give the same bits, row for row.
"""
import numpy as np
import pytest

import oracle
from bigrig_amd import formats as F
from bigrig_amd import layer as ops
from bigrig_amd import lib as L
from bigrig_amd.spec import E256_SHARED, GPT_OSS_120B, QWEN3_30B_A3B
from tests.gpu_util import bits, build_gpu_layer, to_dev_bits
from tests.helpers import make_layer, make_x, small

pytestmark = pytest.mark.gpu

TOL = 1e-2
AFFINE = small(QWEN3_30B_A3B, hidden=512, inter=256, n_experts=32, top_k=8)
MXFP4_K8 = small(GPT_OSS_120B, hidden=576, inter=320, n_experts=16, top_k=8)
SHARED = small(E256_SHARED, hidden=512, inter=256, n_experts=64, top_k=8, shared_inter=256)


def _forward(spec, pool, sw, x, idx, w, sg, gpu):
    import torch
    T = x.shape[0]
    out = torch.empty((T, spec.hidden), dtype=torch.bfloat16, device=gpu)
    shared = sw.shared if spec.shared_inter else None
    sgd = torch.from_numpy(sg).to(gpu) if shared is not None else None
    ops.moe_forward(spec, pool, to_dev_bits(x, gpu), torch.from_numpy(idx).to(gpu),
                    torch.from_numpy(w).to(gpu), shared, sgd, out=out, flags=L.FWD_FORCE_DECODE)
    torch.cuda.synchronize()
    return bits(out)


@pytest.mark.parametrize("spec", [AFFINE, MXFP4_K8, SHARED], ids=["affine", "mxfp4", "shared"])
@pytest.mark.parametrize("overlap", ["all", "half"])
def test_shared_experts_across_tokens(gpu, spec, overlap):
    import torch
    T, k, E = 8, spec.top_k, spec.n_experts
    lay = make_layer(spec, seed=61)
    _, sw, pool, _ = build_gpu_layer(lay, gpu)
    pool.g2s_device(torch.cuda.current_stream().cuda_stream)
    rng = np.random.default_rng(62)
    common = rng.choice(E, size=k, replace=False)
    idx = np.empty((T, k), np.int32)
    for t in range(T):
        if overlap == "all":        # every token: the same experts, each in its own order
            idx[t] = rng.permutation(common)
        else:                       # half of each token's experts common, the rest its own
            own = rng.choice(np.setdiff1d(np.arange(E), common), size=k - k // 2, replace=False)
            idx[t] = rng.permutation(np.concatenate([common[:k // 2], own]))
    w = rng.random((T, k)).astype(np.float32)
    w /= w.sum(axis=1, keepdims=True)
    sg = rng.random(T).astype(np.float32)
    x = make_x(T, spec.hidden, seed=63)
    got = _forward(spec, pool, sw, x, idx, w, sg, gpu)
    ref, _ = oracle.moe_forward(spec, lay.experts, x, idx, w, lay.shared,
                                sg if spec.shared_inter else None)
    r = oracle.rel_l2(F.bf16_bits_to_f32(got), F.bf16_bits_to_f32(ref))
    assert r < TOL, f"rel L2 vs C oracle {r:.3e}"
    perm = rng.permutation(T)
    got_p = _forward(spec, pool, sw, x[perm], idx[perm], w[perm], sg[perm], gpu)
    assert np.array_equal(got_p, got[perm])
    pool.close()
