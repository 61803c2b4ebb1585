"""The CPU baseline bench.py times (oracle/cpu_baseline.c: fp32 dequant-on-the-fly GEMVs with
OpenMP) computes the real layer: one decode token's output matches the oracle's within 1e-2
relative L2 (the two accumulate in different orders; the baseline never rounds h to bf16), on
4-bit affine layers with bf16 and fp16 scales, with and without renormalised weights."""
import numpy as np
import pytest

import oracle
from bigrig_amd import formats as F
from bigrig_amd.spec import OLMOE_1B_7B, QWEN3_30B_A3B
from tests.helpers import make_layer, make_x, small


@pytest.mark.parametrize("spec", [
    small(QWEN3_30B_A3B, hidden=512, inter=256, n_experts=16, top_k=4),
    small(QWEN3_30B_A3B, hidden=512, inter=128, n_experts=32, top_k=8,
          quant=F.QuantSpec(4, 64, "affine", "float16")),
    small(OLMOE_1B_7B, hidden=256, inter=128, n_experts=8, top_k=2, router_dtype="bfloat16"),
], ids=["qwen3-small", "fp16-scales", "no-renorm"])
def test_cpu_baseline_matches_the_oracle(spec):
    lay = make_layer(spec, seed=31, zipf=0.7)
    blob = np.stack([np.frombuffer(b, np.uint8) for b in lay.experts])
    assert blob.shape == (spec.n_experts, spec.bytes_per_expert)
    for t in range(3):
        x = make_x(1, spec.hidden, seed=310 + t)
        got = oracle.cpu_baseline_decode(spec, x, lay.router, lay.bias, blob.ctypes.data,
                                         blob.shape[1], nthreads=2)
        _, idx, w, _ = oracle.router(x, lay.router, False, lay.bias, spec.top_k, spec.route_mode)
        ref, _ = oracle.moe_forward(spec, lay.experts, x, idx, w)
        r = oracle.rel_l2(F.bf16_bits_to_f32(got), F.bf16_bits_to_f32(ref[0]))
        assert r < 1e-2, f"token {t}: rel L2 {r:.3e}"


def test_cpu_baseline_refuses_other_layouts():
    spec = small(QWEN3_30B_A3B, hidden=256, inter=128, n_experts=8, top_k=2,
                 quant=F.QuantSpec(3, 64, "affine", "bfloat16"))
    with pytest.raises(ValueError):
        oracle.cpu_baseline_decode(spec, np.zeros((1, 256), np.uint16),
                                   np.zeros((8, 256), np.uint16), None, 0, 1)
