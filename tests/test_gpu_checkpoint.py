"""A layer loaded from an MLX checkpoint's safetensors shards into the pinned host store, served
by a bounded HBM pool (refills on misses) and run through the kernels: routing indices
bit-exact and outputs within 1e-2 relative L2 of the oracle on the experts read back from the
checkpoint."""
import numpy as np
import pytest

import oracle
from bigrig_amd import checkpoint as CK
from bigrig_amd import formats as F
from bigrig_amd.layer import MoELayer, StreamingSwitchGLU
from bigrig_amd.pool import ExpertPool, HostStore, PinnedFetcher
from tests.ckpt_util import make_checkpoint
from tests.gpu_util import bits, to_dev_bits
from tests.helpers import make_x

pytestmark = pytest.mark.gpu

QWEN = ({"model_type": "qwen3_moe", "num_experts_per_tok": 4, "norm_topk_prob": True,
         "quantization": {"group_size": 64, "bits": 4}}, F.QuantSpec(4, 64, "affine"), False,
        ".mlp.switch_mlp.", (512, 256))
GPTOSS = ({"model_type": "gpt_oss", "num_experts_per_tok": 4, "swiglu_limit": 7.0,
           "quantization": {"group_size": 32, "bits": 4, "mode": "mxfp4"}},
          F.QuantSpec(4, 32, "mxfp4"), True, ".mlp.experts.", (576, 320))


@pytest.mark.parametrize("case", [QWEN, GPTOSS], ids=["qwen3-affine", "gptoss-mxfp4"])
def test_checkpoint_layer_on_the_gpu(gpu, tmp_path, case):
    cfg, q, has_bias, infix, (H, I) = case
    E, C = 16, 6
    d = str(tmp_path / "ckpt")
    make_checkpoint(d, {0: (H, I, E, q, has_bias)}, infix=infix, config=cfg, shards=2, seed=5)
    man = CK.expert_manifest(d)
    spec = CK.layer_spec(man, 0)
    store = HostStore.from_checkpoint(man)
    experts = [CK.read_expert(man, 0, e) for e in range(E)]
    for e in (0, E - 1):
        assert store.tensor(0)[e].numpy().tobytes() == experts[e]
    rng = np.random.default_rng(11)
    router = F.f32_to_bf16_bits(rng.standard_normal((E, H), dtype=np.float32) * 0.02)
    pool = ExpertPool(0, spec, C).build()
    sw = StreamingSwitchGLU(pool, PinnedFetcher(store))
    moe = MoELayer(spec, to_dev_bits(router, gpu), sw)
    for T in (1, 7, 40):
        print(f"[checkpoint] {spec.quant.mode} H={H} I={I} E={E} C={C} T={T}", flush=True)
        x = make_x(T, H, seed=300 + T)
        _, idx, w, _ = oracle.router(x, router, False, None, spec.top_k, spec.route_mode)
        gidx, _, _ = moe.route(to_dev_bits(x, gpu))
        assert np.array_equal(gidx.cpu().numpy(), idx)
        out = moe(to_dev_bits(x, gpu))
        ref, _ = oracle.moe_forward(spec, experts, x, idx, w)
        r = oracle.rel_l2(F.bf16_bits_to_f32(bits(out)), F.bf16_bits_to_f32(ref))
        assert r < 1e-2, f"T={T}: rel L2 {r:.3e}"
    assert pool.admits > C, "a bounded pool refilled slots from the checkpoint-backed store"
    pool.close()
