"""The workload's full-size layers on the GPU (every expert resident, synthetic weights generated
and quantized on the device, admitted through the pool's device path): every output is finite,
the whole call's routing matches the oracle (indices bit-exact, weights to 1e-5), and the layer
outputs of the compared tokens are within 1e-2 relative L2 of the oracle, as a whole and token by
token. Decode calls compare every token. A prefill chunk compares the tokens of the first and
last row of every 64-row run of every expert's bucket (`tile_edge_tokens`): the oracle cannot
run a whole 2048-token chunk in seconds, and those rows include the first and last row of every
M tile the grouped GEMM forms, for every expert the chunk hits.

The sizes: Qwen3-30B-A3B shape (hidden 2048, 128 experts, top-8, inter 768, 4-bit affine) for a
2048-token prefill chunk and a 1-token decode step; gpt-oss-120b shape (hidden 2880, 128
experts, top-4, inter 2880, MXFP4 + biases, clamped SwiGLU) for a 512-token chunk and one
decode token; 256 experts + shared expert (inter 512) at batch 8 and batch 1; the OLMoE-1B-7B
layer (hidden 2048, 64 experts, inter 1024, fp32 router, softmax top-8 without renormalisation)
at batch 1 and 8; the Qwen3 shape with unquantized bf16 experts (Qwen3-30B-A3B-bf16, 9.4 MB per
expert) for a 2048-token chunk and decode at batch 1 and 8. The Qwen3 and 256-expert routers
carry the Zipf(1.1) bias, the others none.
"""
import numpy as np
import pytest

import oracle
from bigrig_amd import formats as F
from bigrig_amd import layer as ops
from bigrig_amd.spec import E256_SHARED, GPT_OSS_120B, OLMOE_1B_7B, QWEN3_30B_A3B, QWEN3_30B_A3B_BF16
from tests.gpu_util import per_token_rel_l2, tile_edge_tokens

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _bits(t):
    import torch
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


# the configurations with a Zipf-biased router (Qwen3-30B-A3B shape and the 256-expert layer);
# the OLMoE and gpt-oss layers route on the plain logits
ZIPF = {QWEN3_30B_A3B: 1.1, E256_SHARED: 1.1, QWEN3_30B_A3B_BF16: 1.1}


def _layer(spec, seed):
    """(pool, experts uint8 [E, bytes] on the GPU, router w, Zipf bias or None, shared, shared
    gate w)."""
    import torch

    from bigrig_amd import synth
    from bigrig_amd.pool import ExpertPool
    experts = synth.make_layer_experts(spec, seed=seed)
    pool = ExpertPool(0, spec, spec.n_experts).build()
    for e in range(spec.n_experts):
        pool.touch([e], [0])
        pool.admit_device(e, experts[e].data_ptr())
    pool.g2s_device(torch.cuda.current_stream().cuda_stream)
    pool.device.sync()
    wr = synth.router_weights(spec, seed=seed + 1)
    bias = (synth.zipf_bias_torch(spec.n_experts, ZIPF[spec], seed=seed + 2) if spec in ZIPF
            else None)
    shared = sgw = None
    if spec.shared_inter:
        shared = synth.make_layer_experts(spec, seed=seed + 3, shared=True)[0].contiguous()
        g = torch.Generator(device="cuda")
        g.manual_seed(seed + 4)
        sgw = (torch.randn(spec.hidden, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    return pool, experts, wr, bias, shared, sgw


@pytest.mark.parametrize("spec,T", [(QWEN3_30B_A3B, 2048), (QWEN3_30B_A3B, 1), (GPT_OSS_120B, 512),
                                    (GPT_OSS_120B, 1), (E256_SHARED, 8), (E256_SHARED, 1),
                                    (OLMOE_1B_7B, 1), (OLMOE_1B_7B, 8), (QWEN3_30B_A3B_BF16, 2048),
                                    (QWEN3_30B_A3B_BF16, 1), (QWEN3_30B_A3B_BF16, 8)],
                         ids=["qwen3-prefill2048", "qwen3-decode1", "gptoss-prefill512",
                              "gptoss-decode1", "e256shared-decode8", "e256shared-decode1",
                              "olmoe-decode1", "olmoe-decode8", "qwen3bf16-prefill2048",
                              "qwen3bf16-decode1", "qwen3bf16-decode8"])
def test_full_size_layer(gpu, spec, T):
    import torch

    from bigrig_amd import synth
    print(f"[full-size] H={spec.hidden} E={spec.n_experts} I={spec.inter} T={T}", flush=True)
    pool, experts, wr, bias, shared, sgw = _layer(spec, seed=100 + T)
    x = synth.activations(T, spec.hidden, seed=200 + T)
    k = spec.top_k
    idx = torch.empty((T, k), dtype=torch.int32, device=gpu)
    w = torch.empty((T, k), dtype=torch.float32, device=gpu)
    out = ops.moe_block(spec, pool, x, wr, bias, sgw, shared, out_idx=idx, out_w=w,
                        flags=ops.path_flag(T, spec.top_k))
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out.float()).all()), "non-finite layer outputs"

    xb_all = _bits(x)
    wr_h = wr.cpu().numpy() if spec.router_dtype == "float32" else _bits(wr)
    sgw_h = None if sgw is None else _bits(sgw)
    _, oidx_all, ow_all, osg_all = oracle.router(xb_all, wr_h, spec.router_dtype == "float32",
                                                 None if bias is None else bias.cpu().numpy(), k,
                                                 spec.route_mode, sgw_h)
    assert np.array_equal(idx.cpu().numpy(), oidx_all), "routing indices differ from the oracle"
    np.testing.assert_allclose(w.cpu().numpy(), ow_all, rtol=1e-5, atol=1e-7)

    toks = tile_edge_tokens(oidx_all, spec.n_experts) if T > 8 else list(range(T))
    oidx, ow = oidx_all[toks], ow_all[toks]
    osg = None if osg_all is None else osg_all[toks]
    # only the compared tokens' experts travel to the host; the other entries alias one of them
    need = sorted(set(int(e) for e in oidx.reshape(-1)))
    host = {e: experts[e].cpu().numpy().tobytes() for e in need}
    elist = [host.get(e, host[need[0]]) for e in range(spec.n_experts)]
    sh = None if shared is None else shared.cpu().numpy().tobytes()
    print(f"[full-size] oracle over {len(toks)} tokens, {len(need)} experts", flush=True)
    ref, _ = oracle.moe_forward(spec, elist, xb_all[toks], oidx, ow, sh, osg)
    got = F.bf16_bits_to_f32(_bits(out)[toks])
    want = F.bf16_bits_to_f32(ref)
    assert np.abs(want).max() > 1e-3, "degenerate layer: the oracle output is (near) zero"
    r = oracle.rel_l2(got, want)
    rt = per_token_rel_l2(got, want)
    worst = int(np.argmax(rt))
    print(f"[full-size] {len(toks)} tokens: rel L2 {r:.2e}, worst token {toks[worst]} "
          f"{rt[worst]:.2e}", flush=True)
    assert r < TOL, f"rel L2 {r:.3e} against the oracle"
    assert rt[worst] < TOL, f"token {toks[worst]}: rel L2 {rt[worst]:.3e} against the oracle"
    pool.close()
    del experts
    torch.cuda.empty_cache()
