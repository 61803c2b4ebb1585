"""A row of the prefill GEMM gives the same bits whatever tile it lands in.

The grouped GEMM cuts each expert's rows into M tiles of 128 rows, its last tile 32, 64 or 128
rows high by what is left. A row's output must not depend on the tile height or on which pairs
share its tile: the reference's central invariant is that a layer's rows do not depend on how a
step is split (bigrig_engine/stream.py:25-30; spans, stream.py:1521-1561). Here every pair of a
chunk runs once as one pair list (hot experts in full 128-row tiles), then again as pair lists of
at most 48 pairs per expert (every row in a 64-row or 32-row tile, at other tile boundaries),
both through brx_moe_forward_pairs with the shared expert's pairs included, and every row is
compared bit for bit. The block's outputs are also checked against the oracle: on the full-size
chunk on the tile-edge tokens (the first and last row of every M tile of every expert), on the
small layers on every token.
"""
import numpy as np
import pytest

import oracle
from bigrig_amd import formats as F
from bigrig_amd import layer as ops
from bigrig_amd import lib as L
from bigrig_amd.spec import E256_SHARED, QWEN3_30B_A3B, QWEN3_30B_A3B_3BIT
from tests.gpu_util import bits, build_gpu_layer, per_token_rel_l2, tile_edge_tokens, to_dev_bits
from tests.helpers import make_layer, make_x, small

pytestmark = pytest.mark.gpu

TOL = 1e-2
SPLIT = 48   # pairs per expert in a split list: 64- and 32-row tiles, boundaries unlike 128's


def _whole_vs_split(spec, pool, x, idx, shared=None):
    """Every pair of the chunk (routed pairs p = t * k + j, then one shared-expert pair per token
    when `shared` is given) through brx_moe_forward_pairs: once as a single list and once as
    lists of at most SPLIT pairs per expert. Returns (whole rows, split rows, the largest
    expert's pair count)."""
    import torch
    T, k = idx.shape
    H, E = spec.hidden, spec.n_experts
    dev = x.device
    idx_h = idx.cpu().numpy() if hasattr(idx, "cpu") else np.asarray(idx)
    pexp = idx_h.reshape(-1).astype(np.int32)
    ptok = np.repeat(np.arange(T, dtype=np.int32), k)
    if shared is not None:
        pexp = np.concatenate([pexp, np.full(T, E, np.int32)])
        ptok = np.concatenate([ptok, np.arange(T, dtype=np.int32)])
    rows = pexp.size
    rank = np.zeros(rows, np.int64)
    for e in np.unique(pexp):
        q = np.flatnonzero(pexp == e)
        rank[q] = np.arange(q.size)

    def run(sel):
        sel = sel.astype(np.int32)
        ops.forward_pairs(spec, pool, x, torch.from_numpy(ptok[sel]).to(dev),
                          torch.from_numpy(pexp[sel]).to(dev), torch.from_numpy(sel).to(dev), y,
                          L.FWD_FORCE_PREFILL, shared=shared)

    y = torch.full((rows, H), float("nan"), dtype=torch.bfloat16, device=dev)
    run(np.arange(rows))
    torch.cuda.synchronize()
    whole = bits(y)
    y = torch.full((rows, H), float("nan"), dtype=torch.bfloat16, device=dev)
    for r in range(int(rank.max()) // SPLIT + 1):
        run(np.flatnonzero(rank // SPLIT == r))
    torch.cuda.synchronize()
    split = bits(y)
    return whole, split, int(np.bincount(pexp, minlength=E + 1).max())


@pytest.mark.parametrize("spec", [QWEN3_30B_A3B, QWEN3_30B_A3B_3BIT], ids=["4bit", "3bit"])
def test_full_chunk_rows_independent_of_tiles(gpu, spec):
    """The 2048-token Qwen3-shape chunk with the Zipf(1.1) router: its hot experts hold
    hundreds to ~2000 pairs each, most of its rows in full 128-row tiles."""
    import torch

    from bigrig_amd import synth
    from tests.test_gpu_full_size import _layer
    T = 2048
    print(f"[tiles] full chunk {spec.quant.bits}-bit T={T}", flush=True)
    pool, experts, wr, bias, _, _ = _layer(spec, seed=900 + spec.quant.bits)
    if bias is None:   # the Zipf(1.1) router bias of the Qwen3-shape configurations
        bias = synth.zipf_bias_torch(spec.n_experts, 1.1, seed=902)
    x = synth.activations(T, spec.hidden, seed=901)
    k = spec.top_k
    idx = torch.empty((T, k), dtype=torch.int32, device=gpu)
    w = torch.empty((T, k), dtype=torch.float32, device=gpu)
    out = ops.moe_block(spec, pool, x, wr, bias, out_idx=idx, out_w=w, flags=L.FWD_FORCE_PREFILL)
    whole, split, most = _whole_vs_split(spec, pool, x, idx)
    print(f"[tiles] busiest expert {most} pairs", flush=True)
    assert most > 256, "the chunk has no expert with several full tiles"
    assert np.array_equal(whole, split), \
        f"{int((whole != split).any(-1).sum())} rows differ between the tile kernels"
    # the block's output on every tile edge against the oracle
    idx_h, w_h = idx.cpu().numpy(), w.cpu().numpy()
    toks = tile_edge_tokens(idx_h, spec.n_experts)
    need = sorted(set(int(e) for e in idx_h[toks].reshape(-1)))
    host = {e: experts[e].cpu().numpy().tobytes() for e in need}
    elist = [host.get(e, host[need[0]]) for e in range(spec.n_experts)]
    ref, _ = oracle.moe_forward(spec, elist, bits(x)[toks], idx_h[toks], w_h[toks])
    got = F.bf16_bits_to_f32(bits(out)[toks])
    want = F.bf16_bits_to_f32(ref)
    rt = per_token_rel_l2(got, want)
    print(f"[tiles] {len(toks)} tokens: rel L2 {oracle.rel_l2(got, want):.2e}, worst {rt.max():.2e}",
          flush=True)
    assert oracle.rel_l2(got, want) < TOL and rt.max() < TOL
    pool.close()
    del experts
    torch.cuda.empty_cache()


@pytest.mark.parametrize("spec", [
    small(QWEN3_30B_A3B, hidden=512, inter=256, n_experts=8, top_k=2, act="silu_mlp"),
    small(QWEN3_30B_A3B, hidden=512, inter=512, n_experts=8, top_k=2,
          quant=F.QuantSpec(4, 32, "mxfp4"), has_bias=True, act="swiglu_clamped",
          route="topk_softmax"),
    small(E256_SHARED, hidden=512, inter=256, n_experts=16, top_k=4, shared_inter=256),
    small(QWEN3_30B_A3B, hidden=512, inter=256, n_experts=8, top_k=2,
          quant=F.QuantSpec(4, 64, "affine", "float16")),
    # scale rows of 18 and 10 bytes: 2-byte scale copies, which 32- and 64-row tiles read from
    # a per-tile table and 128-row tiles copy stage by stage
    small(QWEN3_30B_A3B, hidden=576, inter=320, n_experts=8, top_k=2,
          quant=F.QuantSpec(4, 32, "mxfp4"), has_bias=True, act="swiglu_clamped",
          route="topk_softmax"),
    small(QWEN3_30B_A3B, hidden=512, inter=384, n_experts=8, top_k=2,
          quant=F.QuantSpec(2, 128, "affine")),
], ids=["silu-mlp", "mxfp4-clamped", "shared", "fp16-scales", "mxfp4-unpaired", "2bit-g128"])
def test_small_layer_rows_independent_of_tiles(gpu, spec):
    """Small layers with a strongly biased router, so one expert takes several full tiles (a
    partial last one too): two-layer experts, MXFP4 with biases and the clamped SwiGLU, a shared
    expert (every token's shared pair), fp16 scales, and layouts whose scales are copied 2 bytes
    a stage (MXFP4 with 18-byte scale rows, 2-bit groups of 128)."""
    import torch
    T = 700
    lay = make_layer(spec, seed=77, zipf=4.0)
    moe, sw, pool, _ = build_gpu_layer(lay, gpu)
    # the pair lists read the pool's device table directly: upload it (the layer's own forward
    # does this on its first call)
    pool.g2s_device(torch.cuda.current_stream().cuda_stream)
    pool.device.sync()
    x = make_x(T, spec.hidden, seed=78)
    xd = to_dev_bits(x, gpu)
    print(f"[tiles] small {spec.act} {spec.quant.mode} T={T}", flush=True)
    _, idx, w, sg = oracle.router(x, lay.router, False, lay.bias, spec.top_k, spec.route_mode,
                                  lay.sgate_w)
    shared = None
    if spec.shared_inter:
        shared = torch.from_numpy(np.frombuffer(lay.shared, np.uint8).copy()).to(gpu)
    whole, split, most = _whole_vs_split(spec, pool, xd, idx, shared)
    assert most > 256
    bad = np.flatnonzero(np.isnan(F.bf16_bits_to_f32(whole)).any(-1))
    pexp = np.concatenate([idx.reshape(-1), np.full(T if shared is not None else 0, spec.n_experts)])
    assert bad.size == 0, (f"{bad.size} rows with NaN, experts {np.unique(pexp[bad]).tolist()}, "
                           f"first rows {bad[:8].tolist()}, expert sizes "
                           f"{np.bincount(pexp, minlength=spec.n_experts + 1).tolist()}")
    assert np.array_equal(whole, split), \
        f"{int((whole != split).any(-1).sum())} rows differ between the tile kernels"
    ref, yref = oracle.moe_forward(spec, lay.experts, x, idx, w, lay.shared, sg, want_unreduced=True)
    nr = idx.size   # the routed rows (the shared expert's rows follow them)
    r = oracle.rel_l2(F.bf16_bits_to_f32(whole[:nr]), F.bf16_bits_to_f32(yref.reshape(nr, -1)))
    print(f"[tiles] unreduced rows rel L2 {r:.2e}", flush=True)
    assert r < TOL
    # the whole block (router, grouped GEMMs, combine, shared expert) against the oracle
    out = moe(xd)
    torch.cuda.synchronize()
    r2 = oracle.rel_l2(F.bf16_bits_to_f32(bits(out)), F.bf16_bits_to_f32(ref))
    assert r2 < TOL, f"block rel L2 {r2:.3e}"
    pool.close()


@pytest.mark.parametrize("spec", [
    small(QWEN3_30B_A3B, hidden=64, inter=64, n_experts=8, top_k=2),
    small(QWEN3_30B_A3B, hidden=192, inter=192, n_experts=8, top_k=2,
          quant=F.QuantSpec(4, 32, "mxfp4"), has_bias=True, act="swiglu_clamped", route="topk_softmax"),
    small(QWEN3_30B_A3B, hidden=128, inter=320, n_experts=8, top_k=2, quant=F.QuantSpec(3, 64, "affine")),
    small(QWEN3_30B_A3B, hidden=128, inter=64, n_experts=8, top_k=2, quant=F.QuantSpec(8, 64, "affine")),
    small(QWEN3_30B_A3B, hidden=192, inter=64, n_experts=8, top_k=2, quant=F.QuantSpec(16, 0, "none")),
], ids=["4bit-K64", "mxfp4-K192", "3bit-K128-I320", "8bit-K64", "bf16-K192"])
def test_narrow_widths_rows_independent_of_tiles(gpu, spec):
    """Contractions of one, two and three 64-wide stages (a stage pair cut short by an odd
    count, a single stage) through every tile height, bit for bit between tile heights and
    within 1e-2 of the oracle."""
    T = 600
    lay = make_layer(spec, seed=91, zipf=4.0)
    _, _, pool, _ = build_gpu_layer(lay, gpu)
    import torch
    pool.g2s_device(torch.cuda.current_stream().cuda_stream)
    pool.device.sync()
    x = make_x(T, spec.hidden, seed=92)
    xd = to_dev_bits(x, gpu)
    print(f"[tiles] narrow H={spec.hidden} I={spec.inter} {spec.quant.mode} {spec.quant.bits}-bit", flush=True)
    _, idx, w, _ = oracle.router(x, lay.router, False, lay.bias, spec.top_k, spec.route_mode)
    whole, split, most = _whole_vs_split(spec, pool, xd, idx)
    assert most > 128
    assert np.array_equal(whole, split), \
        f"{int((whole != split).any(-1).sum())} rows differ between the tile kernels"
    _, yref = oracle.moe_forward(spec, lay.experts, x, idx, w, want_unreduced=True)
    nr = idx.size
    r = oracle.rel_l2(F.bf16_bits_to_f32(whole[:nr]), F.bf16_bits_to_f32(yref.reshape(nr, -1)))
    assert r < TOL, f"unreduced rows rel L2 {r:.3e}"
    pool.close()
