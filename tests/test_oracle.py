"""Pins for the oracle (CPU): the C restatement and the float64 truth.

Each function of the oracle is checked against something it does not itself compute: closed
forms, hand-derived known answers that a different summation order would get wrong, a torch
float32/float64 SwiGLU MLP, brute force on tiny shapes, and the reference's own legality and
permutation oracles for the expert-sorted spans (tests/test_pairsort.py:28-102). Several tests
plant a plausible mistake in the oracle's inputs or arithmetic and check that the same
tolerance catches it.
"""
import numpy as np
import pytest

import oracle
from bigrig_amd import formats as F
from bigrig_amd.layer import StreamingSwitchGLU
from bigrig_amd.spec import E256_SHARED, GPT_OSS_120B, OLMOE_1B_7B, QWEN3_30B_A3B
from tests.helpers import make_layer, make_x, small

BF16_ONE = 0x3F80


@pytest.fixture(scope="module", autouse=True)
def _built():
    oracle.build(force=False)


# ------------------------------------------------------------------ router dot order
def test_lane_tree_one_hot_is_exact():
    rng = np.random.default_rng(0)
    H = 2048
    w = rng.standard_normal(H).astype(np.float32)
    for h in (0, 7, 8, 511, 512, 1024 + 3, H - 1):
        x = np.zeros(H, np.uint16)
        x[h] = F.f32_to_bf16_bits(np.array([-1.5], np.float32))[0]
        assert oracle.dot_lane_tree(x, w, True) == np.float32(-1.5) * w[h]


def test_lane_tree_small_integers_are_exact():
    rng = np.random.default_rng(1)
    for H in (64, 512, 2048, 2880):
        xi = rng.integers(-8, 9, H)
        wi = rng.integers(-8, 9, H)
        x = F.f32_to_bf16_bits(xi.astype(np.float32))
        got = oracle.dot_lane_tree(x, wi.astype(np.float32), True)
        assert got == float(np.dot(xi, wi))
        got_bf = oracle.dot_lane_tree(x, F.f32_to_bf16_bits(wi.astype(np.float32)), False)
        assert got_bf == float(np.dot(xi, wi))


def test_lane_tree_order_known_answers():
    """Summation-order KATs. Lane l sums 8-element chunks l, l+64, ... with fmaf; the 64 lane
    sums then combine pairwise at strides 32, 16, ..., 1. Element order would give 1 here."""
    H = 1024
    x = np.full(H, BF16_ONE, np.uint16)
    # lane 0 holds 2^24 (chunk 0) then +1 (chunk 64): fp32 rounds 2^24+1 to even -> 2^24;
    # lane 1 holds -2^24 (chunk 1). Tree: 2^24 + -2^24 = 0.
    w = np.zeros(H, np.float32)
    w[0], w[8 * 64], w[8] = 2.0 ** 24, 1.0, -(2.0 ** 24)
    assert oracle.dot_lane_tree(x, w, True) == 0.0
    # lane 0: 2^24, lane 32: 1, lane 1: -2^24. Stride 32 first: 2^24 + 1 -> 2^24, then
    # stride 1 cancels it: 0. Stride 1 first would give (2^24 - 2^24) + 1 = 1.
    w = np.zeros(H, np.float32)
    w[0], w[8 * 32], w[8] = 2.0 ** 24, 1.0, -(2.0 ** 24)
    assert oracle.dot_lane_tree(x, w, True) == 0.0
    # and a sum whose order does not matter comes out exact
    w = np.zeros(H, np.float32)
    w[0], w[8 * 32], w[8] = 2.0 ** 20, 1.0, -(2.0 ** 20)
    assert oracle.dot_lane_tree(x, w, True) == 1.0


def test_lane_tree_error_bound_vs_f64():
    rng = np.random.default_rng(2)
    for H in (2048, 2880):
        x = make_x(4, H, seed=H)
        w = rng.standard_normal((4, H)).astype(np.float32) * 0.02
        for t in range(4):
            got = oracle.dot_lane_tree(x[t], w[t], True)
            xf = F.bf16_bits_to_f32(x[t]).astype(np.float64)
            exact = float(xf @ w[t].astype(np.float64))
            bound = (H // 64 * 8 + 6) * 2.0 ** -24 * float(np.abs(xf) @ np.abs(w[t]))
            assert abs(got - exact) <= bound


# ------------------------------------------------------------------ router
ROUTE_SPECS = [OLMOE_1B_7B, QWEN3_30B_A3B, E256_SHARED, GPT_OSS_120B]


@pytest.mark.parametrize("spec", ROUTE_SPECS, ids=lambda s: f"E{s.n_experts}k{s.top_k}m{s.route_mode}")
def test_router_matches_f64_away_from_ties(spec):
    lay = make_layer(small(spec, inter=64), seed=3, bank=2, zipf=1.1)
    x = make_x(32, spec.hidden, seed=4)
    w_f32 = spec.router_dtype == "float32"
    lg, idx, wts, _ = oracle.router(x, lay.router, w_f32, lay.bias, spec.top_k, spec.route_mode)
    lg64, idx64, w64 = oracle.router_f64(x, lay.router, w_f32, lay.bias, spec.top_k,
                                        spec.route_mode)
    assert np.abs(lg - lg64).max() < 1e-5
    # rows whose (k)th and (k+1)th logits are clearly apart must pick the same set in order
    srt = -np.sort(-lg64, axis=-1)
    clear = np.min(np.diff(-srt[:, :spec.top_k + 1], axis=-1), axis=-1) > 1e-4
    assert clear.sum() >= 16
    assert np.array_equal(idx[clear], idx64[clear])
    assert np.allclose(wts[clear], w64[clear], rtol=2e-6, atol=1e-7)
    # every row: k distinct ids in range, sorted by logit (test_frontier.py:42-45)
    assert all(len(set(r)) == spec.top_k for r in idx)
    assert idx.min() >= 0 and idx.max() < spec.n_experts
    sel = np.take_along_axis(lg, idx, -1)
    assert (np.diff(sel, axis=-1) <= 0).all()


def test_router_weight_rules():
    spec = small(QWEN3_30B_A3B, n_experts=16, top_k=4, hidden=128)
    rng = np.random.default_rng(5)
    wr = rng.standard_normal((16, 128)).astype(np.float32) * 0.3
    x = make_x(8, 128, seed=6)
    lg, idx0, w0, _ = oracle.router(x, wr, True, None, 4, 0)
    _, idx1, w1, _ = oracle.router(x, wr, True, None, 4, 1)
    _, idx2, w2, _ = oracle.router(x, wr, True, None, 4, 2)
    assert np.array_equal(idx0, idx1) and np.array_equal(idx0, idx2)
    # softmax over all E: the k weights sum to less than one, and equal softmax(lg)[idx]
    p = np.exp(lg.astype(np.float64) - lg.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    assert np.allclose(w0, np.take_along_axis(p, idx0, -1), rtol=1e-6)
    assert (w0.sum(-1) < 1).all()
    # renorm and top-k-then-softmax both sum to one and agree (the gpt-oss rule equals renorm)
    assert np.allclose(w1.sum(-1), 1, atol=1e-6) and np.allclose(w2.sum(-1), 1, atol=1e-6)
    assert np.allclose(w1, w2, rtol=1e-6)
    # k == E softmax-topk is a plain softmax
    _, idxE, wE, _ = oracle.router(x, wr, True, None, 16, 0)
    assert np.allclose(np.take_along_axis(p, idxE, -1), wE, rtol=1e-6)


def test_router_ties_go_to_the_lower_id():
    rng = np.random.default_rng(7)
    wr = rng.standard_normal((16, 256)).astype(np.float32) * 0.01
    x = make_x(3, 256, seed=8)
    xs = F.bf16_bits_to_f32(x)
    # experts 3 and 11 share one row that wins by a wide margin for every token: identical
    # logits, both chosen, 3 first; a third copy at 12 is chosen only when k >= 3
    top = np.sign(xs.sum(0)).astype(np.float32)
    for e in (3, 11, 12):
        wr[e] = top
    _, idx, _, _ = oracle.router(x, wr, True, None, 2, 1)
    assert (idx == [3, 11]).all()
    _, idx, _, _ = oracle.router(x, wr, True, None, 3, 1)
    assert (idx == [3, 11, 12]).all()


def test_router_shared_gate_and_errors():
    rng = np.random.default_rng(9)
    H = 256
    wr = F.f32_to_bf16_bits(rng.standard_normal((8, H)).astype(np.float32) * 0.02)
    sgw = F.f32_to_bf16_bits(rng.standard_normal(H).astype(np.float32) * 0.05)
    x = make_x(5, H, seed=10)
    _, _, _, sg = oracle.router(x, wr, False, None, 2, 1, shared_gate_w=sgw)
    d = F.bf16_bits_to_f32(x).astype(np.float64) @ F.bf16_bits_to_f32(sgw).astype(np.float64)
    assert np.allclose(sg, 1 / (1 + np.exp(-d)), rtol=1e-6)
    with pytest.raises(ValueError):
        oracle.router(x, wr, False, None, 9, 1)          # k > E
    with pytest.raises(ValueError):
        oracle.router(x[:, :250], wr[:, :250], False, None, 2, 1)   # H not a multiple of 8


# ------------------------------------------------------------------ sigmoid / group-limited
def test_exp_rt_is_within_two_ulp():
    """The routing exponential against float64 exp over its whole normal range and the
    reduction's edges (n ln2 +- ln2/2), where a wrong split constant or a dropped Taylor term
    shows first."""
    xs = np.concatenate([np.linspace(-87.0, 88.0, 20001, dtype=np.float32),
                         (np.arange(-120, 121) * np.log(2) / 2).astype(np.float32),
                         np.float32([0.0, -0.0, 1e-8, -1e-8, 0.5, -0.5])])
    xs = xs[(xs > -87.0) & (xs < 88.5)]
    got = oracle.exp_rt(xs).astype(np.float64)
    want = np.exp(xs.astype(np.float64))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    assert (np.abs(got - want) <= 2 * ulp).all(), np.max(np.abs(got - want) / ulp)
    assert oracle.exp_rt(np.float32([0.0]))[0] == 1.0
    assert np.isinf(oracle.exp_rt(np.float32([100.0]))[0])
    assert oracle.exp_rt(np.float32([-200.0]))[0] == 0.0


def _onehot_router(logits):
    """(x bits [1, 8], fp32 router [E, 8]) whose logits are exactly `logits`: x = e_0."""
    E = len(logits)
    w = np.zeros((E, 8), np.float32)
    w[:, 0] = logits
    x = np.zeros((1, 8), np.uint16)
    x[0, 0] = 0x3F80                      # bf16 1.0
    return x, w


def test_group_limited_kats():
    """Hand-built logits where each rule's choice is known. Two groups of four experts, one
    group kept, top-2:
      - sigmoid: group 0 = [3, -3, -3, -3], group 1 = [2, 2, -3, -3]. Top-2 sums pick group 1
        (0.881 + 0.881 > 0.953 + 0.047), where scoring by the maximum would pick group 0; the
        tied pair goes lower id first; the weights are the plain sigmoids.
      - a selection bias of +1 on expert 1 moves the choice to group 0 ([1, 0]) while the
        weights stay sigmoid(logit): the bias selects, it does not weigh.
      - softmax groups score by their maximum logit: group 0, experts [0, 1]."""
    lg = np.float32([3, -3, -3, -3, 2, 2, -3, -3])
    x, w = _onehot_router(lg)
    sig = lambda v: 1.0 / (1.0 + np.exp(-np.float64(v)))
    _, idx, wt, _ = oracle.router(x, w, True, None, 2, 3, n_group=2, topk_group=1)
    assert idx.tolist() == [[4, 5]]
    np.testing.assert_allclose(wt[0], [sig(2), sig(2)], rtol=1e-6)
    bias = np.zeros(8, np.float32)
    bias[1] = 1.0
    lgo, idx, wt, _ = oracle.router(x, w, True, bias, 2, 3, n_group=2, topk_group=1)
    assert idx.tolist() == [[1, 0]] and (lgo == lg).all()     # logits stay raw
    np.testing.assert_allclose(wt[0], [sig(-3), sig(3)], rtol=1e-6)
    _, idx, wt, _ = oracle.router(x, w, True, None, 2, 0, n_group=2, topk_group=1)
    assert idx.tolist() == [[0, 1]]
    p = np.exp(lg - lg.max()) / np.exp(lg - lg.max()).sum()
    np.testing.assert_allclose(wt[0], p[[0, 1]], rtol=1e-6)
    # renormalised sigmoid weights sum to one, then carry the scale
    _, _, wt, _ = oracle.router(x, w, True, None, 2, 4, n_group=2, topk_group=1, scale=2.5)
    np.testing.assert_allclose(wt.sum(), 2.5, rtol=1e-6)


GROUP_RULES = [  # (E, k, mode, n_group, topk_group, scale, bias)
    (256, 8, 4, 8, 4, 2.5, True),        # DeepSeek-V3 shape
    (256, 8, 3, 8, 4, 1.0, False),
    (64, 6, 0, 8, 3, 16.0, False),       # DeepSeek-V2-style softmax groups
    (128, 8, 4, 0, 0, 1.0, True),        # sigmoid, no groups
    (64, 4, 1, 4, 2, 1.0, False),
]


@pytest.mark.parametrize("rule", GROUP_RULES, ids=lambda r: f"E{r[0]}k{r[1]}m{r[2]}g{r[3]}/{r[4]}")
def test_group_rules_match_f64(rule):
    """The C rule against the float64 closed form (sorting, group top-2 from sorted groups),
    rows in order with weights to 2e-6."""
    E, k, mode, ng, tg, scale, with_bias = rule
    rng = np.random.default_rng(E + 7 * k + mode)
    H = 256
    wr = rng.standard_normal((E, H)).astype(np.float32) * 0.05
    bias = (rng.standard_normal(E).astype(np.float32) * 0.05) if with_bias else None
    x = make_x(48, H, seed=E + mode)
    _, idx, wt, _ = oracle.router(x, wr, True, bias, k, mode, n_group=ng, topk_group=tg,
                                  scale=scale)
    _, idx64, w64 = oracle.router_f64(x, wr, True, bias, k, mode, n_group=ng, topk_group=tg,
                                      scale=scale)
    assert np.array_equal(idx, idx64)
    np.testing.assert_allclose(wt, w64, rtol=2e-6, atol=1e-7)
    if ng > 1:    # every pick lies in at most topk_group groups
        assert max(len(set((r // (E // ng)).tolist())) for r in idx) <= tg


def test_group_rule_reductions():
    """Special cases that reduce to the plain rules: keeping every group is no limit; sigmoid
    without bias picks the softmax top-k (both monotonic in the logit); the scale multiplies the
    weights exactly."""
    rng = np.random.default_rng(21)
    E, H, k = 64, 128, 6
    wr = rng.standard_normal((E, H)).astype(np.float32) * 0.05
    x = make_x(16, H, seed=22)
    for mode in (0, 1, 3, 4):
        base = oracle.router(x, wr, True, None, k, mode)
        allg = oracle.router(x, wr, True, None, k, mode, n_group=8, topk_group=8)
        assert np.array_equal(base[1], allg[1]) and np.array_equal(base[2], allg[2])
    _, i_soft, _, _ = oracle.router(x, wr, True, None, k, 0)
    lg, i_sig, w_sig, _ = oracle.router(x, wr, True, None, k, 3)
    assert np.array_equal(i_soft, i_sig)
    np.testing.assert_allclose(w_sig, 1 / (1 + np.exp(-np.take_along_axis(lg, i_sig, -1)
                                                     .astype(np.float64))), rtol=1e-6)
    _, _, w1, _ = oracle.router(x, wr, True, None, k, 4, n_group=8, topk_group=2)
    _, _, w3, _ = oracle.router(x, wr, True, None, k, 4, n_group=8, topk_group=2, scale=3.0)
    assert np.array_equal(w3, w1 * np.float32(3.0))
    with pytest.raises(ValueError):
        oracle.router(x, wr, True, None, k, 4, n_group=8, topk_group=0)
    with pytest.raises(ValueError):
        oracle.router(x, wr, True, None, 20, 4, n_group=8, topk_group=2)   # k > 2 groups of 8


# ------------------------------------------------------------------ dequant
@pytest.mark.parametrize("q", [F.QuantSpec(4, 64, "affine", "bfloat16"),
                               F.QuantSpec(4, 64, "affine", "float16"),
                               F.QuantSpec(4, 32, "mxfp4"),
                               F.QuantSpec(3, 64, "affine", "bfloat16"),
                               F.QuantSpec(2, 128, "affine", "bfloat16"),
                               F.QuantSpec(6, 64, "affine", "float16"),
                               F.QuantSpec(8, 64, "affine", "bfloat16"),
                               F.QuantSpec(16, 0, "none")],
                         ids=["bf16", "f16", "mxfp4", "3bit", "2bit-g128", "6bit-f16", "8bit", "unquantized"])
def test_c_dequant_equals_numpy_bitwise(q):
    """The C dequant and formats.dequantize_projection (pinned by closed form in test_formats)
    agree bit for bit, projection by projection."""
    base = GPT_OSS_120B if q.mode == "mxfp4" else QWEN3_30B_A3B
    spec = small(base, hidden=256, inter=128, quant=q)
    rng = np.random.default_rng(11)
    blob = F.make_expert(rng, 256, 128, q, has_bias=spec.has_bias)
    arrs = F.split_expert(blob, spec.expert_spec())
    for p, name in enumerate(F.PROJECTIONS):
        want = F.dequantize_projection(arrs, name, q)
        got = oracle.dequant(spec, blob, p)
        assert got.shape == want.shape
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ------------------------------------------------------------------ layer
LAYER_SPECS = {
    "olmoe": small(OLMOE_1B_7B, hidden=256, inter=128, n_experts=16, top_k=4),
    "qwen3": small(QWEN3_30B_A3B, hidden=256, inter=128, n_experts=16, top_k=4),
    "shared": small(E256_SHARED, hidden=256, inter=64, n_experts=16, top_k=4, shared_inter=64),
    "gptoss": small(GPT_OSS_120B, hidden=256, inter=128, n_experts=16, top_k=4),
    "mlp": small(QWEN3_30B_A3B, hidden=256, inter=128, n_experts=16, top_k=4, act="silu_mlp"),
    "3bit": small(QWEN3_30B_A3B, hidden=256, inter=128, n_experts=16, top_k=4,
                  quant=F.QuantSpec(3, 64, "affine", "bfloat16")),
    "unquantized": small(E256_SHARED, hidden=256, inter=128, n_experts=16, top_k=4, shared_inter=128,
                         quant=F.QuantSpec(16, 0, "none")),
}


def _route(lay, x):
    s = lay.spec
    _, idx, w, sg = oracle.router(x, lay.router, s.router_dtype == "float32", lay.bias, s.top_k,
                                  s.route_mode, shared_gate_w=lay.sgate_w)
    return idx, w, sg


@pytest.mark.parametrize("name", list(LAYER_SPECS))
def test_layer_vs_f64_truth(name):
    spec = LAYER_SPECS[name]
    lay = make_layer(spec, seed=12)
    x = make_x(6, spec.hidden, seed=13)
    idx, w, sg = _route(lay, x)
    out, yun = oracle.moe_forward(spec, lay.experts, x, idx, w, lay.shared, sg,
                                  want_unreduced=True)
    ref, yref = oracle.moe_forward_f64(spec, lay.experts, x, idx, w, lay.shared, sg)
    assert oracle.rel_l2(F.bf16_bits_to_f32(out), ref) < 4e-3
    assert oracle.rel_l2(F.bf16_bits_to_f32(yun), yref) < 4e-3
    # the combine: out = bf16(sum_j w_j * y_j (+ g * shared)) over the bf16 rows
    yr = F.bf16_bits_to_f32(yun).astype(np.float64)
    comb = np.einsum("tk,tkh->th", w.astype(np.float64), yr)
    if lay.shared is not None:
        # the shared expert's rows, computed as a routed expert (shared_inter == inter here)
        _, ysh = oracle.moe_forward(spec, [lay.shared] * spec.n_experts, x,
                                    np.zeros_like(idx), np.ones_like(w), want_unreduced=True)
        comb += sg[:, None].astype(np.float64) * F.bf16_bits_to_f32(ysh[:, 0]).astype(np.float64)
    got = F.bf16_bits_to_f32(out).astype(np.float64)
    # bf16 rounding of the sum, plus the fp32 summation error of its terms (a sum that cancels
    # keeps the absolute error of its largest terms)
    mag = np.einsum("tk,tkh->th", np.abs(w.astype(np.float64)), np.abs(yr))
    if lay.shared is not None:
        mag += np.abs(comb)
    assert np.all(np.abs(got - comb) <= 2.0 ** -8 * np.abs(comb) + 16 * 2.0 ** -24 * mag)


def test_layer_threads_do_not_change_bits():
    spec = LAYER_SPECS["qwen3"]
    lay = make_layer(spec, seed=14)
    x = make_x(5, spec.hidden, seed=15)
    idx, w, _ = _route(lay, x)
    a, _ = oracle.moe_forward(spec, lay.experts, x, idx, w, nthreads=1)
    b, _ = oracle.moe_forward(spec, lay.experts, x, idx, w, nthreads=4)
    assert np.array_equal(a, b)


def test_single_expert_is_a_swiglu_mlp_torch():
    """k=1 with weight 1 reduces to a plain SwiGLU MLP; torch fp32 on the dequantized matrices."""
    import torch
    spec = small(QWEN3_30B_A3B, hidden=256, inter=128, n_experts=4, top_k=1)
    lay = make_layer(spec, seed=16)
    x = make_x(7, spec.hidden, seed=17)
    e = 2
    out, _ = oracle.moe_forward(spec, lay.experts, x, np.full((7, 1), e), np.ones((7, 1)))
    arrs = F.split_expert(lay.experts[e], spec.expert_spec())
    Wg, Wu, Wd = (torch.from_numpy(F.dequantize_projection(arrs, p, spec.quant))
                  for p in F.PROJECTIONS)
    xt = torch.from_numpy(F.bf16_bits_to_f32(x))
    h = (torch.nn.functional.silu(xt @ Wg.T) * (xt @ Wu.T)).to(torch.bfloat16).float()
    ref = (h @ Wd.T).numpy()
    got = F.bf16_bits_to_f32(out)
    assert oracle.rel_l2(got, ref) < 5e-3
    # planted mistakes: gate and up swapped, or scales and biases read from each other's
    # arrays -- the same tolerance rejects both
    bad = ((torch.nn.functional.silu(xt @ Wu.T) * (xt @ Wg.T)).to(torch.bfloat16).float()
           @ Wd.T).numpy()
    assert oracle.rel_l2(got, bad) > 5e-2
    sw = dict(arrs)
    for p in F.PROJECTIONS:
        sw[(p, "scales")], sw[(p, "biases")] = arrs[(p, "biases")], arrs[(p, "scales")]
    Bg, Bu, Bd = (torch.from_numpy(F.dequantize_projection(sw, p, spec.quant))
                  for p in F.PROJECTIONS)
    bad2 = ((torch.nn.functional.silu(xt @ Bg.T) * (xt @ Bu.T)).to(torch.bfloat16).float()
            @ Bd.T).numpy()
    assert oracle.rel_l2(got, bad2) > 5e-2


def test_unquantized_single_expert_is_a_swiglu_mlp_torch():
    """Unquantized (bf16) experts, k=1 with weight 1: the plain SwiGLU MLP on the bf16 weights
    themselves (the mx.gather_mm branch, stream.py:1626-1628), torch fp32; the weights are the
    packed bytes read as bf16 (a planted byte swap of each weight fails the same tolerance)."""
    import torch
    q = F.QuantSpec(16, 0, "none")
    spec = small(QWEN3_30B_A3B, hidden=256, inter=128, n_experts=4, top_k=1, quant=q)
    lay = make_layer(spec, seed=36)
    assert len(lay.experts[0]) == 3 * 256 * 128 * 2
    x = make_x(7, spec.hidden, seed=37)
    e = 3
    out, _ = oracle.moe_forward(spec, lay.experts, x, np.full((7, 1), e), np.ones((7, 1)))
    raw = np.frombuffer(lay.experts[e], np.uint16)
    Wg, Wu, Wd = (torch.from_numpy(F.bf16_bits_to_f32(raw[i * 256 * 128:(i + 1) * 256 * 128])
                                   .reshape(s)) for i, s in enumerate([(128, 256), (128, 256), (256, 128)]))
    xt = torch.from_numpy(F.bf16_bits_to_f32(x))
    h = (torch.nn.functional.silu(xt @ Wg.T) * (xt @ Wu.T)).to(torch.bfloat16).float()
    got = F.bf16_bits_to_f32(out)
    assert oracle.rel_l2(got, (h @ Wd.T).numpy()) < 5e-3
    swapped = [torch.from_numpy(F.bf16_bits_to_f32(F.f32_to_bf16_bits(W.numpy()).byteswap()))
               for W in (Wg, Wu, Wd)]
    bad = ((torch.nn.functional.silu(xt @ swapped[0].T) * (xt @ swapped[1].T)).to(torch.bfloat16).float()
           @ swapped[2].T).numpy()
    assert not np.isfinite(bad).all() or oracle.rel_l2(got, bad) > 5e-2


def test_single_two_layer_expert_is_a_silu_mlp_torch():
    """act silu_mlp with k=1, weight 1 is the plain MLP fc2(silu(fc1 x)) (stream.py:1167-1169):
    torch fp32 on the dequantized fc1 / fc2, h rounded to bf16 as the layer stores it. Planted
    mistakes -- the activation after fc2 instead of between, or fc1 used as a gated pair -- fail
    the same tolerance."""
    import torch
    spec = small(QWEN3_30B_A3B, hidden=256, inter=128, n_experts=4, top_k=1, act="silu_mlp")
    lay = make_layer(spec, seed=26)
    x = make_x(7, spec.hidden, seed=27)
    e = 1
    out, _ = oracle.moe_forward(spec, lay.experts, x, np.full((7, 1), e), np.ones((7, 1)))
    es = spec.expert_spec()
    assert list(es) == ["fc1", "fc2"] and len(lay.experts[e]) == F.spec_bytes(es)
    arrs = F.split_expert(lay.experts[e], es)
    W1, W2 = (torch.from_numpy(F.dequantize_projection(arrs, p, spec.quant)) for p in es)
    xt = torch.from_numpy(F.bf16_bits_to_f32(x))
    h = torch.nn.functional.silu(xt @ W1.T).to(torch.bfloat16).float()
    got = F.bf16_bits_to_f32(out)
    assert oracle.rel_l2(got, (h @ W2.T).numpy()) < 5e-3
    late = torch.nn.functional.silu((xt @ W1.T) @ W2.T).numpy()
    assert oracle.rel_l2(got, late) > 5e-2
    gated = ((torch.nn.functional.silu(xt @ W1.T) * (xt @ W1.T)) @ W2.T).numpy()
    assert oracle.rel_l2(got, gated) > 5e-2


def test_three_bit_layer_dequantizes_the_packed_codes():
    """3-bit affine: the oracle's dequant reads code k at bits [3k, 3k + 3) of the row, so a
    row whose codes are a known sequence dequantizes to s * q + b of exactly that sequence."""
    spec = small(QWEN3_30B_A3B, hidden=128, inter=64, n_experts=1, top_k=1,
                 quant=F.QuantSpec(3, 64, "affine", "bfloat16"))
    es = spec.expert_spec()
    arrs = F.split_expert(F.make_expert(np.random.default_rng(28), 128, 64, spec.quant), es)
    codes = (np.arange(64 * 128) * 5 + 3) % 8
    arrs[("gate_proj", "weight")] = F.pack_bits(codes.reshape(64, 128), 3)
    s = np.full(arrs[("gate_proj", "scales")].shape, 0x3F80, np.uint16)     # 1.0
    b = np.full(s.shape, 0xBF00, np.uint16)                                  # -0.5
    arrs[("gate_proj", "scales")], arrs[("gate_proj", "biases")] = s, b
    blob = F.join_expert(arrs, es)
    got = oracle.dequant(spec, blob, 0)
    assert np.array_equal(got, codes.reshape(64, 128).astype(np.float32) - 0.5)


def test_brute_force_tiny_layer_torch_f64():
    """E=4, H=I=64: every (token, expert) product by torch float64 against the f64 truth."""
    import torch
    spec = small(QWEN3_30B_A3B, hidden=64, inter=64, n_experts=4, top_k=2)
    lay = make_layer(spec, seed=18)
    x = make_x(3, 64, seed=19)
    idx, w, _ = _route(lay, x)
    ref, _ = oracle.moe_forward_f64(spec, lay.experts, x, idx, w)
    xt = torch.from_numpy(F.bf16_bits_to_f32(x)).double()
    want = torch.zeros((3, 64), dtype=torch.float64)
    for t in range(3):
        for j in range(2):
            arrs = F.split_expert(lay.experts[int(idx[t, j])], spec.expert_spec())
            Wg, Wu, Wd = (torch.from_numpy(F.dequantize_projection(arrs, p, spec.quant)).double()
                          for p in F.PROJECTIONS)
            g = Wg @ xt[t]
            h = g * torch.sigmoid(g) * (Wu @ xt[t])
            want[t] += float(w[t, j]) * (Wd @ h)
    assert np.allclose(ref, want.numpy(), rtol=1e-12, atol=1e-15)
    out, _ = oracle.moe_forward(spec, lay.experts, x, idx, w)
    assert oracle.rel_l2(F.bf16_bits_to_f32(out), want.numpy()) < 4e-3


def test_zero_expert_gives_exact_zero():
    for base in (QWEN3_30B_A3B, GPT_OSS_120B):
        spec = small(base, hidden=128, inter=64, n_experts=2, top_k=1, has_bias=False)
        blob = bytes(spec.bytes_per_expert)
        x = make_x(3, 128, seed=20)
        out, _ = oracle.moe_forward(spec, [blob, blob], x, np.zeros((3, 1)), np.ones((3, 1)))
        assert not np.any(out & 0x7FFF)


def test_zero_scale_makes_w_the_bias_closed_form():
    """s = 0: every weight of a group equals its bias, W = repeat(b, 64)."""
    spec = small(QWEN3_30B_A3B, hidden=128, inter=64, n_experts=1, top_k=1)
    rng = np.random.default_rng(21)
    arrs = F.split_expert(F.make_expert(rng, 128, 64, spec.quant), spec.expert_spec())
    for p in F.PROJECTIONS:
        arrs[(p, "scales")] = np.zeros_like(arrs[(p, "scales")])
        arrs[(p, "biases")] = F.f32_to_bf16_bits(
            rng.standard_normal(arrs[(p, "biases")].shape).astype(np.float32) * 0.05)
    blob = F.join_expert(arrs, spec.expert_spec())
    W = [np.repeat(F.bf16_bits_to_f32(arrs[(p, "biases")]).astype(np.float64), 64, axis=1)
         for p in F.PROJECTIONS]
    x = make_x(4, 128, seed=22)
    xf = F.bf16_bits_to_f32(x).astype(np.float64)
    g, u = xf @ W[0].T, xf @ W[1].T
    want = (g / (1 + np.exp(-g)) * u) @ W[2].T
    out, _ = oracle.moe_forward(spec, [blob], x, np.zeros((4, 1)), np.ones((4, 1)))
    assert oracle.rel_l2(F.bf16_bits_to_f32(out), want) < 4e-3


def test_clamped_swiglu_is_active_and_matched():
    """gpt-oss activation with pre-activations large enough that both clamps bind."""
    spec = LAYER_SPECS["gptoss"]
    assert (spec.act, spec.alpha, spec.limit) == ("swiglu_clamped", pytest.approx(1.702), 7.0)
    # closed form at a clamped point: g=10 -> 7, u=-9 -> -7
    a = oracle.act_f64(spec, np.array([10.0]), np.array([-9.0]))[0]
    assert a == pytest.approx(7.0 / (1 + np.exp(-1.702 * 7.0)) * (-6.0), rel=1e-12)
    lay = make_layer(spec, seed=23, expert_std=0.5)
    x = make_x(4, spec.hidden, seed=24)
    idx, w, _ = _route(lay, x)
    Wg, Wu, _, bg, bu, _ = oracle.expert_weights_f64(spec, lay.experts[int(idx[0, 0])])
    xf = F.bf16_bits_to_f32(x[0]).astype(np.float64)
    assert (Wg @ xf + bg).max() > 7 and np.abs(Wu @ xf + bu).max() > 7
    out, _ = oracle.moe_forward(spec, lay.experts, x, idx, w)
    ref, _ = oracle.moe_forward_f64(spec, lay.experts, x, idx, w)
    assert oracle.rel_l2(F.bf16_bits_to_f32(out), ref) < 4e-3
    # a planted mistake: the plain SwiGLU in place of the clamped one is rejected
    plain = small(spec, act="swiglu")
    bad, _ = oracle.moe_forward_f64(plain, lay.experts, x, idx, w)
    assert oracle.rel_l2(bad, ref) > 5e-2


# ------------------------------------------------------------------ bucketing
def test_sort_pairs_is_a_stable_argsort():
    rng = np.random.default_rng(25)
    for T, k, E in ((1, 8, 128), (69, 8, 128), (2048, 8, 128), (33, 4, 64), (5, 2, 8)):
        idx = rng.integers(0, E, (T, k)).astype(np.int32)
        order, offs = oracle.sort_pairs(idx, E)
        assert np.array_equal(order, np.argsort(idx.reshape(-1), kind="stable"))
        assert np.array_equal(offs, np.concatenate([[0], np.cumsum(np.bincount(idx.reshape(-1),
                                                                              minlength=E))]))
    with pytest.raises(ValueError):
        oracle.sort_pairs(np.array([[0, 8]]), 8)


CHUNK_CASES = ((69, 8, 128, 11), (69, 8, 128, 9), (400, 8, 128, 40), (7, 2, 16, 3),
               (1, 8, 128, 8), (69, 8, 128, 128))


@pytest.mark.parametrize("n_tok,k,E,C", CHUNK_CASES)
def test_pair_chunks_are_legal(n_tok, k, E, C):
    """tests/test_pairsort.py:28-49: spans hold at most C distinct experts, tile every pair
    exactly once, none empty, and an expert lives in exactly one span."""
    rng = np.random.default_rng(n_tok * 1000 + C)
    flat = rng.integers(0, E, size=(n_tok, k))
    spe = np.sort(flat.reshape(-1))
    spans = StreamingSwitchGLU._pair_chunks(spe, C)
    assert spans[0][0] == 0 and spans[-1][1] == spe.size
    assert all(hi > lo for lo, hi in spans)
    assert all(a[1] == b[0] for a, b in zip(spans, spans[1:]))
    assert all(len(np.unique(spe[lo:hi])) <= C for lo, hi in spans)
    owners = {}
    for i, (lo, hi) in enumerate(spans):
        for e in np.unique(spe[lo:hi]):
            assert owners.setdefault(int(e), i) == i


@pytest.mark.parametrize("n_tok,k,E,C", ((69, 8, 128, 11), (33, 4, 64, 5), (400, 8, 128, 40),
                                         (5, 2, 8, 3)))
def test_pair_unsort_puts_every_row_back(n_tok, k, E, C):
    """tests/test_pairsort.py:86-102: pair (t, r) computes t*1000 + expert; after the spans
    and the inverse permutation every value is back at (t, r)."""
    rng = np.random.default_rng(n_tok + C)
    flat = rng.integers(0, E, size=(n_tok, k))
    pe = flat.reshape(-1)
    order = np.argsort(pe, kind="stable")
    spe, tok = pe[order], order // k
    rows = np.full(pe.size, -1, np.int64)
    for lo, hi in StreamingSwitchGLU._pair_chunks(spe, C):
        rows[order[lo:hi]] = tok[lo:hi] * 1000 + spe[lo:hi]     # written straight to its row
    assert np.array_equal(rows.reshape(n_tok, k), np.arange(n_tok)[:, None] * 1000 + flat)
    # the planted mistake (no unsort) is caught
    flat_sorted = np.concatenate([tok[lo:hi] * 1000 + spe[lo:hi] for lo, hi in
                                  StreamingSwitchGLU._pair_chunks(spe, C)])
    assert not np.array_equal(flat_sorted.reshape(n_tok, k),
                              np.arange(n_tok)[:, None] * 1000 + flat)
