"""The whole-layer residency plan (autoconfig.py:52-109), on the CPU: the reference's recorded
configuration, the refusals, and a brute-force search for the same optimum on small grids."""
import itertools

from bigrig_amd.hostserve import plan_full_layers


def test_reference_configuration():
    # "uniform 36 slots" vs "10 whole + 11 elsewhere" on 48 layers of 128 experts, top-8
    # (autoconfig.py:69-72)
    assert plan_full_layers(48, 128, 8, 36) == (10, 11)
    whole, rest = plan_full_layers(48, 128, 8, 36)
    assert whole * 128 + rest * (48 - whole) <= 36 * 48


def test_refusals():
    assert plan_full_layers(48, 128, 8, 128) == (0, 128)     # already whole
    assert plan_full_layers(48, 128, 8, 200) == (0, 200)
    assert plan_full_layers(1, 128, 8, 36) == (0, 36)        # nothing to redistribute
    assert plan_full_layers(48, 9, 8, 4) == (0, 4)            # floor 9 >= 9 experts
    assert plan_full_layers(48, 128, 8, 8) == (0, 8)          # below the floor everywhere
    assert plan_full_layers(48, 128, 8, 10) == (0, 10)        # floor fits, no whole layer does
    assert plan_full_layers(4, 16, 2, 8, floor_over_topk=0)[1] >= 2


def _search(L, E, k, cap, over=1):
    floor = max(1, k + over)
    budget = cap * L
    if cap >= E or L < 2 or floor >= E or budget < floor * L:
        return 0, cap
    for whole in range(L - 1, 0, -1):
        best = None
        for rest in range(floor, E + 1):
            if whole * E + rest * (L - whole) <= budget:
                best = rest
        if best is not None:
            return whole, best
    return 0, cap


def test_matches_brute_force():
    for L, E, k, cap in itertools.product(range(1, 7), range(2, 13), range(1, 4), range(1, 14)):
        assert plan_full_layers(L, E, k, cap) == _search(L, E, k, cap), (L, E, k, cap)


def _spend(whole, rest, n_layers, n_experts):
    return n_experts * whole + rest * (n_layers - whole)


def test_sweep_never_overspends_or_starves():
    """The properties the reference's planner tests hold it to (tests/test_fulllayers.py:33-131):
    no plan spends more slots than the uniform one, none leaves a layer at or below top-k, none
    holds every layer whole, more memory never means fewer whole layers, re-planning from the
    streamed capacity does not ratchet up."""
    for n_layers in (2, 4, 12, 24, 48, 64):
        for n_experts in (8, 16, 60, 64, 128, 256):
            for top_k in (1, 2, 4, 8, 16):
                if top_k >= n_experts:
                    continue
                prev = -1
                for cap in range(top_k, n_experts + 1):
                    whole, rest = plan_full_layers(n_layers, n_experts, top_k, cap)
                    assert _spend(whole, rest, n_layers, n_experts) <= cap * n_layers
                    assert whole < n_layers
                    if whole:
                        assert top_k < rest <= n_experts
                        w2, _ = plan_full_layers(n_layers, n_experts, top_k, rest)
                        assert w2 <= whole
                    if cap < n_experts:
                        assert whole >= prev, (n_layers, n_experts, top_k, cap)
                        prev = whole


def test_nonsense_in_a_safe_plan_out():
    for args in ((0, 128, 8, 36), (48, 0, 8, 36), (48, 128, 0, 36), (48, 128, 8, 0),
                 (-4, 128, 8, 36), (48, 128, 200, 36), (48, 8, 8, 8)):
        whole, rest = plan_full_layers(*args)
        assert whole >= 0 and rest >= 0 and whole < max(1, args[0]), (args, whole, rest)
