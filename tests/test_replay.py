"""Native trace replay (libbrx_replay.so) on the CPU: equal to the Python restatement to the
request on random sequences (LRU, LFUDA with its knobs, Belady), on the reference's known
answers (tests/test_pool.py:24-43 of the reference), and on the recorded miss-rate frontier of
the shipped Qwen3 routing trace; refusals of malformed input."""
import json
import os
import re

import numpy as np
import pytest

from bigrig_amd import policy as P
from bigrig_amd import replay as R

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _py(name, seq, C, E, ranks=None, **kw):
    if name == "belady":
        return P.belady(seq, C)["misses"]
    if name == "lru":
        return P.simulate(seq, C, E, P.LRU, ranks)["misses"]
    return P.simulate(seq, C, E, lambda c, e: P.LFUDA(c, e, **kw), ranks)["misses"]


def test_exports_every_declared_symbol():
    lib = R.load()
    decl = open(os.path.join(ROOT, "include", "brx_replay.h")).read()
    names = set(re.findall(r"\b(brx_\w+)\s*\(", decl))
    assert names >= {"brx_replay", "brx_replay_trace", "brx_lfuda_defaults", "brx_replay_last_error"}
    for n in names:
        assert hasattr(lib, n), n


def test_known_answers():
    seq = [1, 2, 3] * 3
    assert R.misses("lru", seq, 3, 8) == 3
    assert R.misses("lru", seq, 2, 8) == 9          # the classic LRU thrash
    assert R.misses("belady", seq, 2, 8) < 9
    assert R.misses("lru", seq, 8, 8) == 3
    assert R.misses("lfuda", [], 3, 8) == 0


@pytest.mark.parametrize("E,C", [(8, 1), (8, 3), (16, 5), (64, 16), (12, 12)])
def test_equal_to_python_on_random_sequences(E, C):
    rng = np.random.default_rng(E * 100 + C)
    for trial in range(4):
        n = int(rng.integers(1, 400))
        # skewed requests, so frequency matters
        seq = (rng.zipf(1.3, n) - 1) % E if trial % 2 else rng.integers(0, E, n)
        seq = [int(x) for x in seq]
        ranks = [int(x) for x in rng.integers(0, 8, n)]
        for name in ("lru", "lfuda", "belady"):
            assert R.misses(name, seq, C, E, ranks) == _py(name, seq, C, E, ranks), (name, trial)
        for kw in ({"rank_weight": 0.5}, {"fcap": None}, {"keep_ghost": False},
                   {"ghost_decay": 1.0}, {"fcap": 3.0, "ghost_decay": 0.25}):
            got = R.misses("lfuda", seq, C, E, ranks, lfuda=R.lfuda_params(**kw))
            assert got == _py("lfuda", seq, C, E, ranks, **kw), (kw, trial)


def test_belady_is_a_lower_bound():
    rng = np.random.default_rng(3)
    for _ in range(10):
        seq = rng.integers(0, 12, 300)
        C = int(rng.integers(2, 8))
        b = R.misses("belady", seq, C, 12)
        assert b <= R.misses("lru", seq, C, 12) and b <= R.misses("lfuda", seq, C, 12)


@pytest.mark.parametrize("frac", ["0.1", "0.25", "0.5"])
def test_trace_sweep_reproduces_recorded_frontier(frac):
    """data/results/frontier_locality_qwen3.json: LRU, LFUDA ('miss') and Belady over the first
    8 layers of the shipped Qwen3 trace, to the request, through the threaded sweep."""
    with open(os.path.join(GOLDEN, "frontier_locality_qwen3.json")) as f:
        cur = json.load(f)["curve"]
    idx = np.load(os.path.join(GOLDEN, "qwen3_full.npz"))["idx"].astype(np.int32)
    pt = cur["points"][frac]
    C, n_layers = pt["capacity"], cur["layers"]
    req = cur["tokens"] * cur["k"]
    sub = idx[:n_layers, :cur["tokens"], :cur["k"]]
    for name, key in (("lru", "lru"), ("lfuda", "miss"), ("belady", "belady")):
        m = R.trace_misses(name, sub, [C], 128, threads=4)
        assert int(m.sum()) == round(pt[key] * req * n_layers), (name, frac)


def test_sweep_cells_equal_single_calls():
    idx = np.load(os.path.join(GOLDEN, "qwen3_full.npz"))["idx"].astype(np.int32)[:4, :300]
    caps = [8, 16, 40]
    for name in ("lru", "lfuda", "belady"):
        m = R.trace_misses(name, idx, caps, 128, threads=3)
        for ci, C in enumerate(caps):
            for l in range(idx.shape[0]):
                seq, ranks = P.layer_sequence(idx, l)
                assert m[ci, l] == R.misses(name, seq, C, 128, ranks)
    ev = R.evaluate("lfuda", idx, caps)
    ref = P.evaluate(P.LFUDA, idx.astype(np.int64), caps)
    for C in caps:
        assert abs(ev[C] - ref[C]) < 1e-12


def test_refusals():
    with pytest.raises(ValueError, match="outside"):
        R.misses("lru", [0, 9], 2, 8)
    with pytest.raises(ValueError, match="capacity"):
        R.misses("lru", [0, 1], 0, 8)
    with pytest.raises(ValueError, match="no native policy"):
        R.misses("opt", [0, 1], 2, 8)
    with pytest.raises(ValueError, match="layers, tokens, k"):
        R.trace_misses("lru", np.zeros((4, 8), np.int32), [2])
    with pytest.raises(ValueError, match="outside"):
        R.trace_misses("lru", np.full((2, 3, 2), 5, np.int32), [2], n_experts=4)


ZOO = ("wlfu", "s3fifo", "arc", "lirs", "gaterank", "coact")


@pytest.mark.parametrize("name", ZOO)
@pytest.mark.parametrize("E,C", [(8, 1), (8, 3), (16, 5), (64, 16), (12, 12), (256, 38)])
def test_zoo_native_equals_python(name, E, C):
    """Every policy of the zoo: the native replay and the Python restatement give the same
    misses request for request, on uniform and Zipf-skewed streams whose ranks follow top-8
    tokens (so coact sees token boundaries and gaterank the rank bonus)."""
    rng = np.random.default_rng(E * 7 + C)
    cls = P.POLICIES[name]
    for trial in range(3):
        T = int(rng.integers(1, 120))
        k = min(8, E)
        toks = [rng.choice(E, size=k, replace=False, p=None if trial % 2 == 0 else
                           (lambda w: w / w.sum())(1.0 / np.arange(1, E + 1) ** 1.1))
                for _ in range(T)]
        seq = [int(e) for t in toks for e in t]
        ranks = [r for _ in toks for r in range(k)]
        py = P.simulate(seq, C, E, cls, ranks)["misses"]
        assert R.misses(name, seq, C, E, ranks) == py, (name, trial)


@pytest.mark.parametrize("name", ZOO + ("lru", "lfuda"))
def test_zoo_obeys_the_cache_contract_on_the_trace(name):
    """The reference's audit (tests/test_pool.py section 3): replaying 600 tokens of a real
    routing trace at C=16, victim() always names a resident expert and the cache never holds
    more than C; and no policy beats the Belady bound."""
    idx = np.load(os.path.join(GOLDEN, "qwen3_full.npz"))["idx"].astype(np.int64)
    seq, ranks = P.layer_sequence(idx[:, :600], 0)
    C, E = 16, 128
    pol = P.POLICIES[name](C, E)
    inside = set()
    for e, r in zip(seq, ranks):
        if e in inside:
            pol.touch(e, r)
            continue
        if len(inside) >= C:
            v = pol.victim()
            assert v in inside, (name, v)
            inside.discard(v)
            pol.evicted(v)
        inside.add(e)
        pol.admit(e, r)
        assert len(inside) <= C
    b = P.belady(seq, C)["misses"]
    assert P.simulate(seq, C, E, P.POLICIES[name], ranks)["misses"] >= b


def test_audit_catches_a_cheating_policy():
    """The audit has teeth: a policy naming a non-resident expert is caught."""
    class Cheater(P.Policy):
        def victim(self, exclude=()):
            return 99

    inside = {1, 2}
    assert Cheater(2, 128).victim() not in inside


def test_select_policy_measures_every_candidate():
    """select_policy (pool.py:219-250): reports the LRU and Belady bounds, scores every
    candidate, and the reported best is the highest scorer, natively and in Python alike."""
    idx = np.load(os.path.join(GOLDEN, "qwen3_full.npz"))["idx"].astype(np.int64)[:, :300]
    r = P.select_policy(idx, 16, layers=1)
    assert r["lru"] > r["belady"] > 0
    assert set(r["policies"]) == set(P.CANDIDATES)
    assert all("gap_pct" in v for v in r["policies"].values()), r
    best = max(r["policies"], key=lambda n: r["policies"][n]["gap_pct"])
    assert r["best"] == best
    r2 = P.select_policy(idx, 16, layers=1, native=False)
    for n in P.CANDIDATES:
        assert r2["policies"][n]["miss_rate"] == pytest.approx(r["policies"][n]["miss_rate"])
    assert P.recommended(16, 128).name == "lfuda"
    with pytest.raises(ImportError):
        P.make_policy("no_such_policy", 16, 128)


def _zoo_vectors():
    z = np.load(os.path.join(GOLDEN, "policy_zoo_vectors.npz"))
    cases = sorted({k.split("/")[0] for k in z.files})
    return z, cases


@pytest.mark.parametrize("name", ("wlfu", "s3fifo", "arc", "lirs", "gaterank", "coact", "lfuda",
                                  "lru"))
def test_zoo_matches_the_reference_vectors(name):
    """tests/golden/policy_zoo_vectors.npz holds the reference's own policies' misses and first
    256 victims (written by tests/golden/make_policy_vectors.py from the reference's pure-Python
    policy modules) on uniform and Zipf token streams and two layers of the Qwen3 trace, at
    capacities 4-38. The Python restatement reproduces every victim; the native replay every
    miss count."""
    z, cases = _zoo_vectors()
    cls = P.POLICIES[name]
    n = 0
    for case in cases:
        seq = z[f"{case}/seq"].astype(np.int64)
        ranks = z[f"{case}/ranks"].astype(np.int64)
        E = int(z[f"{case}/n_experts"])
        for key in z.files:
            if not key.startswith(f"{case}/{name}/") or not key.endswith("/misses"):
                continue
            C = int(key.split("/")[2][1:])
            want_m = int(z[key])
            want_v = z[key.replace("/misses", "/victims")].astype(np.int64).tolist()
            pol = cls(C, E)
            inside, misses, vic = set(), 0, []
            for e, r in zip(seq.tolist(), ranks.tolist()):
                if e in inside:
                    pol.touch(e, r)
                    continue
                misses += 1
                if len(inside) >= C:
                    v = pol.victim()
                    if v >= 0:
                        inside.discard(v)
                        pol.evicted(v)
                    vic.append(v)
                inside.add(e)
                pol.admit(e, r)
            assert misses == want_m, (case, C)
            assert vic[:len(want_v)] == want_v, (case, C)
            assert R.misses(name, seq, C, E, ranks) == want_m, (case, C, "native")
            n += 1
    assert n >= 20
