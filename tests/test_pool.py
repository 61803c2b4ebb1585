"""Residency bookkeeping and eviction policies (CPU).

Pins: the reference's policy known answers (tests/test_pool.py:24-52), its slot-table
invariants and error cases (tests/test_stream.py:72-223, 488-503), and its recorded trace
replays: `data/results/frontier_locality_qwen3.json` over `data/traces/qwen3_full.npz` (both
copied to tests/golden), which the LRU, LFUDA and Belady replays here must reproduce to the
request.
"""
import json
import os

import numpy as np
import pytest

from bigrig_amd import policy as P
from bigrig_amd.layer import StreamingSwitchGLU
from bigrig_amd.pool import ExpertPool
from bigrig_amd.spec import QWEN3_30B_A3B
from tests.helpers import small

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ------------------------------------------------------------------ policies
def test_lru_known_answers():
    seq = [1, 2, 3] * 3
    r = P.simulate(seq, 3, 8, P.LRU)
    assert (r["misses"], r["hits"]) == (3, 6)
    assert P.simulate(seq, 2, 8, P.LRU)["misses"] == 9
    assert P.belady(seq, 2)["misses"] < 9
    assert P.simulate(seq, 8, 8, P.LRU)["misses"] == 3
    for c in (1, 2, 3, 8):
        r = P.simulate(seq, c, 8, P.LRU)
        assert r["hits"] + r["misses"] == len(seq)


def test_belady_is_a_lower_bound():
    rng = np.random.default_rng(0)
    for _ in range(12):
        s = rng.integers(0, 12, 300).tolist()
        C = int(rng.integers(2, 8))
        b = P.belady(s, C)["misses"]
        assert P.simulate(s, C, 12, P.LRU)["misses"] >= b
        assert P.simulate(s, C, 12, P.LFUDA)["misses"] >= b


def test_belady_brute_force_tiny():
    """Belady equals the minimum over every eviction choice on tiny sequences."""
    def best(seq, C):
        # exhaustive search over states (resident set) per position
        states = {frozenset(): 0}
        for e in seq:
            nxt = {}
            for st, m in states.items():
                if e in st:
                    cands = [(st, m)]
                elif len(st) < C:
                    cands = [(st | {e}, m + 1)]
                else:
                    cands = [((st - {v}) | {e}, m + 1) for v in st]
                for s2, m2 in cands:
                    if s2 not in nxt or m2 < nxt[s2]:
                        nxt[s2] = m2
            states = nxt
        return min(states.values())

    rng = np.random.default_rng(1)
    for _ in range(30):
        seq = rng.integers(0, 5, 12).tolist()
        C = int(rng.integers(1, 4))
        assert P.belady(seq, C)["misses"] == best(seq, C)


def test_lfuda_known_answers():
    """Hand-worked LFUDA: count+1 per use, key = L + count, victim = min (key, last tick),
    L rises to the evicted key, a ghost keeps half its count."""
    p = P.LFUDA(2, 8)
    p.admit(1); p.admit(2); p.touch(1)          # credit 1:2, 2:1; priorities 2, 1
    assert p.victim() == 2
    p.evicted(2)                                # age = 1; ghost credit(2) = 0.5
    assert p.age == 1.0 and p.credit[2] == 0.5
    p.admit(3)                                  # prio(3) = 1 + 1 = 2, used later than 1
    assert p.prio[3] == 2.0 and p.victim() == 1  # tie on priority 2: the older use goes
    assert p.victim(exclude={1}) == 3
    assert p.victim(exclude={1, 3}) == -1
    p.evicted(1)
    p.admit(2)                                  # ghost: 0.5 + 1 = 1.5, prio = age + 1.5 = 3.5
    assert p.credit[2] == 1.5 and p.prio[2] == pytest.approx(3.5)
    # the credit saturates at 12
    for _ in range(20):
        p.touch(3)
    assert p.credit[3] == 12.0


def _frontier():
    with open(os.path.join(GOLDEN, "frontier_locality_qwen3.json")) as f:
        return json.load(f)["curve"]


def _trace():
    return np.load(os.path.join(GOLDEN, "qwen3_full.npz"))["idx"].astype(np.int64)


@pytest.mark.parametrize("frac", ["0.1", "0.25", "0.5"])
def test_trace_replay_reproduces_recorded_frontier(frac):
    """data/results/frontier_locality_qwen3.json: LFUDA ('miss'), LRU and Belady mean miss
    rates over the first 8 layers of the Qwen3 routing trace, to the request."""
    cur = _frontier()
    idx = _trace()
    pt = cur["points"][frac]
    C, n_layers = pt["capacity"], cur["layers"]
    req = cur["tokens"] * cur["k"]
    for name, rate in (("lru", lambda s, r: P.simulate(s, C, 128, P.LRU, r)),
                       ("miss", lambda s, r: P.simulate(s, C, 128, P.LFUDA, r)),
                       ("belady", lambda s, r: P.belady(s, C))):
        misses = sum(rate(*P.layer_sequence(idx, l))["misses"] for l in range(n_layers))
        assert misses == round(pt[name] * req * n_layers), (name, frac)


# ------------------------------------------------------------------ the pool, on recording slots
class RecordingSlots:
    """Stands in for the HBM slots: records each write and each table upload."""

    def __init__(self):
        self.writes = []
        self.tables = []

    def write(self, slot, blob):
        self.writes.append((slot, bytes(blob[:4])))
        return len(blob)

    def write_device(self, slot, ptr, n):
        self.writes.append((slot, ptr))
        return n

    def set_table(self, g2s, stream):
        self.tables.append(np.array(g2s, copy=True))

    def close(self):
        pass


SPEC = small(QWEN3_30B_A3B, hidden=128, inter=64, n_experts=16, top_k=4)
BLOCK = bytes(SPEC.bytes_per_expert)


def fresh(C=6, E=16, policy="lfuda"):
    spec = small(SPEC, n_experts=E)
    return ExpertPool(0, spec, C, policy=policy, slots=RecordingSlots()).build()


def test_tables_agree_both_ways():
    C = 6
    p = fresh(C)
    assert (p.g2s < 0).all()
    for e in range(C):
        p.touch([e], [0])
        p.admit(e, BLOCK)
    assert sorted(p.s2g.tolist()) == list(range(C))
    assert all(p.g2s[p.s2g[s]] == s for s in range(C))
    # the free list pops from the end: expert 0 went to slot C-1
    assert [p.slot_of(e) for e in range(C)] == list(range(C - 1, -1, -1))
    before = set(p.s2g.tolist())
    p.touch([C], [0])
    p.admit(C, BLOCK)
    assert len(set(p.s2g.tolist()) - before) == 1 and (p.s2g >= 0).sum() == C
    assert sum(1 for e in range(16) if p.g2s[e] >= 0) == C


def test_protected_experts_are_never_evicted_and_errors():
    C = 6
    p = fresh(C)
    need = list(range(C))
    for e in need:
        p.touch([e], [0])
        p.admit(e, BLOCK, protect=need)
    assert all(p.g2s[e] >= 0 for e in need)
    writes = len(p.device.writes)
    g2s = p.g2s.copy()
    p.touch([C + 1], [0])
    with pytest.raises(RuntimeError, match="top-k"):
        p.admit(C + 1, BLOCK, protect=list(range(C + 2)))
    assert np.array_equal(p.g2s, g2s) and len(p.device.writes) == writes
    with pytest.raises(ValueError):
        fresh(17)
    with pytest.raises(ValueError):
        fresh(0)
    p2 = ExpertPool(0, SPEC, 6, slots=RecordingSlots())
    with pytest.raises(RuntimeError):
        p2.admit(0, BLOCK)
    p3 = fresh()
    p3.touch([0], [0])
    with pytest.raises(ValueError, match="manifest accounts"):
        p3.admit(0, BLOCK[:-4])
    assert p3.g2s[0] == -1 and not p3.device.writes


def test_churn_pool_and_policy_agree():
    """200 steps of 8 experts out of 32 at C=12 (tests/test_stream.py:148-184)."""
    pd = fresh(12, 32)
    assert pd.policy.excludes
    rng = np.random.default_rng(0)
    for _ in range(200):
        want = sorted(rng.choice(32, size=8, replace=False).tolist())
        for e in pd.touch(want, list(range(8))):
            pd.admit(e, BLOCK, protect=want)
        assert all(pd.g2s[e] >= 0 for e in want)
    pool_r = {int(e) for e in range(32) if pd.g2s[e] >= 0}
    assert pool_r == pd.policy.held
    assert pd.policy.victim() in pool_r
    assert pd.policy.age <= pd.evicts * 1.2 + 1
    assert all(pd.g2s[pd.s2g[s]] == s for s in range(12) if pd.s2g[s] >= 0)
    # a policy without exclude= (LRU): the pool chooses for itself, and the views still agree
    pl = fresh(12, 32, policy="lru")
    assert not pl.policy.excludes
    for _ in range(120):
        want = sorted(rng.choice(32, size=8, replace=False).tolist())
        for e in pl.touch(want, list(range(8))):
            pl.admit(e, BLOCK, protect=want)
    assert {int(e) for e in range(32) if pl.g2s[e] >= 0} == pl.policy.held


def test_residency_is_counted():
    pc = fresh(8, 8)
    assert not pc.full
    for e in range(8):
        pc.touch([e], [0])
        pc.admit(e, BLOCK)
    assert pc.full and pc.resident == int((pc.g2s >= 0).sum())
    pe = fresh(4, 8)
    for e in range(8):
        pe.touch([e], [0])
        pe.admit(e, BLOCK)
    assert not pe.full and pe.resident == int((pe.g2s >= 0).sum()) == 4


def test_device_table_uploads_only_on_change():
    """tests/test_stream.py:488-503: the device table equals the host's and is not re-sent on
    a hit; g2s is uploaded whole, -1 for absent experts (the kernels never read those)."""
    pf = fresh(16, 16)
    for e in range(16):
        pf.touch([e], [0])
        pf.admit(e, BLOCK)
    pf.g2s_device(None)
    assert len(pf.device.tables) == 1 and np.array_equal(pf.device.tables[0], pf.g2s)
    pf.g2s_device(None)
    pf.touch([0], [0])
    pf.g2s_device(None)
    assert len(pf.device.tables) == 1
    pp = fresh(4, 16)
    for e in range(5):
        pp.touch([e], [0])
        pp.admit(e, BLOCK)
    pp.g2s_device(None)
    pp.g2s_device(None)
    assert len(pp.device.tables) == 1 and (pp.device.tables[0] == -1).sum() == 12


class _Fetcher:
    def __init__(self):
        self.calls = []

    def fetch(self, keys):
        self.calls.append(list(keys))
        return {k: bytes([k[1] % 256]) * SPEC.bytes_per_expert for k in keys}


def test_ensure_order_rules_fix_slot_numbers():
    """stream.py:922-978: a step's experts are touched in ascending id with their best rank,
    misses admitted in ascending id with the step protected, so slot numbers are a function of
    the request history alone. A warm full pass maps expert e to slot E-1-e."""
    pool = fresh(16, 16)
    sw = StreamingSwitchGLU(pool, _Fetcher())
    for e in range(16):
        sw.ensure(np.array([[e]]))
    assert [pool.slot_of(e) for e in range(16)] == [15 - e for e in range(16)]
    # a bounded pool: request [[9, 3, 5, 3]] admits 3, 5, 9 in that order
    pool = fresh(6, 16)
    f = _Fetcher()
    sw = StreamingSwitchGLU(pool, f)
    slots = sw.ensure(np.array([[9, 3, 5, 3]]))
    assert f.calls == [[(0, 3), (0, 5), (0, 9)]]
    assert [pool.slot_of(e) for e in (3, 5, 9)] == [5, 4, 3]
    assert slots.tolist() == [[3, 5, 4, 5]]
    assert [w[0] for w in pool.device.writes] == [5, 4, 3]
    # best rank: expert 3 appears at ranks 1 and 3, the policy sees rank 1
    assert pool.miss_ranks == {3: 1, 5: 2, 9: 0}
    # a step that needs more experts than the pool holds is refused before any write
    n = len(pool.device.writes)
    with pytest.raises(RuntimeError, match="pool holds"):
        sw.ensure(np.array([[0, 1, 2, 4, 6, 7, 8]]))
    assert len(pool.device.writes) == n
    with pytest.raises(KeyError):
        sw.ensure(np.array([[16]]))


def test_ensure_replay_is_deterministic_and_bounded():
    """Replaying the Qwen3 trace's layer 0 through ensure() at C=32 twice gives the same slot
    history, the pool never holds more than C, and every step's experts are resident after it."""
    idx = _trace()[0, :300]
    spec = small(SPEC, n_experts=128, top_k=8)

    def run():
        pool = ExpertPool(0, spec, 32, slots=RecordingSlots()).build()
        sw = StreamingSwitchGLU(pool, _Fetcher())
        hist = []
        for t in range(idx.shape[0]):
            s = sw.ensure(idx[t:t + 1])
            assert (s >= 0).all() and (pool.s2g >= 0).sum() <= 32
            assert all(pool.s2g[s[0, j]] == idx[t, j] for j in range(8))
            hist.append(s.copy())
        return np.concatenate(hist), pool.stats()

    h1, st1 = run()
    h2, st2 = run()
    assert np.array_equal(h1, h2) and st1["misses"] == st2["misses"]
    assert 0.2 < st1["miss_rate"] < 0.6
