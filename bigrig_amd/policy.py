"""Eviction policies for one layer's expert pool, and the trace tools that measure them.

The contract is the reference's (bigrig_engine/pool.py:29-50): `admit(e, rank)` when an expert
was just placed in a slot, `touch(e, rank)` when a resident expert is requested again,
`victim(exclude)` names the expert to evict (or -1), `evicted(e)` when it really left.

LFUDA is the shipped default (pool.py:126-167): LFU with dynamic aging, counts kept across
eviction and halved there ("ghost" counts), saturating at fcap=12, ties broken by recency
(bigrig_engine/policies/lfuda.py:67-161). Restated here line for line in behaviour, because
slot numbers, and therefore the pool's bit-exact slot lookups, depend on which expert it evicts.
"""
from __future__ import annotations

from collections import OrderedDict, defaultdict


class Policy:
    name = "policy"

    def __init__(self, capacity: int, n_experts: int):
        self.capacity, self.n_experts = capacity, n_experts

    def admit(self, e: int, rank: int = 0) -> None: ...

    def touch(self, e: int, rank: int = 0) -> None: ...

    def victim(self, exclude=()) -> int:
        raise NotImplementedError

    def evicted(self, e: int) -> None: ...


class LRU(Policy):
    """Least recently used (pool.py:53-72). Its victim() takes no exclusion set, so a pool
    using it chooses a legal victim itself when LRU's is protected (stream.py:644-690)."""
    name = "lru"

    def __init__(self, capacity, n_experts):
        super().__init__(capacity, n_experts)
        self.od: OrderedDict = OrderedDict()

    def admit(self, e, rank=0):
        self.od[e] = True
        self.od.move_to_end(e)

    def touch(self, e, rank=0):
        self.od.move_to_end(e)

    def victim(self):
        return next(iter(self.od)) if self.od else -1

    def evicted(self, e):
        self.od.pop(e, None)


class LFUDA(Policy):
    """LFU with dynamic aging (lfuda.py:67-161).

    key(e) = L + count(e), re-anchored to the current age L on every use; count saturates at
    fcap; L rises to the key of each evicted expert; an evicted expert keeps its count,
    multiplied by ghost_decay. victim(exclude) = the resident expert (minus exclude) with the
    smallest (key, last-use tick).
    """
    name = "lfuda"

    def __init__(self, capacity, n_experts, rank_weight: float = 0.0, keep_ghost: bool = True,
                 fcap: float | None = 12.0, ghost_decay: float = 0.5):
        super().__init__(capacity, n_experts)
        self.rank_weight = float(rank_weight)
        self.keep_ghost = bool(keep_ghost)
        self.fcap = fcap
        self.ghost_decay = float(ghost_decay)
        self.L = 0.0
        self.cnt: dict = {}
        self.key: dict = {}
        self.last: dict = {}
        self.resident: set = set()
        self.tick = 0

    def _credit(self, rank: int) -> float:
        return 1.0 if self.rank_weight == 0.0 else 1.0 + self.rank_weight / (1.0 + rank)

    def _bump(self, e: int, rank: int) -> None:
        self.tick += 1
        self.last[e] = self.tick
        c = self.cnt.get(e, 0.0) + self._credit(rank)
        if self.fcap is not None and c > self.fcap:
            c = self.fcap
        self.cnt[e] = c
        self.key[e] = self.L + c

    def admit(self, e: int, rank: int = 0) -> None:
        self.resident.add(e)
        if not self.keep_ghost:
            self.cnt.pop(e, None)
        self._bump(e, rank)

    def touch(self, e: int, rank: int = 0) -> None:
        self._bump(e, rank)

    def victim(self, exclude=()) -> int:
        pool = self.resident if not exclude else (self.resident - set(exclude))
        if not pool:
            return -1
        return min(pool, key=lambda x: (self.key.get(x, 0.0), self.last.get(x, 0)))

    def evicted(self, e: int) -> None:
        k = self.key.pop(e, self.L)
        if k > self.L:
            self.L = k
        self.resident.discard(e)
        if not self.keep_ghost:
            self.cnt.pop(e, None)
            self.last.pop(e, None)
        elif self.ghost_decay != 1.0:
            self.cnt[e] = self.cnt.get(e, 0.0) * self.ghost_decay


POLICIES = {"lfuda": LFUDA, "lru": LRU}


def make_policy(name: str, capacity: int, n_experts: int) -> Policy:
    if name not in POLICIES:
        raise ImportError(f"no policy named {name!r}. Available: {', '.join(sorted(POLICIES))}")
    return POLICIES[name](capacity, n_experts)


# ------------------------------------------------------------------ trace replay
def simulate(seq, capacity: int, n_experts: int, policy_factory, ranks=None) -> dict:
    """Replay one layer's request sequence through a cache (pool.py:252-279): a miss evicts
    victim() when full, then admits."""
    pol = policy_factory(capacity, n_experts)
    resident: set = set()
    misses = hits = 0
    ranks = ranks if ranks is not None else [0] * len(seq)
    for e, r in zip(seq, ranks):
        e = int(e)
        if e in resident:
            hits += 1
            pol.touch(e, r)
            continue
        misses += 1
        if len(resident) >= capacity:
            v = pol.victim()
            if v >= 0:
                resident.discard(v)
                pol.evicted(v)
        resident.add(e)
        pol.admit(e, r)
    n = max(1, hits + misses)
    return {"policy": getattr(pol, "name", "?"), "misses": misses, "hits": hits,
            "requests": n, "miss_rate": misses / n}


def belady(seq, capacity: int) -> dict:
    """Optimal offline eviction (furthest next use), exact (pool.py:282-316)."""
    seq = [int(x) for x in seq]
    nxt: dict = defaultdict(list)
    for i, e in enumerate(seq):
        nxt[e].append(i)
    pos = {e: 0 for e in nxt}
    resident: set = set()
    misses = hits = 0
    for e in seq:
        pos[e] += 1
        if e in resident:
            hits += 1
            continue
        misses += 1
        if len(resident) >= capacity:
            far, victim = -1, None
            for r in resident:
                q, p = nxt[r], pos[r]
                nu = q[p] if p < len(q) else float("inf")
                if nu > far:
                    far, victim = nu, r
            resident.discard(victim)
        resident.add(e)
    n = max(1, hits + misses)
    return {"policy": "belady", "misses": misses, "hits": hits, "requests": n,
            "miss_rate": misses / n}


def layer_sequence(idx, layer: int):
    """One layer's requests from a routing trace idx [layers, tokens, k], flattened in router-
    rank order within each token (pool.py:337-358), with their ranks."""
    L, T, k = idx.shape
    seq = [int(idx[layer, t, r]) for t in range(T) for r in range(k)]
    ranks = [r for _ in range(T) for r in range(k)]
    return seq, ranks


def evaluate(policy_factory, idx, capacities, layers=None) -> dict:
    """Mean miss rate over layers per capacity on a routing trace (pool.py:337-358)."""
    L, T, k = idx.shape
    E = int(idx.max()) + 1
    layers = range(L) if layers is None else layers
    out = {}
    for C in capacities:
        rates = []
        for l in layers:
            seq, ranks = layer_sequence(idx, l)
            rates.append(simulate(seq, C, E, policy_factory, ranks)["miss_rate"])
        out[C] = sum(rates) / len(rates)
    return out
