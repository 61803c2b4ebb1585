"""Eviction policies for one layer's expert pool, and the trace replays that score them.

Contract (the reference's, bigrig_engine/pool.py:29-50): `admit(e, rank)` after expert e was
placed in a slot, `touch(e, rank)` when a resident expert is requested again, `victim()` names
the expert to evict (or -1), `evicted(e)` when it has really left. `rank` is the expert's
position in the router's top-k for the request. A policy whose `excludes` is True takes
`victim(exclude=...)`, a set of experts it must not name; for the others the pool picks a legal
victim itself when the policy names a protected one (stream.py:644-690).

Every policy here keeps its per-expert state in arrays indexed by expert id (E <= 512) and picks
its victim as a lexicographic minimum over its candidates; ordered lists (LRU lists, FIFO
queues, the LIRS stack) are a membership code per expert plus the clock value at which it
entered its list, so "oldest of list X" is the smallest entry stamp among X's members. The
rules -- which decide which expert leaves and therefore every slot number a pool hands out --
are those of the reference's policies:

  lru       least recently admitted-or-touched (pool.py:53-72);
  lfuda     LFU with dynamic aging: credit 1 (or 1 + w/(1 + rank)) per use, saturating at fcap,
            priority = age + credit, victim = lowest (priority, last use), the age rises to the
            evicted priority, an evicted expert keeps its credit times ghost_decay
            (policies/lfuda.py:67-173) -- the shipped default (pool.py:126-167);
  wlfu      fewest uses in a sliding window of the last 128 requests, then least recent
            (pool.py:75-118);
  s3fifo    S3-FIFO: probationary FIFO of ~10% of capacity, main FIFO, ghost FIFO of ids, a hit
            counter capped at 3 (policies/s3fifo.py:1-144);
  arc       Adaptive Replacement Cache (Megiddo and Modha, FAST '03) with the target size of the
            recency list learned from ghost hits, updated on admission (policies/arc.py:1-129);
  lirs      LIRS (Jiang and Zhang, 2002): inter-reference recency, 5% of capacity for resident
            HIR experts, non-resident history bounded to 25% of capacity (policies/lirs.py);
  gaterank  recency with a rank bonus: key = max(old key, tick + 16 * w(rank)), w linear over
            top-8 (policies/gaterank.py);
  coact     decayed self-use plus windowed co-activation affinity (policies/coact.py).

The same rules run natively in csrc/replay.cpp (libbrx_replay.so) for trace sweeps; both are
pinned to each other request for request and to the reference's recorded frontier.
"""
from __future__ import annotations

from collections import deque

import numpy as np

_NONE = 0


class Policy:
    """The policy contract (pool.py:29-50)."""
    name = "policy"
    excludes = False

    def __init__(self, capacity: int, n_experts: int):
        self.capacity, self.n_experts = int(capacity), int(n_experts)

    def admit(self, e: int, rank: int = 0) -> None: ...

    def touch(self, e: int, rank: int = 0) -> None: ...

    def victim(self, exclude=()) -> int:
        raise NotImplementedError

    def evicted(self, e: int) -> None: ...


def _argmin2(mask: np.ndarray, primary, secondary: np.ndarray) -> int:
    """Index of the smallest (primary, secondary) among mask's True entries (primary None:
    secondary alone), -1 when the mask is empty. Secondary values are distinct."""
    cand = np.flatnonzero(mask)
    if cand.size == 0:
        return -1
    if primary is not None:
        p = primary[cand]
        cand = cand[p == p.min()]
    return int(cand[np.argmin(secondary[cand])])


class _Clocked(Policy):
    """A clock, the set of experts the policy counts resident, and per expert (a list indexed
    by expert id) the clock value of its last use -- the tie-break of every policy below. The
    per-step policies keep plain lists: a pool consults them for a handful of experts per layer
    and token, where array-library calls would cost more than the work."""

    def __init__(self, capacity, n_experts):
        super().__init__(capacity, n_experts)
        self.clock = 0
        self.held = set()
        self.used_at = [0] * self.n_experts

    def _stamp(self, e: int) -> None:
        self.clock += 1
        self.used_at[e] = self.clock

    def _lowest(self, primary, exclude=()) -> int:
        """The held expert outside `exclude` with the smallest (primary[e], used_at[e])
        (primary None: used_at alone), -1 if there is none."""
        used = self.used_at
        best, bp, bu = -1, 0.0, 0
        for e in self.held:
            if exclude and e in exclude:
                continue
            p = primary[e] if primary is not None else 0.0
            if best < 0 or p < bp or (p == bp and used[e] < bu):
                best, bp, bu = e, p, used[e]
        return best


class LRU(_Clocked):
    """Least recently admitted or touched (pool.py:53-72). Its victim ignores exclusions."""
    name = "lru"

    def admit(self, e, rank=0):
        self.held.add(e)
        self._stamp(e)

    def touch(self, e, rank=0):
        self._stamp(e)

    def victim(self, exclude=()):
        return self._lowest(None)

    def evicted(self, e):
        self.held.discard(e)


class LFUDA(_Clocked):
    """LFU with dynamic aging (policies/lfuda.py:67-161), over per-expert lists.

    credit[e] accumulates per use (saturating at fcap) and survives eviction scaled by
    ghost_decay; prio[e] = age at the last use + credit; the victim is the resident expert with
    the lowest (prio, last use) outside `exclude`; evicting raises the age to the victim's prio.
    """
    name = "lfuda"
    excludes = True

    def __init__(self, capacity, n_experts, rank_weight: float = 0.0, keep_ghost: bool = True,
                 fcap: float | None = 12.0, ghost_decay: float = 0.5):
        super().__init__(capacity, n_experts)
        self.rank_weight = float(rank_weight)
        self.keep_ghost = bool(keep_ghost)
        self.fcap = None if fcap is None else float(fcap)
        self.ghost_decay = float(ghost_decay)
        self.age = 0.0
        self.credit = [0.0] * self.n_experts
        self.prio = [0.0] * self.n_experts

    def _use(self, e: int, rank: int) -> None:
        self._stamp(e)
        gain = 1.0 if self.rank_weight == 0.0 else 1.0 + self.rank_weight / (1.0 + rank)
        c = self.credit[e] + gain
        if self.fcap is not None and c > self.fcap:
            c = self.fcap
        self.credit[e] = c
        self.prio[e] = self.age + c

    def admit(self, e, rank=0):
        self.held.add(e)
        if not self.keep_ghost:
            self.credit[e] = 0.0
        self._use(e, rank)

    def touch(self, e, rank=0):
        self._use(e, rank)

    def victim(self, exclude=()):
        return self._lowest(self.prio, exclude)

    def evicted(self, e):
        if e in self.held:
            self.age = max(self.age, self.prio[e])
        self.held.discard(e)
        if not self.keep_ghost:
            self.credit[e] = 0.0
        elif self.ghost_decay != 1.0:
            self.credit[e] *= self.ghost_decay


class WindowedLFU(_Clocked):
    """Fewest uses among the last `window` requests, ties to the least recent (pool.py:75-118)."""
    name = "wlfu"

    def __init__(self, capacity, n_experts, window: int = 128):
        super().__init__(capacity, n_experts)
        self.window = int(window)
        self.recent: deque = deque()
        self.uses = [0] * self.n_experts

    def _use(self, e):
        self._stamp(e)
        self.recent.append(e)
        self.uses[e] += 1
        if len(self.recent) > self.window:
            self.uses[self.recent.popleft()] -= 1

    def admit(self, e, rank=0):
        self.held.add(e)
        self._use(e)

    def touch(self, e, rank=0):
        self._use(e)

    def victim(self, exclude=()):
        return self._lowest(self.uses)

    def evicted(self, e):
        self.held.discard(e)


class _Lists(Policy):
    """Membership of every expert in one of a few ordered lists: `where[e]` is the list (0:
    none) and `since[e]` the clock value at which e entered at the list's newest end, so the
    oldest member of a list is its smallest `since`."""

    def __init__(self, capacity, n_experts, n_lists: int):
        super().__init__(capacity, n_experts)
        self.clock = 0
        self.where = np.zeros(self.n_experts, dtype=np.int8)
        self.since = np.zeros(self.n_experts, dtype=np.int64)
        self.size = [0] * (n_lists + 1)

    def _put(self, e: int, lst: int) -> None:
        """Move e to the newest end of list `lst` (0: out of every list)."""
        self.size[int(self.where[e])] -= 1
        self.size[lst] += 1
        self.where[e] = lst
        self.clock += 1
        self.since[e] = self.clock

    def _oldest(self, lst: int) -> int:
        return _argmin2(self.where == lst, None, self.since) if self.size[lst] else -1


class S3FIFO(_Lists):
    """S3-FIFO (policies/s3fifo.py). Lists: 1 probationary S, 2 main M, 3 ghost G (ids only).
    victim() takes its expert out of its queue itself; evicted() cleans up after a victim the
    pool chose instead."""
    name = "s3fifo"
    _S, _M, _G = 1, 2, 3

    def __init__(self, capacity, n_experts):
        super().__init__(capacity, n_experts, 3)
        self.s_target = max(1, int(round(0.10 * self.capacity)))
        self.ghost_max = max(1, int(round(1.0 * self.capacity)))
        self.hits = np.zeros(self.n_experts, dtype=np.int64)

    def admit(self, e, rank=0):
        if self.where[e] in (self._S, self._M):
            return
        self.hits[e] = 0
        self._put(e, self._M if self.where[e] == self._G else self._S)

    def touch(self, e, rank=0):
        if self.hits[e] < 3:
            self.hits[e] += 1

    def victim(self, exclude=()):
        while self.size[self._S] or self.size[self._M]:
            if self.size[self._S] >= self.s_target or not self.size[self._M]:
                e = self._oldest(self._S)
                if self.hits[e] > 1:               # proved itself in probation: to M
                    self.hits[e] = 0
                    self._put(e, self._M)
                    continue
                self.hits[e] = 0
                self._put(e, self._G)              # one-hit wonder: remembered as a ghost
                if self.size[self._G] > self.ghost_max:
                    self._put(self._oldest(self._G), _NONE)
                return e
            e = self._oldest(self._M)
            if self.hits[e] > 0:                   # second chance at M's newest end
                self.hits[e] -= 1
                self._put(e, self._M)
                continue
            self.hits[e] = 0
            self._put(e, _NONE)
            return e
        return -1

    def evicted(self, e):
        self.hits[e] = 0
        if self.where[e] in (self._S, self._M):
            self._put(e, _NONE)


class ARC(_Lists):
    """Adaptive Replacement Cache (policies/arc.py). Lists: 1 T1 (seen once), 2 T2 (seen
    again), 3 B1 and 4 B2 (ids evicted from T1 / T2). `target` is the learned size of T1; a
    ghost hit moves it on admission (the victim was chosen before the arrival is known)."""
    name = "arc"
    _T1, _T2, _B1, _B2 = 1, 2, 3, 4

    def __init__(self, capacity, n_experts):
        super().__init__(capacity, n_experts, 4)
        self.target = 0.0

    def _trim(self) -> None:
        n = self.size
        c = self.capacity
        while n[self._T1] + n[self._B1] > c and n[self._B1]:
            self._put(self._oldest(self._B1), _NONE)
        while n[self._T1] + n[self._T2] + n[self._B1] + n[self._B2] > 2 * c:
            if n[self._B2]:
                self._put(self._oldest(self._B2), _NONE)
            elif n[self._B1]:
                self._put(self._oldest(self._B1), _NONE)
            else:
                break

    def admit(self, e, rank=0):
        n, w = self.size, int(self.where[e])
        if w == self._B1:
            self.target = min(float(self.capacity),
                              self.target + max(1.0, n[self._B2] / max(1, n[self._B1])))
            self._put(e, self._T2)
        elif w == self._B2:
            self.target = max(0.0, self.target - max(1.0, n[self._B1] / max(1, n[self._B2])))
            self._put(e, self._T2)
        else:
            self._put(e, self._T1)
        self._trim()

    def touch(self, e, rank=0):
        self._put(e, self._T2)

    def victim(self, exclude=()):
        n = self.size
        if n[self._T1] and (n[self._T1] > self.target or not n[self._T2]):
            return self._oldest(self._T1)
        if n[self._T2]:
            return self._oldest(self._T2)
        return -1

    def evicted(self, e):
        w = int(self.where[e])
        if w == self._T1:
            self._put(e, self._B1)
        elif w == self._T2:
            self._put(e, self._B2)
        self._trim()


class LIRS(Policy):
    """LIRS (policies/lirs.py): experts with a short inter-reference recency hold LIR status and
    stay; the others (HIR) queue in Q and leave first. The recency stack S holds every LIR
    expert plus HIR experts -- resident or not -- more recent than the oldest LIR one, so a
    re-reference found in S means a short reuse distance. LIR experts are capped at capacity -
    hir_slots; non-resident history in S at hist_slots."""
    name = "lirs"
    _LIR, _HIR = 1, 2

    def __init__(self, capacity, n_experts, hir_ratio: float = 0.05, min_hir: int = 1,
                 hist_ratio: float | None = 0.25):
        super().__init__(capacity, n_experts)
        C, E = self.capacity, self.n_experts
        self.hir_slots = max(1, min(max(int(min_hir), int(round(hir_ratio * C))), C - 1))
        self.lir_slots = C - self.hir_slots
        self.hist_slots = None if hist_ratio is None else max(1, int(round(hist_ratio * C)))
        self.clock = 0
        self.status = np.zeros(E, dtype=np.int8)        # 0 unknown, LIR, HIR
        self.held = np.zeros(E, dtype=bool)
        self.in_s = np.zeros(E, dtype=bool)
        self.s_at = np.zeros(E, dtype=np.int64)          # entry into S's top
        self.in_q = np.zeros(E, dtype=bool)
        self.q_at = np.zeros(E, dtype=np.int64)          # entry into Q's back
        self.n_lir = 0
        self.n_ghost = 0                                 # non-resident experts in S

    def _tick(self) -> int:
        self.clock += 1
        return self.clock

    def _s_push(self, e):
        self.in_s[e] = True
        self.s_at[e] = self._tick()

    def _q_push(self, e):
        self.in_q[e] = True
        self.q_at[e] = self._tick()

    def _s_bottom(self) -> int:
        return _argmin2(self.in_s, None, self.s_at)

    def _prune(self) -> None:
        """Pop HIR experts off the bottom of S until it is LIR; a popped non-resident expert is
        forgotten."""
        while True:
            b = self._s_bottom()
            if b < 0 or self.status[b] == self._LIR:
                return
            self.in_s[b] = False
            if not self.held[b]:
                self.status[b] = 0
                self.n_ghost -= 1

    def _trim_history(self) -> None:
        if self.hist_slots is None:
            return
        while self.n_ghost > self.hist_slots:
            b = _argmin2(self.in_s & ~self.held, None, self.s_at)
            if b < 0:
                self.n_ghost = 0
                return
            self.in_s[b] = False
            self.status[b] = 0
            self.n_ghost -= 1

    def _make_lir(self, e) -> None:
        self.status[e] = self._LIR
        self.n_lir += 1
        self._s_push(e)
        self.in_q[e] = False
        while self.n_lir > self.lir_slots:               # the oldest LIR expert becomes HIR
            self._prune()
            b = self._s_bottom()
            if b < 0:
                break
            self.in_s[b] = False
            self.status[b] = self._HIR
            self.n_lir -= 1
            if self.held[b]:
                self._q_push(b)
            self._prune()
        self._prune()

    def admit(self, e, rank=0):
        found = bool(self.in_s[e])
        if found and not self.held[e]:
            self.n_ghost -= 1
        self.held[e] = True
        if found:
            self._make_lir(e)
        elif self.n_lir < self.lir_slots:
            self.status[e] = self._LIR
            self.n_lir += 1
            self._s_push(e)
        else:
            self.status[e] = self._HIR
            self._s_push(e)
            self._q_push(e)

    def touch(self, e, rank=0):
        if self.status[e] == self._LIR:
            was_bottom = self._s_bottom() == e
            self._s_push(e)
            if was_bottom:
                self._prune()
        elif self.in_s[e]:
            self._make_lir(e)
        else:
            self._s_push(e)
            self._q_push(e)

    def victim(self, exclude=()):
        if self.in_q.any():
            return _argmin2(self.in_q, None, self.q_at)
        self._prune()
        v = _argmin2(self.in_s & self.held, None, self.s_at)
        if v >= 0:
            return v
        held = np.flatnonzero(self.held)
        return int(held[0]) if held.size else -1

    def evicted(self, e):
        self.held[e] = False
        self.in_q[e] = False
        if self.status[e] == self._LIR:
            self.n_lir -= 1
            self.in_s[e] = False
            self.status[e] = 0
        elif self.in_s[e]:
            self.n_ghost += 1
        self._prune()
        self._trim_history()


class GateRank(Policy):
    """Recency with a router-rank bonus (policies/gaterank.py): a use at tick t and rank r gives
    key t + boost * w(r), w(r) = max(0, (k - 1 - r) / (k - 1)) (linear over top-k), never lower
    than the expert's previous key while resident; the victim is the lowest (key, expert id)."""
    name = "gaterank"

    def __init__(self, capacity, n_experts, boost: float = 16.0, k: int = 8,
                 monotone: bool = True):
        super().__init__(capacity, n_experts)
        self.boost = float(boost)
        self.k = int(k)
        self.monotone = bool(monotone)
        self.ticks = 0
        self.key = np.full(self.n_experts, np.nan, dtype=np.float64)

    def _w(self, r: int) -> float:
        return 1.0 if self.k <= 1 else max(0.0, (self.k - 1 - r) / (self.k - 1))

    def _use(self, e, rank):
        self.ticks += 1
        v = self.ticks + self.boost * self._w(rank)
        old = self.key[e]
        if self.monotone and not np.isnan(old) and old > v:
            v = float(old)
        self.key[e] = v

    def admit(self, e, rank=0):
        self._use(e, rank)

    def touch(self, e, rank=0):
        self._use(e, rank)

    def victim(self, exclude=()):
        live = ~np.isnan(self.key)
        if not live.any():
            return -1
        cand = np.flatnonzero(live)
        return int(cand[np.argmin(self.key[cand])])

    def evicted(self, e):
        self.key[e] = np.nan


class CoAct(Policy):
    """Co-activation aware eviction (policies/coact.py).

    score(x) = selfuse(x) + beta * affinity(x); the victim is the resident expert with the
    lowest (score, last use). selfuse decays with a half-life in requests; affinity is the
    credit x received from the last `window` requests y (P(x | y) from same-token counts,
    decayed), granted while x is resident and withdrawn when y leaves the window. A global
    growth factor g stands in for decaying every value each request (values are stored times
    g). Tokens are recognised from the rank stream: a rank not above the previous one opens a
    new token."""
    name = "coact"

    def __init__(self, capacity, n_experts, half_life: float = 128.0, beta: float = 0.8,
                 window: int = 12, max_nb: int = 64, min_support: int = 4, ghost: bool = True,
                 rank_w: float = 0.0):
        super().__init__(capacity, n_experts)
        E = self.n_experts
        self.decay = 0.5 ** (1.0 / float(half_life))
        self.beta, self.window = float(beta), int(window)
        self.max_nb, self.min_support = int(max_nb), int(min_support)
        self.ghost, self.rank_w = bool(ghost), float(rank_w)
        self.held = np.zeros(E, dtype=bool)
        self.selfuse = np.zeros(E, dtype=np.float64)
        self.affinity = np.zeros(E, dtype=np.float64)
        self.last = np.zeros(E, dtype=np.int64)
        self.g = 1.0
        self.t = 0
        self.pairs = [dict() for _ in range(E)]    # partner -> same-token count, in first-seen order
        self.tokens = np.zeros(E, dtype=np.int64)  # tokens containing the expert
        self.token = []
        self.prev_rank = 1 << 30
        self.recent: deque = deque()               # [expert, g at entry, {x: credit granted}]

    def _support(self, y) -> int:
        d = int(self.tokens[y])
        return d if d > self.min_support else self.min_support

    def _end_token(self):
        tok = self.token
        for i, a in enumerate(tok):
            self.tokens[a] += 1
            pa = self.pairs[a]
            for b in tok[i + 1:]:
                pa[b] = pa.get(b, 0) + 1
                pb = self.pairs[b]
                pb[a] = pb.get(a, 0) + 1
            if len(pa) > 2 * self.max_nb:             # keep the most frequent partners
                self.pairs[a] = dict(sorted(pa.items(), key=lambda kv: -kv[1])[:self.max_nb])
        self.token = []

    def _clock(self, e, rank):
        if rank <= self.prev_rank:
            self._end_token()
        self.prev_rank = rank
        self.token.append(e)
        self.t += 1
        self.g /= self.decay
        if self.g > 1e120:                            # rescale before the range runs out
            s = self.g
            self.selfuse /= s
            self.affinity /= s
            for ent in self.recent:
                ent[1] /= s
                for x in ent[2]:
                    ent[2][x] /= s
            self.g = 1.0

    def _grant(self, e):
        """Credit every resident partner of e for this request; retire the request that leaves
        the window."""
        given = {}
        if self.beta:
            scale = self.g / self._support(e)
            for x, c in self.pairs[e].items():
                if x != e and self.held[x]:
                    v = c * scale
                    self.affinity[x] += v
                    given[x] = v
        self.recent.append([e, self.g, given])
        while len(self.recent) > self.window:
            _, _, gone = self.recent.popleft()
            for x, v in gone.items():
                if self.held[x]:
                    self.affinity[x] -= v

    def _seed(self, e) -> float:
        """Affinity of an expert admitted now: the credit it would have received from the
        requests in the window, recorded so that it is withdrawn with them."""
        if not self.beta:
            return 0.0
        total = 0.0
        for ent in self.recent:
            y, gy, given = ent
            if y == e:
                continue
            v = given.get(e)
            if v is None:
                c = self.pairs[y].get(e)
                if not c:
                    continue
                v = (c / self._support(y)) * gy
                given[e] = v
            total += v
        return total

    def _credit(self, rank) -> float:
        return self.g * (1.0 + self.rank_w / (1.0 + rank))

    def admit(self, e, rank=0):
        self._clock(e, rank)
        self.held[e] = True
        self.affinity[e] = self._seed(e)
        if not self.ghost:
            self.selfuse[e] = 0.0
        self.selfuse[e] += self._credit(rank)
        self.last[e] = self.t
        self._grant(e)

    def touch(self, e, rank=0):
        self._clock(e, rank)
        self.selfuse[e] += self._credit(rank)
        self.last[e] = self.t
        self._grant(e)

    def victim(self, exclude=()):
        return _argmin2(self.held, self.selfuse + self.beta * self.affinity, self.last)

    def evicted(self, e):
        self.held[e] = False
        self.affinity[e] = 0.0
        if not self.ghost:
            self.selfuse[e] = 0.0


POLICIES = {"lru": LRU, "lfuda": LFUDA, "wlfu": WindowedLFU, "windowed_lfu": WindowedLFU,
            "s3fifo": S3FIFO, "arc": ARC, "lirs": LIRS, "gaterank": GateRank, "coact": CoAct}
CANDIDATES = ("lfuda", "s3fifo", "gaterank", "lirs", "arc", "coact")


def make_policy(name: str, capacity: int, n_experts: int) -> Policy:
    """A policy by the name the reference's pool takes (pool.py:189-216), in its shipped
    configuration. Unknown names raise ImportError, as the reference's resolver does."""
    cls = POLICIES.get(name)
    if cls is None:
        raise ImportError(f"no policy named {name!r}. Available: {', '.join(sorted(POLICIES))}")
    return cls(capacity, n_experts)


def recommended(capacity: int = 0, n_experts: int = 0):
    """The default policy (pool.py:126-167): LFUDA in its shipped configuration; with no sizes,
    the factory."""
    return LFUDA(capacity, n_experts) if capacity else LFUDA


# ------------------------------------------------------------------ trace replay
def simulate(seq, capacity: int, n_experts: int, policy_factory, ranks=None) -> dict:
    """Replay one layer's requests through a cache of `capacity` experts (pool.py:252-279): a
    hit touches, a miss first evicts victim() when the cache is full, then admits."""
    pol = policy_factory(capacity, n_experts)
    inside = np.zeros(n_experts, dtype=bool)
    count = 0
    misses = 0
    n = len(seq)
    rk = ranks if ranks is not None else [0] * n
    for e, r in zip(seq, rk):
        e, r = int(e), int(r)
        if inside[e]:
            pol.touch(e, r)
            continue
        misses += 1
        if count >= capacity:
            v = pol.victim()
            if v >= 0:
                inside[v] = False
                count -= 1
                pol.evicted(v)
        inside[e] = True
        count += 1
        pol.admit(e, r)
    total = max(1, n)
    return {"policy": getattr(pol, "name", "?"), "misses": misses, "hits": n - misses,
            "requests": total, "miss_rate": misses / total}


def next_use(seq) -> np.ndarray:
    """For each request, the position of the same expert's next request (len(seq) + expert id
    when it never comes back: distinct, and beyond every real position)."""
    s = np.asarray(seq, dtype=np.int64)
    n = s.size
    out = np.empty(n, dtype=np.int64)
    seen = {}
    for i in range(n - 1, -1, -1):
        e = int(s[i])
        out[i] = seen.get(e, n + e)
        seen[e] = i
    return out


def belady(seq, capacity: int) -> dict:
    """The optimal offline bound (pool.py:282-316): on a miss with the cache full, evict the
    resident expert whose next request is furthest away. A max-heap of (next use, expert) with
    stale entries skipped."""
    import heapq
    nu = next_use(seq)
    due = {}                      # resident expert -> position of its next request
    heap = []
    misses = 0
    for i, e in enumerate(seq):
        e = int(e)
        if e in due:
            due[e] = int(nu[i])
            heapq.heappush(heap, (-due[e], e))
            continue
        misses += 1
        if len(due) >= capacity:
            while True:
                d, v = heapq.heappop(heap)
                if due.get(v) == -d:
                    del due[v]
                    break
        due[e] = int(nu[i])
        heapq.heappush(heap, (-due[e], e))
    n = max(1, len(seq))
    return {"policy": "belady", "misses": misses, "hits": len(seq) - misses, "requests": n,
            "miss_rate": misses / n}


def layer_sequence(idx, layer: int):
    """(requests, ranks) of one layer of a routing trace idx [layers, tokens, k]: each token's
    experts in router-rank order (pool.py:337-358)."""
    L, T, k = idx.shape
    seq = np.asarray(idx[layer], dtype=np.int64).reshape(-1)
    ranks = np.tile(np.arange(k, dtype=np.int64), T)
    return seq.tolist(), ranks.tolist()


def evaluate(policy_factory, idx, capacities, layers=None) -> dict:
    """Mean miss rate over layers per capacity on a routing trace (pool.py:337-358)."""
    L = idx.shape[0]
    E = int(np.max(idx)) + 1
    rows = range(L) if layers is None else layers
    seqs = [layer_sequence(idx, l) for l in rows]
    out = {}
    for C in capacities:
        rates = [simulate(seq, C, E, policy_factory, ranks)["miss_rate"] for seq, ranks in seqs]
        out[C] = sum(rates) / len(rates)
    return out


def select_policy(idx, capacity: int, candidates=None, layers: int = 2,
                  n_experts: int | None = None, native: bool = True) -> dict:
    """Measure every candidate on the first `layers` layers of a routing trace at `capacity`
    and pick the one that captures the largest share of the LRU-to-Belady gap
    (pool.py:219-250). A candidate that fails is reported with its error, never dropped. With
    `native`, the replay runs in libbrx_replay.so."""
    names = list(candidates or CANDIDATES)
    idx = np.asarray(idx)
    n_l = min(layers, idx.shape[0])
    E = n_experts or int(idx.max()) + 1
    sub = np.ascontiguousarray(idx[:n_l], dtype=np.int32)
    per = sub.shape[1] * sub.shape[2]

    def rate(name):
        if native:
            from . import replay as R
            return float(R.trace_misses(name, sub, [capacity], E).sum()) / (n_l * per)
        if name == "belady":
            return float(np.mean([belady(layer_sequence(sub, l)[0], capacity)["miss_rate"]
                                  for l in range(n_l)]))
        cls = POLICIES[name]
        return float(np.mean([simulate(seq, capacity, E, cls, ranks)["miss_rate"]
                              for seq, ranks in (layer_sequence(sub, l) for l in range(n_l))]))

    lru, bel = rate("lru"), rate("belady")
    out = {"lru": lru, "belady": bel, "policies": {}}
    for n in names:
        try:
            v = rate(n)
            gap = (lru - v) / (lru - bel) * 100.0 if lru > bel else 0.0
            out["policies"][n] = {"miss_rate": v, "gap_pct": gap}
        except Exception as ex:                       # reported, not hidden
            out["policies"][n] = {"error": str(ex)[:120]}
    ok = {n: d for n, d in out["policies"].items() if "gap_pct" in d}
    out["best"] = max(ok, key=lambda n: ok[n]["gap_pct"]) if ok else "lru"
    out["best_gap_pct"] = ok[out["best"]]["gap_pct"] if ok else 0.0
    return out
