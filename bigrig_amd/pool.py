"""The bounded expert pool of one layer: HBM slots, expert<->slot tables, eviction policy.

`ExpertPool` keeps the residency of the reference's ExpertPool (bigrig_engine/stream.py:454-811)
-- the same slot-assignment and victim rules and the same errors, so the same requests produce
the same slot numbers -- over slots that live in HBM (libbrx `brx_pool_*`). Where the reference wrote an MLX slot tensor
(`self._slots[...][slot] = arrays[i]`, stream.py:765-769) this issues an asynchronous copy of
the expert's packed bytes from pinned host memory on a side stream; the library orders that
copy after every forward that may still read the slot, and the next forward after the copy.

`HostStore` is the pinned host copy of every expert a pool can admit, laid out as the blob
(stream.py:106-186), and `PinnedFetcher` serves it under the reference fetcher's duck type
(`fetch(keys) -> {(layer, e): region}`, test_plan_invariance.py:79-87).
"""
from __future__ import annotations

import os
import time
from dataclasses import dataclass

import numpy as np

from . import formats as F
from .policy import make_policy
from .spec import LayerSpec


@dataclass
class PinnedRegion:
    """One expert's packed bytes in pinned host memory."""
    ptr: int
    nbytes: int
    owner: object = None   # keeps the backing allocation alive

    def __len__(self) -> int:
        return self.nbytes


class HostStore:
    """Packed experts in pinned (page-locked) host memory, one [E, bytes_per_expert] block per
    layer. Replaces the reference's page-cache reads (WeightStore, fetch.py:161-387): a miss is
    one PCIe copy from here."""

    def __init__(self):
        self._layers = {}

    def add_layer(self, layer: int, experts) -> None:
        """experts: list of equal-length bytes, or a uint8 array [E, bytes_per_expert]."""
        import torch
        if isinstance(experts, np.ndarray):
            arr = np.ascontiguousarray(experts, dtype=np.uint8)
        else:
            n = {len(b) for b in experts}
            if len(n) != 1:
                raise ValueError(f"layer {layer}: experts differ in size {sorted(n)}")
            arr = np.frombuffer(b"".join(experts), dtype=np.uint8).reshape(len(experts), -1)
        t = torch.empty(arr.shape, dtype=torch.uint8, pin_memory=True)
        t.numpy()[...] = arr
        self._layers[int(layer)] = t

    def add_layer_tensor(self, layer: int, t) -> None:
        """A pinned torch uint8 tensor [E, bytes_per_expert] (e.g. filled from the GPU)."""
        if not t.is_pinned():
            raise ValueError("HostStore tensors must be pinned")
        self._layers[int(layer)] = t

    @classmethod
    def from_blob(cls, path: str, manifest: F.Manifest, layers=None) -> "HostStore":
        """Read every expert region of `layers` (default: all) from a packed blob."""
        st = cls()
        mm = np.memmap(path, dtype=np.uint8, mode="r")
        for li in sorted(int(x) for x in manifest.layers) if layers is None else layers:
            e = manifest.layers[str(li)]
            E, per = int(e["n_experts"]), int(e["bytes_per_expert"])
            rows = []
            for x in range(E):
                o, n = manifest.region(li, x)
                if n != per:
                    raise ValueError(f"region {li}:{x} is {n} bytes, layer says {per}")
                rows.append(np.asarray(mm[o:o + n]))
            st.add_layer(li, np.stack(rows))
        return st

    @classmethod
    def from_checkpoint(cls, model_dir_or_manifest, layers=None) -> "HostStore":
        """Read every routed expert of `layers` (default: all) straight out of an MLX
        checkpoint's safetensors shards into pinned memory, each expert's segments in packing
        order, so a row holds exactly the bytes a packed blob region would (direct.py:145-240)."""
        import torch

        from . import checkpoint as CK
        man = (model_dir_or_manifest if isinstance(model_dir_or_manifest, CK.CheckpointManifest)
               else CK.expert_manifest(model_dir_or_manifest))
        st = cls()
        fds = {}
        try:
            for li in sorted(int(x) for x in man.layers) if layers is None else layers:
                ent = man.layers[str(li)]
                E, per = int(ent["n_experts"]), int(ent["bytes_per_expert"])
                t = torch.empty((E, per), dtype=torch.uint8, pin_memory=True)
                rows = t.numpy()
                for e in range(E):
                    CK.read_expert_into(man, li, e, rows[e], fds)
                st._layers[int(li)] = t
        finally:
            for fd in fds.values():
                os.close(fd)
        return st

    def region(self, layer: int, e: int) -> PinnedRegion:
        t = self._layers.get(int(layer))
        if t is None or not 0 <= int(e) < t.shape[0]:
            raise KeyError((layer, e))
        row = t[int(e)]
        return PinnedRegion(row.data_ptr(), row.numel(), t)

    def tensor(self, layer: int):
        return self._layers[int(layer)]

    def layers(self):
        return sorted(self._layers)

    @property
    def nbytes(self) -> int:
        return sum(t.numel() for t in self._layers.values())


class PinnedFetcher:
    """The fetcher duck type over a HostStore: every expert is already in pinned memory, so
    prefetch/drop/warm have nothing to do."""

    def __init__(self, store: HostStore):
        self.store = store
        self.fetches = 0

    def fetch(self, keys) -> dict:
        self.fetches += len(keys)
        return {k: self.store.region(*k) for k in keys}

    def prefetch(self, keys) -> None:
        pass

    def drop(self, keys) -> None:
        pass

    def warm(self, keys) -> None:
        pass


class DeviceSlots:
    """The HBM side of a pool: libbrx slot array + device table, and the side copy stream the
    refills run on (default priority)."""

    def __init__(self, spec: LayerSpec, capacity: int, device: int = 0, copy_stream=None):
        import ctypes as C

        import torch
        from . import lib as L
        L.init(device)
        self._L = L
        self.spec = spec
        self.desc = spec.desc()
        h = C.c_void_p()
        L.check(L.load().brx_pool_create(C.byref(self.desc), capacity, C.byref(h)))
        self.handle = h
        self.capacity = capacity
        self.copy_stream = copy_stream if copy_stream is not None else torch.cuda.Stream(device)
        self._stage = None          # pinned staging for non-pinned sources, and its event
        self._stage_ev = None

    def write(self, slot: int, blob) -> int:
        """Queue the copy of one expert into `slot`; returns the bytes copied."""
        import torch
        L = self._L
        cs = self.copy_stream.cuda_stream
        if isinstance(blob, PinnedRegion):
            L.check(L.load().brx_pool_refill_async(self.handle, slot, blob.ptr, blob.nbytes, cs))
            return blob.nbytes
        raw = np.frombuffer(blob, dtype=np.uint8)
        if self._stage_ev is not None:
            # the previous copy out of the staging buffer must have finished before the buffer
            # is rewritten or handed back to torch's pinned-memory cache
            self._stage_ev.synchronize()
        if self._stage is None or self._stage.numel() < raw.nbytes:
            self._stage = torch.empty(raw.nbytes, dtype=torch.uint8, pin_memory=True)
        self._stage.numpy()[:raw.nbytes] = raw
        L.check(L.load().brx_pool_refill_async(self.handle, slot, self._stage.data_ptr(),
                                               raw.nbytes, cs))
        self._stage_ev = torch.cuda.Event()
        self._stage_ev.record(self.copy_stream)
        return raw.nbytes

    def write_range(self, slot0: int, host_ptr: int, n: int, host_stride: int, nbytes: int) -> int:
        """Queue the copies of n experts in pinned host memory (expert i at host_ptr + i *
        host_stride) into slots slot0 .. slot0 + n - 1, one transfer when they are back to back
        on both sides; returns the bytes copied."""
        L = self._L
        L.check(L.load().brx_pool_refill_range_async(self.handle, slot0, n, host_ptr, host_stride,
                                                     nbytes, self.copy_stream.cuda_stream))
        return n * nbytes

    def write_device(self, slot: int, dev_ptr: int, nbytes: int, src_stream=None) -> int:
        """Queue the copy of an expert staged in device memory into `slot`. The source is
        written by work on `src_stream` (default: the current stream), so the copy stream
        first waits for everything queued there; without that wait the copy can read the
        staging buffer before its producer has finished writing it."""
        import torch
        L = self._L
        src = src_stream if src_stream is not None else torch.cuda.current_stream()
        ready = torch.cuda.Event()
        ready.record(src)
        self.copy_stream.wait_event(ready)
        L.check(L.load().brx_pool_refill_from_device_async(self.handle, slot, dev_ptr, nbytes,
                                                           self.copy_stream.cuda_stream))
        return nbytes

    def set_table(self, g2s: np.ndarray, stream) -> None:
        import ctypes as C
        L = self._L
        t = np.ascontiguousarray(g2s, dtype=np.int32)
        L.check(L.load().brx_pool_set_g2s(self.handle, t.ctypes.data_as(C.POINTER(C.c_int32)),
                                          t.size, stream))

    def slot_ptr(self, slot: int) -> int:
        import ctypes as C
        L = self._L
        out = C.c_void_p()
        L.check(L.load().brx_pool_slot_ptr(self.handle, slot, C.byref(out)))
        return out.value

    def sync(self) -> None:
        self._L.check(self._L.load().brx_pool_sync(self.handle))

    def check(self) -> None:
        """Wait for the pool's work, then raise (BrxError, code BRX_ERANGE) if a forward routed to
        an expert that was neither resident nor host-backed (its rows were written as NaN)."""
        self._L.check(self._L.load().brx_pool_check(self.handle))

    def close(self) -> None:
        if self.handle is not None:
            self._L.check(self._L.load().brx_pool_destroy(self.handle))
            self.handle = None


def step_requests(indices, ranks=None):
    """The distinct experts of one step in ascending id, each with the best (lowest) router rank
    it was requested at: the order and the rank the pool is told about them (stream.py:933-950).
    `ranks` defaults to the position along the last axis of `indices` (the router's top-k
    order)."""
    gi = np.asarray(indices, dtype=np.int64)
    if ranks is None and gi.ndim >= 1 and gi.size <= 256:   # a decode step: plain loops
        best = {}
        for row in gi.reshape(-1, gi.shape[-1]).tolist():
            for r, e in enumerate(row):
                if r < best.get(e, r + 1):
                    best[e] = r
        uniq = sorted(best)
        return uniq, [best[e] for e in uniq]
    if ranks is None:
        rk = np.broadcast_to(np.arange(gi.shape[-1], dtype=np.int64), gi.shape) if gi.ndim else gi * 0
    else:
        rk = np.asarray(ranks, dtype=np.int64)
    ids, rs = gi.reshape(-1), rk.reshape(-1)
    if ids.size <= 256:                                # a decode step: a dict is cheapest
        best = {}
        for e, r in zip(ids.tolist(), rs.tolist()):
            if r < best.get(e, r + 1):
                best[e] = r
        uniq = sorted(best)
        return uniq, [best[e] for e in uniq]
    order = np.lexsort((rs, ids))                     # by id, then rank
    uniq, first = np.unique(ids[order], return_index=True)
    return uniq.tolist(), rs[order][first].tolist()


class ExpertPool:
    """C slots of expert weights for ONE layer and the tables that say which expert is where.

    The residency rules are the reference's (stream.py:454-811), since they decide every slot
    number a forward looks up:
      * g2s [E] and s2g [C] int32 tables, -1 for absent / free;
      * slots never used are handed out from the top down (the first admission takes slot
        C - 1), and a slot freed by an eviction goes straight to the admission that caused it;
      * a victim is the policy's, unless it is protected (the step's own experts) or the policy
        cannot exclude; then the unprotected slot admitted longest ago;
      * every error is raised before a slot or a table is touched.
    The tables here are plain arrays: `admitted_at[slot]` orders slots by admission for the
    fallback, `_fresh` counts the never-used slots left.
    """

    def __init__(self, layer: int, spec: LayerSpec, capacity: int, policy: str = "lfuda",
                 slots=None, device: int = 0):
        n_experts = spec.n_experts
        if not 1 <= capacity <= n_experts:
            raise ValueError(
                f"capacity must be in [1, {n_experts}], got {capacity}. A pool larger than the "
                f"expert count wastes memory; a pool of zero cannot serve any token.")
        self.layer, self.spec = int(layer), spec
        self.n_experts, self.capacity = int(n_experts), int(capacity)
        self.policy = make_policy(policy, capacity, n_experts)
        self.g2s = np.full(n_experts, -1, dtype=np.int32)
        self.s2g = np.full(capacity, -1, dtype=np.int32)
        self.admitted_at = np.zeros(capacity, dtype=np.int64)
        self._bpe = spec.bytes_per_expert
        self._fresh = self.capacity
        self._admissions = 0
        self.resident = 0               # experts in slots (counted: read per layer per token)
        self._table_stale = True
        self.miss_ranks = {}            # rank of each miss of the latest touch(), for admission
        self.uses = np.zeros(n_experts, dtype=np.int64)
        self.hits = self.misses = self.admits = self.evicts = 0
        self.admit_seconds = 0.0
        self.refill_bytes = 0
        self.last_evicted = -1          # the expert the latest claim_slot() evicted, -1 if none
        self.host_served = False        # set by HostServedPool: entries are then set one by one
        self._slots = slots
        self._device = device
        self.built = False

    # -- construction -------------------------------------------------------
    @property
    def bytes_per_expert(self) -> int:
        return self._bpe

    def build(self):
        """Allocate the C slots in HBM (ExpertPool.build, stream.py:570-597)."""
        if self._slots is None:
            self._slots = DeviceSlots(self.spec, self.capacity, self._device)
        self.built = True
        return self

    @property
    def device(self):
        return self._slots

    def nbytes(self) -> int:
        return self.capacity * self.bytes_per_expert


    # -- residency ----------------------------------------------------------
    def slot_of(self, e: int) -> int:
        return int(self.g2s[e])

    def touch(self, experts, ranks=None) -> list:
        """Count a request for each expert; tell the policy about the resident ones (in the
        given order) and return the others, the misses (stream.py:622-642)."""
        ex = [int(e) for e in experts]
        rk = [0] * len(ex) if ranks is None else [int(r) for r in ranks]
        table, uses, pol = self.g2s, self.uses, self.policy
        need, miss_ranks = [], {}
        for e, r in zip(ex, rk):
            uses[e] += 1
            if table[e] >= 0:
                pol.touch(e, r)
            else:
                need.append(e)
                miss_ranks[e] = r
        self.hits += len(ex) - len(need)
        self.misses += len(need)
        self.miss_ranks = miss_ranks
        return need

    def claim_slot(self, protect=()) -> int:
        """A slot for the next admission (stream.py:644-690): a never-used one while any is
        left, else the slot of an evicted expert."""
        self.last_evicted = -1
        if self._fresh:
            self._fresh -= 1
            return self._fresh
        keep = {int(x) for x in protect}
        pol = self.policy
        v = pol.victim(exclude=keep) if pol.excludes else pol.victim()
        ok = v is not None and 0 <= v < self.n_experts and v not in keep and self.g2s[v] >= 0
        if not ok:
            occupied = self.s2g >= 0
            if keep:
                occupied &= ~np.isin(self.s2g, np.fromiter(keep, dtype=np.int64))
            cand = np.flatnonzero(occupied)
            if cand.size == 0:
                raise RuntimeError(
                    f"layer {self.layer}: every one of {self.capacity} slots holds an expert this "
                    f"step still needs. Capacity must be at least top-k.")
            v = int(self.s2g[cand[np.argmin(self.admitted_at[cand])]])
        v = int(v)
        slot = int(self.g2s[v])
        pol.evicted(v)
        self.g2s[v] = -1
        self.s2g[slot] = -1
        self.resident -= 1
        self._table_stale = True
        self.evicts += 1
        self.last_evicted = v
        return slot

    def admit(self, e: int, blob, protect=()) -> int:
        """Write expert e's packed bytes into a slot and return the slot (stream.py:692-705,
        757-780). `blob` is a PinnedRegion or any bytes-like object."""
        if not self.built:
            raise RuntimeError("build() must run before admit()")
        want = self.bytes_per_expert
        if len(blob) != want:
            raise ValueError(
                f"layer {self.layer} expert {e}: the manifest accounts for {want} bytes but the "
                f"region supplied {len(blob)}. Refusing to write a partially-filled slot.")
        t0 = time.perf_counter()
        slot = self.claim_slot(protect)
        self.refill_bytes += self._slots.write(slot, blob)
        self.record_admission(e, slot, t0)
        return slot

    def admit_device(self, e: int, dev_ptr: int, protect=(), src_stream=None) -> int:
        """Admit from device memory (an expert staged on the GPU, stream.py:957-961), ordered
        after the work queued on `src_stream` (default: the current stream), which wrote it."""
        if not self.built:
            raise RuntimeError("build() must run before admit()")
        t0 = time.perf_counter()
        slot = self.claim_slot(protect)
        self._slots.write_device(slot, dev_ptr, self.bytes_per_expert, src_stream)
        self.record_admission(e, slot, t0)
        return slot

    def record_admission(self, e: int, slot: int, t0: float) -> None:
        """Tables, admission order and policy after expert e was placed in `slot`."""
        e, slot = int(e), int(slot)
        if self.s2g[slot] < 0:
            self.resident += 1
        self.g2s[e] = slot
        self.s2g[slot] = e
        self._table_stale = True
        self._admissions += 1
        self.admitted_at[slot] = self._admissions
        self.policy.admit(e, int(self.miss_ranks.get(e, 0)))
        self.admits += 1
        self.admit_seconds += time.perf_counter() - t0

    @property
    def full(self) -> bool:
        """Every expert resident, so no request can miss (stream.py:782-789)."""
        return self.capacity == self.n_experts and self.resident == self.n_experts

    def g2s_device(self, stream) -> None:
        """Upload the table when residency changed (stream.py:791-797); stream-ordered."""
        if self._table_stale and not self.host_served:
            self._slots.set_table(self.g2s, stream)
            self._table_stale = False

    def stats(self) -> dict:
        n = self.hits + self.misses
        return {"layer": self.layer, "capacity": self.capacity, "n_experts": self.n_experts,
                "hits": self.hits, "misses": self.misses, "miss_rate": self.misses / n if n else 0.0,
                "admits": self.admits, "evicts": self.evicts,
                "resident_bytes": self.resident * self.bytes_per_expert,
                "refill_bytes": self.refill_bytes, "admit_seconds": self.admit_seconds}

    def close(self) -> None:
        if self._slots is not None and hasattr(self._slots, "close"):
            self._slots.close()
        self.built = False
