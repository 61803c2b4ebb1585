"""Bounded pools whose misses are detected and served on the device, from pinned host memory.

The reference keeps a layer whose pool can miss off its sync-free path: it reads the routing
back to the host (`np.array(indices)`, stream.py:1440-1450) to find the misses and admit them
before the layer computes, a read that drains the queue every layer (2.23 ms a layer, 73% of a
token: autoconfig.py:61-66, stream.py:1583-1590). Its remedy is to hold some layers whole so
they never need it (`plan_full_layers`, autoconfig.py:52-109; restated in `plan_full_layers`
below).

A GPU here can read pinned host memory directly. Given host backing
(`brx_pool_set_host_backing`), a pool's table entry of -1 makes the kernels read that expert
from the layer's pinned host store instead of a slot: the miss is found and served on the
device, so a bounded layer takes the sync-free path too. Residency is kept behind the
forwards: each step's routing is copied back asynchronously into pinned buffers, and when a
copy has landed the host runs the pool's own bookkeeping over it (touch, victim, admit with
its policy; `ExpertPool`, stream.py:622-780), retiring each victim's entry on the compute stream
(`brx_pool_publish_async`) and copying the admitted expert into its slot on the copy stream,
which then sets the entry (`brx_pool_admit_async`). Every forward reads each expert from a slot
or from the host store -- the same bytes -- so its outputs equal the fully resident layer's bit
for bit, whatever residency is at the time.

Two rules keep the table consistent with the slots: a victim's entry is retired in stream order
before any later forward, and its slot is rewritten only after every forward already issued
(the library's write-after-read wait); an expert whose admission copy has not finished is never
chosen as a victim (its table write on the copy stream could otherwise land after the retirement).
"""
from __future__ import annotations

import ctypes as C
import time

import numpy as np

from . import lib as L
from .pool import ExpertPool, HostStore, step_requests


def plan_full_layers(n_layers: int, n_experts: int, top_k: int, capacity: int,
                     floor_over_topk: int = 1) -> tuple:
    """(layers to hold whole, capacity of the others) spending no more slots than `capacity`
    in every layer would (autoconfig.py:52-109).

    Whole layers take n_experts slots each; the rest share what is left, each at least
    top_k + floor_over_topk slots. As many layers as possible are held whole (at most
    n_layers - 1), the rest get the largest equal capacity that fits. (0, capacity) when the pool
    is already whole, the floor cannot be met, or nothing can be held whole."""
    n_layers, n_experts = int(n_layers), int(n_experts)
    top_k, capacity = int(top_k), int(capacity)
    floor = max(1, top_k + int(floor_over_topk))
    budget = capacity * n_layers
    if capacity >= n_experts or n_layers < 2 or floor >= n_experts or budget < floor * n_layers:
        return 0, capacity
    # the most whole layers with every other layer at the floor
    whole = min(n_layers - 1, (budget - floor * n_layers) // (n_experts - floor))
    while whole > 0:
        rest = min(n_experts, (budget - whole * n_experts) // (n_layers - whole))
        if rest >= floor and whole * n_experts + rest * (n_layers - whole) <= budget:
            return whole, rest
        whole -= 1
    return 0, capacity


class HostServedPool:
    """Host backing and behind-the-forwards residency for one layer's `ExpertPool`."""

    def __init__(self, pool: ExpertPool, store: HostStore, copy_stream=None, depth: int = 16):
        import torch
        if not pool.built:
            raise RuntimeError("build() the pool before giving it host backing")
        if pool.admits or pool.resident:
            raise RuntimeError("host backing is given to a fresh pool, before any admission")
        t = store.tensor(pool.layer)
        E, per = pool.n_experts, pool.bytes_per_expert
        if tuple(t.shape) != (E, per):
            raise ValueError(f"layer {pool.layer}: the host store holds {tuple(t.shape)}, the pool "
                             f"needs ({E}, {per})")
        if per % 256:
            raise ValueError(f"layer {pool.layer}: {per} bytes per expert is not a multiple of 256, "
                             f"the alignment the kernels read an expert with")
        self.pool, self.store = pool, store
        self._t = t
        L.check(L.load().brx_pool_set_host_backing(pool.device.handle, t.data_ptr(), per,
                                                   t.numel()))
        pool.host_served = True            # its whole-table uploads are off: entries are set here
        self.copy_stream = copy_stream if copy_stream is not None else pool.device.copy_stream
        self.depth = int(depth)
        self._ring = []                    # [(pinned int32 buffer, n, k, event)] in issue order
        self._spare = []
        self._pending = {}                 # expert -> event after its admission copy
        self.steps = 0
        self.admit_bytes = 0
        self.service_seconds = 0.0
        self._torch = torch

    # -- routing back to the host, asynchronously -------------------------------------------
    def record(self, idx, stream=None) -> None:
        """Queue the copy of one step's routing `idx` [T, k] (device int32) into pinned memory,
        after the forward that produced it on `stream`. Keeps at most `depth` copies
        unprocessed (the oldest is then waited for)."""
        torch = self._torch
        n, k = idx.numel(), idx.shape[-1]
        buf = None
        for i, b in enumerate(self._spare):
            if b.numel() >= n:
                buf = self._spare.pop(i)
                break
        if buf is None:
            buf = torch.empty(max(n, 64), dtype=torch.int32, pin_memory=True)
        s = stream if stream is not None else torch.cuda.current_stream()
        with torch.cuda.stream(s):
            buf[:n].copy_(idx.reshape(-1), non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(s)
        self._ring.append((buf, n, k, ev))
        self.steps += 1
        while len(self._ring) > self.depth:
            self._process(self._ring.pop(0), stream, wait=True)

    def service(self, stream=None) -> int:
        """Run the bookkeeping over every routing copy that has landed (in issue order) and
        queue the admissions it decides. Returns the steps processed. Never waits."""
        done = 0
        while self._ring and self._ring[0][3].query():
            self._process(self._ring.pop(0), stream)
            done += 1
        return done

    def drain(self, stream=None) -> int:
        """Process every recorded step, waiting for the copies still in flight."""
        done = 0
        while self._ring:
            self._process(self._ring.pop(0), stream, wait=True)
            done += 1
        return done

    def _process(self, entry, stream, wait: bool = False) -> None:
        buf, n, k, ev = entry
        if wait:
            ev.synchronize()
        gi = buf[:n].numpy().astype(np.int64).reshape(-1, k)
        self._spare.append(buf)
        t0 = time.perf_counter()
        self._admit_step(gi, stream)
        self.service_seconds += time.perf_counter() - t0

    # -- residency ------------------------------------------------------------------------
    def _admit_step(self, gi: np.ndarray, stream) -> None:
        """ensure() of one step without the wait: touch in ascending id with the best rank
        (stream.py:933-950), then admit the misses in ascending id while a slot can be freed
        outside the step's experts and the admissions still in flight (stream.py:957-969)."""
        torch = self._torch
        pool = self.pool
        uniq, ranks = step_requests(gi)
        keep = [i for i, e in enumerate(uniq) if 0 <= e < pool.n_experts]
        uniq, ranks = [uniq[i] for i in keep], [ranks[i] for i in keep]
        need = pool.touch(uniq, ranks)
        if not need:
            return
        for e, ev in list(self._pending.items()):
            if ev.query():
                del self._pending[e]
        protect = set(uniq) | set(self._pending)
        s = stream if stream is not None else torch.cuda.current_stream()
        lib = L.load()
        handle = pool.device.handle
        for e in need:
            t0 = time.perf_counter()
            try:
                slot = pool.claim_slot(protect)
            except RuntimeError:
                break                      # every slot holds a protected expert: serve from host
            v = pool.last_evicted
            if v >= 0:
                ve, vs = (C.c_int32 * 1)(v), (C.c_int32 * 1)(-1)
                L.check(lib.brx_pool_publish_async(handle, 1, ve, vs, s.cuda_stream))
            region = self.store.region(pool.layer, e)
            L.check(lib.brx_pool_admit_async(handle, e, slot, region.ptr, region.nbytes,
                                             self.copy_stream.cuda_stream))
            done = torch.cuda.Event()
            done.record(self.copy_stream)
            self._pending[e] = done
            protect.add(e)
            pool.record_admission(e, slot, t0)
            pool.refill_bytes += region.nbytes
            self.admit_bytes += region.nbytes

    def stats(self) -> dict:
        st = self.pool.stats()
        st.update({"steps": self.steps, "admit_bytes": self.admit_bytes,
                   "service_seconds": self.service_seconds,
                   "in_flight": len(self._ring), "admissions_pending": len(self._pending)})
        return st
