"""Eviction-policy replay over routing traces in native code (libbrx_replay.so).

The reference studies hit rates by replaying routing traces through its policies in Python
(bigrig_engine/pool.py:219-358). `misses` / `trace_misses` / `evaluate` here run the same
replay (simulate()'s contract; LRU, LFUDA, the rest of the reference's policy zoo -- windowed
LFU, S3-FIFO, ARC, LIRS, gaterank, coact -- and the Belady bound) in C++, every (capacity,
layer) cell of a sweep on its own thread, with results equal to `policy.simulate` /
`policy.belady` to the request. The library is host-only; it fails loudly when unbuilt.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libbrx_replay.so")
POLICY_IDS = {"lru": 0, "lfuda": 1, "belady": 2, "wlfu": 3, "windowed_lfu": 3, "s3fifo": 4,
              "arc": 5, "lirs": 6, "gaterank": 7, "coact": 8}


class LfudaParams(C.Structure):
    _fields_ = [("rank_weight", C.c_double), ("fcap", C.c_double), ("ghost_decay", C.c_double),
                ("keep_ghost", C.c_int32), ("reserved", C.c_int32)]


_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise RuntimeError(f"{LIB} is not built: run python -m bigrig_amd.build")
        lib = C.CDLL(LIB)
        i32p, i64p = C.POINTER(C.c_int32), C.POINTER(C.c_int64)
        lib.brx_replay_last_error.restype = C.c_char_p
        lib.brx_lfuda_defaults.argtypes = [C.POINTER(LfudaParams)]
        lib.brx_replay.argtypes = [C.c_int, i32p, i32p, C.c_int64, C.c_int, C.c_int,
                                   C.POINTER(LfudaParams), i64p]
        lib.brx_replay_trace.argtypes = [C.c_int, i32p, C.c_int, C.c_int, C.c_int, i32p, C.c_int,
                                         C.c_int, C.POINTER(LfudaParams), C.c_int, i64p]
        _lib = lib
    return _lib


def _check(rc: int) -> None:
    if rc != 0:
        raise ValueError(load().brx_replay_last_error().decode())


def lfuda_params(rank_weight: float = 0.0, fcap: float | None = 12.0, ghost_decay: float = 0.5,
                 keep_ghost: bool = True) -> LfudaParams:
    """The knobs of policy.LFUDA (fcap None = no cap)."""
    return LfudaParams(float(rank_weight), 0.0 if fcap is None else float(fcap),
                       float(ghost_decay), int(bool(keep_ghost)), 0)


def _pid(policy: str) -> int:
    if policy not in POLICY_IDS:
        raise ValueError(f"no native policy {policy!r}; have {', '.join(sorted(POLICY_IDS))}")
    return POLICY_IDS[policy]


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a), dtype=np.int32)


def misses(policy: str, seq, capacity: int, n_experts: int, ranks=None,
           lfuda: LfudaParams | None = None) -> int:
    """Misses of one request sequence (policy.simulate / policy.belady)."""
    s = _i32(seq)
    r = None if ranks is None else _i32(ranks)
    if r is not None and r.shape != s.shape:
        raise ValueError("ranks and seq differ in length")
    out = C.c_int64()
    i32p = C.POINTER(C.c_int32)
    _check(load().brx_replay(_pid(policy), s.ctypes.data_as(i32p),
                             None if r is None else r.ctypes.data_as(i32p), s.size,
                             int(capacity), int(n_experts),
                             None if lfuda is None else C.byref(lfuda), C.byref(out)))
    return int(out.value)


def trace_misses(policy: str, idx, capacities, n_experts: int | None = None,
                 lfuda: LfudaParams | None = None, threads: int = 0) -> np.ndarray:
    """Misses per (capacity, layer) of a routing trace idx [layers, tokens, k] replayed in
    router-rank order within each token (policy.layer_sequence): int64 [len(capacities), L]."""
    a = _i32(idx)
    if a.ndim != 3:
        raise ValueError("idx must be [layers, tokens, k]")
    L, T, k = a.shape
    E = int(a.max()) + 1 if n_experts is None else int(n_experts)
    caps = _i32(capacities).reshape(-1)
    out = np.zeros((caps.size, L), dtype=np.int64)
    i32p = C.POINTER(C.c_int32)
    _check(load().brx_replay_trace(_pid(policy), a.ctypes.data_as(i32p), L, T, k,
                                   caps.ctypes.data_as(i32p), caps.size, E,
                                   None if lfuda is None else C.byref(lfuda), int(threads),
                                   out.ctypes.data_as(C.POINTER(C.c_int64))))
    return out


def evaluate(policy: str, idx, capacities, layers=None, threads: int = 0) -> dict:
    """Mean miss rate over layers per capacity (policy.evaluate, pool.py:337-358)."""
    a = np.asarray(idx)
    if layers is not None:
        a = a[list(layers)]
    E = int(np.asarray(idx).max()) + 1
    m = trace_misses(policy, a, capacities, E, threads=threads)
    req = a.shape[1] * a.shape[2]
    return {int(c): float(m[i].mean() / req) for i, c in enumerate(_i32(capacities).reshape(-1))}
