"""The routed-expert operator and the MoE block around it, on libbrx.

`StreamingSwitchGLU` mirrors the reference operator of the same name
(bigrig_engine/stream.py:814-1631): `__call__(x, indices)` returns the UNREDUCED rows
`[..., k, H]` after making every requested expert resident, and the router's weights are applied
by the caller (stream.py:1523-1525). Its paths are the reference's:

* sync-free (every expert resident, `refresh()`): expert ids map to slots on the device, the
  host never reads the routing (stream.py:1377-1385, 1579-1603);
* one host read of the routing, `ensure()` admits the missing experts, one forward
  (stream.py:1447-1449, 1508);
* a chunk that routes to more experts than the pool holds: pairs sorted by expert (stable),
  cut into spans of at most C experts (`_pair_chunks`), each span made resident and computed,
  rows written straight back to their (token, k) positions (stream.py:1521-1561);
* host-served (`host_served=True`, no counterpart in the reference): a bounded pool whose
  misses the kernels read from pinned host memory, so it too stays on the sync-free path, its
  residency updated behind the forwards from routing copied back asynchronously
  (`hostserve.py`).

Whatever the path and the capacity, a row's arithmetic is the same kernel in the same order:
the kernel family is chosen by the call's token count only (decode for <= 8 tokens, the
grouped GEMM above), so outputs are bit-identical at every capacity (stream.py:25-30).

`MoELayer` is the block (mlx_lm's MoE block in the reference): router top-k, the operator,
the router-weighted combine, and an optional always-on shared expert with a sigmoid gate.
"""
from __future__ import annotations

import ctypes as C
import time

import numpy as np

from . import lib as L
from .pool import ExpertPool, step_requests
from .spec import LayerSpec

DECODE_MAX_TOKENS = 8
DECODE_MAX_PAIRS = 64


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _dptr(t) -> int | None:
    return None if t is None else t.data_ptr()


# ------------------------------------------------------------------ thin ops over the C-ABI
def router_topk(spec: LayerSpec, x, w_router, bias=None, shared_gate_w=None, stream=None):
    """(idx int32 [T,k], w fp32 [T,k], shared_gate fp32 [T] | None) on the device."""
    import torch
    x2 = x.reshape(-1, spec.hidden)
    T = x2.shape[0]
    dev = x2.device
    idx = torch.empty((T, spec.top_k), dtype=torch.int32, device=dev)
    w = torch.empty((T, spec.top_k), dtype=torch.float32, device=dev)
    sg = torch.empty(T, dtype=torch.float32, device=dev) if shared_gate_w is not None else None
    d = spec.desc()
    L.check(L.load().brx_router_topk(C.byref(d), _dptr(x2), _dptr(w_router), _dptr(bias),
                                     _dptr(shared_gate_w), T, _dptr(idx), _dptr(w), _dptr(sg),
                                     _stream(stream)))
    return idx, w, sg


def path_flag(n_tokens: int, top_k: int) -> int:
    """The kernel family for a call of n_tokens rows routed to top_k experts each: the decode
    GEMV for at most 8 tokens and 64 (token, expert) pairs, the grouped GEMM otherwise."""
    decode = n_tokens <= DECODE_MAX_TOKENS and n_tokens * top_k <= DECODE_MAX_PAIRS
    return L.FWD_FORCE_DECODE if decode else L.FWD_FORCE_PREFILL


def moe_forward(spec: LayerSpec, pool: ExpertPool, x2, idx, w=None, shared=None, sgate=None,
                out=None, y_unreduced=None, flags=None, stream=None):
    d = spec.desc()
    T = x2.shape[0]
    L.check(L.load().brx_moe_forward(
        C.byref(d), pool.device.handle, _dptr(x2), _dptr(idx), _dptr(w), _dptr(shared),
        _dptr(sgate), T, _dptr(out), _dptr(y_unreduced),
        path_flag(T, spec.top_k) if flags is None else flags, _stream(stream)))


def moe_block(spec: LayerSpec, pool: ExpertPool, x2, router_w, router_bias=None,
              shared_gate_w=None, shared=None, out=None, out_idx=None, out_w=None, flags=0,
              stream=None):
    """The whole MoE block over a fully resident pool: routing, experts, combine (+ shared).
    Returns out [T, H] bf16; out_idx / out_w, when given, receive the routing used."""
    import torch
    T = x2.shape[0]
    if out is None:
        out = torch.empty((T, spec.hidden), dtype=torch.bfloat16, device=x2.device)
    d = spec.desc()
    L.check(L.load().brx_moe_block_forward(
        C.byref(d), pool.device.handle, _dptr(x2), _dptr(router_w), _dptr(router_bias),
        _dptr(shared_gate_w), _dptr(shared), T, _dptr(out), _dptr(out_idx), _dptr(out_w), flags,
        _stream(stream)))
    return out


def forward_pairs(spec: LayerSpec, pool: ExpertPool, x2, pair_tok, pair_exp, pair_row, y_rows,
                  flags: int, shared=None, stream=None):
    d = spec.desc()
    L.check(L.load().brx_moe_forward_pairs(
        C.byref(d), pool.device.handle, _dptr(x2), x2.shape[0], _dptr(pair_tok), _dptr(pair_exp),
        _dptr(pair_row), pair_exp.numel(), y_rows.shape[0], _dptr(shared), _dptr(y_rows), flags,
        _stream(stream)))


def combine(spec: LayerSpec, y_routed, w, out, y_shared=None, sgate=None, stream=None):
    d = spec.desc()
    L.check(L.load().brx_combine(C.byref(d), _dptr(y_routed), _dptr(w), _dptr(y_shared),
                                 _dptr(sgate), w.shape[0], _dptr(out), _stream(stream)))


def dequant(spec: LayerSpec, expert_dev, proj: int, shared: bool = False, stream=None):
    import torch
    inter = spec.shared_inter if shared else spec.inter
    n_out, n_in = (inter, spec.hidden) if proj < 2 else (spec.hidden, inter)
    out = torch.empty((n_out, n_in), dtype=torch.float32, device=expert_dev.device)
    d = spec.desc()
    L.check(L.load().brx_dequant(C.byref(d), _dptr(expert_dev), proj, int(shared), _dptr(out),
                                 _stream(stream)))
    return out


def sort_pairs(spec: LayerSpec, idx, stream=None):
    import torch
    T = idx.shape[0]
    order = torch.empty(T * spec.top_k, dtype=torch.int32, device=idx.device)
    offsets = torch.empty(spec.n_experts + 1, dtype=torch.int32, device=idx.device)
    d = spec.desc()
    L.check(L.load().brx_sort_pairs(C.byref(d), _dptr(idx), T, _dptr(order), _dptr(offsets),
                                    _stream(stream)))
    return order, offsets


# ------------------------------------------------------------------ the operator
class StreamingSwitchGLU:
    """Drop-in semantics of the reference's StreamingSwitchGLU over an HBM ExpertPool."""

    def __init__(self, pool: ExpertPool, fetcher, shared=None, host_served: bool = False):
        """host_served: give the (fresh) pool host backing so misses are served by the kernels
        from the fetcher's pinned host store and residency is kept behind the forwards
        (`hostserve.HostServedPool`); the operator is then always on the sync-free path."""
        self._pool = pool
        self._fetcher = fetcher
        self.spec = pool.spec
        self.shared = shared             # device uint8 tensor of the shared expert, or None
        self.fetch_seconds = 0.0
        self.fetch_bytes = 0
        self.sync_seconds = 0.0
        self.chunked_calls = 0
        self._sync_free = False
        self._serve = None
        if host_served:
            store = getattr(fetcher, "store", None)
            if store is None:
                raise ValueError("host-served misses read the experts from a pinned host store: "
                                 "pass a PinnedFetcher")
            from .hostserve import HostServedPool
            self._serve = HostServedPool(pool, store)
            self._sync_free = True

    # -- residency (stream.py:922-978) -------------------------------------------------------
    def ensure(self, indices, ranks=None) -> np.ndarray:
        """Make every expert in `indices` resident and return `indices` mapped to slots.

        The pool sees the step as its distinct experts in ascending id, each at the best rank
        it was requested at (`step_requests`; ranks default to the top-k position), and admits
        the misses in that order with the whole step protected -- the order that fixes slot
        numbers (stream.py:922-978). A step that needs more experts than the pool holds, or names
        an expert the layer does not have, is refused before anything is written."""
        gi = np.asarray(indices, dtype=np.int64)
        pool = self._pool
        experts, best = step_requests(gi, ranks)
        bad = [e for e in experts if not 0 <= e < pool.n_experts]
        if bad:
            raise KeyError(bad[0])
        need = pool.touch(experts, best)
        if len(need) > pool.capacity:
            raise RuntimeError(
                f"layer {pool.layer} needs {len(need)} experts for one step but the "
                f"pool holds {pool.capacity}. Capacity must be at least top-k; below "
                f"that a token evicts an expert it is still using.")
        if need:
            t0 = time.perf_counter()
            got = self._fetcher.fetch([(pool.layer, e) for e in need])
            self.fetch_seconds += time.perf_counter() - t0
            for e in need:
                region = got[(pool.layer, e)]
                self.fetch_bytes += len(region)
                pool.admit(e, region, protect=experts)
        return pool.g2s[gi]

    def refresh(self) -> bool:
        """Take the sync-free path iff every expert is resident (stream.py:1579-1603), or the
        pool serves its misses from host memory."""
        self._sync_free = self._pool.full or self._serve is not None
        return self._sync_free

    def _before(self, stream=None) -> None:
        """Ahead of a sync-free forward: the table as residency left it (uploaded if it changed),
        or, host-served, the admissions decided from the routing that has come back since."""
        if self._serve is not None:
            self._serve.service(stream)
        else:
            self._pool.g2s_device(_stream(stream))

    def _after(self, idx, stream=None) -> None:
        if self._serve is not None:
            self._serve.record(idx, stream)

    @staticmethod
    def _pair_chunks(sorted_experts: np.ndarray, C: int):
        """Cut pairs already sorted by expert into spans of at most C distinct experts
        (stream.py:1098-1126): span i runs from the (iC)-th distinct expert to the ((i+1)C)-th."""
        uniq, starts = np.unique(sorted_experts, return_index=True)
        n = int(sorted_experts.shape[0])
        return [(int(starts[i]), int(starts[i + C]) if i + C < len(uniq) else n)
                for i in range(0, len(uniq), C)]

    def _host_routing(self, indices) -> np.ndarray:
        """The one device->host read of the routing a streamed layer pays (stream.py:1440-1450)."""
        t0 = time.perf_counter()
        gi = indices.to("cpu").numpy().astype(np.int64)
        self.sync_seconds += time.perf_counter() - t0
        return gi

    def _spans(self, x2, flat: np.ndarray, y_rows, flags: int, stream=None) -> None:
        """Expert-sorted spans (stream.py:1521-1561), each written to its unsorted rows."""
        import torch
        k = flat.shape[1]
        pe = flat.reshape(-1)
        order = np.argsort(pe, kind="stable")
        spe = pe[order]
        tok = order // k
        rank = order % k
        dev = x2.device
        for lo, hi in self._pair_chunks(spe, self._pool.capacity):
            self.ensure(spe[lo:hi], ranks=rank[lo:hi])
            self._pool.g2s_device(_stream(stream))
            t_tok = torch.from_numpy(tok[lo:hi].astype(np.int32)).to(dev)
            t_exp = torch.from_numpy(spe[lo:hi].astype(np.int32)).to(dev)
            t_row = torch.from_numpy(order[lo:hi].astype(np.int32)).to(dev)
            forward_pairs(self.spec, self._pool, x2, t_tok, t_exp, t_row, y_rows, flags,
                          stream=stream)

    def __call__(self, x, indices, stream=None):
        """Unreduced expert rows [..., k, H] (bf16) for `indices` [..., k]."""
        import torch
        H, k = self.spec.hidden, self.spec.top_k
        x2 = x.reshape(-1, H).contiguous()
        T = x2.shape[0]
        flags = path_flag(T, k)
        idx = indices.reshape(-1, k).to(torch.int32).contiguous()
        y = torch.empty((T, k, H), dtype=torch.bfloat16, device=x2.device)
        if self._sync_free:
            self._before(stream)
            moe_forward(self.spec, self._pool, x2, idx, y_unreduced=y, flags=flags, stream=stream)
            self._after(idx, stream)
            return y.reshape(*indices.shape[:-1], k, H)
        gi = self._host_routing(idx)
        if k > self._pool.capacity:
            raise ValueError(
                f"layer {self._pool.layer}: top-k is {k} but the pool holds "
                f"{self._pool.capacity}. A single token cannot be served.")
        if len(np.unique(gi)) <= self._pool.capacity:
            self.ensure(gi)
            self._pool.g2s_device(_stream(stream))
            moe_forward(self.spec, self._pool, x2, idx, y_unreduced=y, flags=flags, stream=stream)
        else:
            self.chunked_calls += 1
            self._spans(x2, gi, y.view(T * k, H), flags, stream)
        return y.reshape(*indices.shape[:-1], k, H)

    def forward_combined(self, x2, idx, w, sgate=None, stream=None):
        """out [T, H] = sum_j w[t,j] * y[t,j] (+ sgate[t] * shared(x_t)), the block's combine
        fused into the expert kernels whenever no span split is needed."""
        import torch
        H, k = self.spec.hidden, self.spec.top_k
        T = x2.shape[0]
        flags = path_flag(T, k)
        out = torch.empty((T, H), dtype=torch.bfloat16, device=x2.device)
        shared = self.shared
        if self._sync_free:
            self._before(stream)
            moe_forward(self.spec, self._pool, x2, idx, w, shared, sgate, out=out, flags=flags,
                        stream=stream)
            self._after(idx, stream)
            return out
        gi = self._host_routing(idx)
        if k > self._pool.capacity:
            raise ValueError(
                f"layer {self._pool.layer}: top-k is {k} but the pool holds "
                f"{self._pool.capacity}. A single token cannot be served.")
        if len(np.unique(gi)) <= self._pool.capacity:
            self.ensure(gi)
            self._pool.g2s_device(_stream(stream))
            moe_forward(self.spec, self._pool, x2, idx, w, shared, sgate, out=out, flags=flags,
                        stream=stream)
            return out
        self.chunked_calls += 1
        y = torch.empty((T * k, H), dtype=torch.bfloat16, device=x2.device)
        self._spans(x2, gi, y, flags, stream)
        ysh = None
        if shared is not None:
            ysh = torch.empty((T, H), dtype=torch.bfloat16, device=x2.device)
            tt = torch.arange(T, dtype=torch.int32, device=x2.device)
            te = torch.full((T,), self.spec.n_experts, dtype=torch.int32, device=x2.device)
            forward_pairs(self.spec, self._pool, x2, tt, te, None, ysh, flags, shared=shared,
                          stream=stream)
        combine(self.spec, y, w, out, ysh, sgate, stream=stream)
        return out


class MoELayer:
    """Router top-k + routed experts + combine (+ shared expert), the block the reference's
    operator is installed in (stream.py:1884-1889)."""

    def __init__(self, spec: LayerSpec, router_w, switch: StreamingSwitchGLU, router_bias=None,
                 shared_gate_w=None):
        self.spec = spec
        self.router_w = router_w
        self.router_bias = router_bias
        self.switch = switch
        self.shared_gate_w = shared_gate_w

    def route(self, x2, stream=None):
        return router_topk(self.spec, x2, self.router_w, self.router_bias,
                           self.shared_gate_w if self.switch.shared is not None else None, stream)

    def __call__(self, x, stream=None):
        x2 = x.reshape(-1, self.spec.hidden).contiguous()
        sw = self.switch
        if sw._sync_free:
            # every expert resident (or served from host memory): routing, experts and combine
            # in one library call, the routing never waited for by the host (stream.py:1377-1394)
            sw._before(stream)
            sgw = self.shared_gate_w if sw.shared is not None else None
            idx = None
            if sw._serve is not None:
                import torch
                idx = torch.empty((x2.shape[0], self.spec.top_k), dtype=torch.int32,
                                  device=x2.device)
            out = moe_block(self.spec, sw._pool, x2, self.router_w, self.router_bias, sgw,
                            sw.shared, out_idx=idx, flags=path_flag(x2.shape[0], self.spec.top_k), stream=stream)
            if idx is not None:
                sw._after(idx, stream)
            return out.reshape(x.shape)
        idx, w, sg = self.route(x2, stream)
        out = sw.forward_combined(x2, idx, w, sg, stream)
        return out.reshape(x.shape)
