"""Moving test layers onto the GPU through the product API."""
from __future__ import annotations

import numpy as np

from bigrig_amd.layer import MoELayer, StreamingSwitchGLU
from bigrig_amd.pool import ExpertPool, HostStore, PinnedFetcher


def to_dev_bits(a: np.ndarray, dev, bf16: bool = True):
    """uint16 bf16 bit patterns -> torch bfloat16 on dev (or uint8/float32/int32 as is)."""
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        t = torch.from_numpy(a.view(np.int16)).to(dev)
        return t.view(torch.bfloat16) if bf16 else t
    return torch.from_numpy(a).to(dev)


def bits(t) -> np.ndarray:
    """torch bfloat16 -> uint16 bit patterns on the host."""
    import torch
    return t.detach().view(torch.int16).cpu().numpy().view(np.uint16)


def bytes_dev(b: bytes, dev):
    import torch
    return torch.from_numpy(np.frombuffer(b, dtype=np.uint8).copy()).to(dev)


def build_gpu_layer(layer, dev, capacity: int | None = None, warm: bool = True, policy="lfuda"):
    """(MoELayer, StreamingSwitchGLU, ExpertPool, HostStore) for a tests.helpers.Layer."""
    spec = layer.spec
    E = spec.n_experts
    C = capacity or E
    store = HostStore()
    store.add_layer(0, layer.experts)
    pool = ExpertPool(0, spec, C, policy=policy).build()
    if warm and C == E:
        for e in range(E):        # as the reference's warm pass fills a whole layer
            pool.touch([e], [0])
            pool.admit(e, store.region(0, e))
    shared = bytes_dev(layer.shared, dev) if layer.shared is not None else None
    sw = StreamingSwitchGLU(pool, PinnedFetcher(store), shared=shared)
    sw.refresh()
    router = to_dev_bits(layer.router, dev)
    bias = None if layer.bias is None else to_dev_bits(layer.bias, dev)
    sgw = None if layer.sgate_w is None else to_dev_bits(layer.sgate_w, dev)
    moe = MoELayer(spec, router, sw, router_bias=bias, shared_gate_w=sgw)
    return moe, sw, pool, store


def tile_edge_tokens(idx: np.ndarray, n_experts: int, block: int = 64) -> list[int]:
    """Tokens to compare a prefill chunk on: for every expert the chunk hits, the tokens of the
    first and last row of each `block`-row run of its bucket (its pairs in pair order t * k + j,
    the stable order the bucketing keeps), and of the bucket's last row.

    The grouped GEMM cuts each bucket into M tiles that start at multiples of 64 rows, so with
    block = 64 every tile's first and last row, of every expert, is among the compared rows:
    a tile variant or an expert whose rows go wrong cannot hide between sampled tokens."""
    T, k = idx.shape
    flat = np.asarray(idx).reshape(-1)
    toks = set()
    for e in range(n_experts):
        p = np.flatnonzero(flat == e)
        n = len(p)
        if n == 0:
            continue
        rows = {n - 1}
        for r0 in range(0, n, block):
            rows.add(r0)
            rows.add(min(r0 + block - 1, n - 1))
        toks.update(int(p[r]) // k for r in rows)
    return sorted(toks)


def per_token_rel_l2(got: np.ndarray, want: np.ndarray) -> np.ndarray:
    """Relative L2 error of each row (token) of got against want."""
    g = np.asarray(got, np.float64)
    w = np.asarray(want, np.float64)
    num = np.sqrt(((g - w) ** 2).sum(-1))
    den = np.sqrt((w ** 2).sum(-1))
    return num / np.maximum(den, 1e-30)
