"""Layer-major prefill with the next layer's experts streamed in while this layer computes.

The reference runs every chunk of a long prompt through layer L before layer L+1
(bigrig_engine/layered.py:85-131), so a layer's experts are read once for the whole prompt
rather than once per chunk, and while layer L computes it reads layer L+1's experts ahead
(StreamHandle.prefill_layer / read_ahead, stream.py:1201-1216, 2009-2034): the reads the chunks
would issue anyway, moved earlier, so the next layer starts with its experts in place.

Here a layer's experts live in pinned host memory (`HostStore`) and a prompt long enough to
route to nearly every expert needs all of them, so the device side is a ring of whole layers:
`depth` slot sets of E slots each in HBM (`LayerRing`). Layer L runs on set L % depth with every
expert resident (the sync-free whole-block path, no host routing read); layer L+1's experts are
copied over PCIe into set (L+1) % depth on the ring's copy stream meanwhile. The library orders
each copy after the last forward that read its set and each forward after the copies into its
set (brx_pool_refill_async / brx_moe_block_forward events), so the host only issues work.
The result of every row is the one a token-major pass gives: the same kernels, per-row
arithmetic independent of the chunk order.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .pool import DeviceSlots, HostStore
from .spec import LayerSpec


@dataclass
class MoEWeights:
    """One MoE block's non-expert weights (device tensors) and where its experts are in the
    host store: router [E, H], optional logit bias [E], optional shared expert and its gate."""
    layer: int
    router: object
    router_bias: object = None
    shared: object = None
    shared_gate_w: object = None


class _SlotSet:
    """A full-residency slot set seen as a pool by the thin ops (they read `.device.handle`)."""

    def __init__(self, slots: DeviceSlots):
        self.device = slots
        self.layer = None


class LayerRing:
    """`depth` sets of E device slots (expert e in slot e), reused round-robin by consecutive
    layers, refilled on one copy stream."""

    def __init__(self, spec: LayerSpec, depth: int = 2, device: int = 0):
        import torch
        if depth < 2:
            raise ValueError("a ring needs two sets for the next layer to load while one computes")
        self.spec = spec
        self.copy_stream = torch.cuda.Stream(device)
        self.sets = [_SlotSet(DeviceSlots(spec, spec.n_experts, device, self.copy_stream))
                     for _ in range(depth)]
        ident = np.arange(spec.n_experts, dtype=np.int32)
        for s in self.sets:
            s.device.set_table(ident, torch.cuda.current_stream(device).cuda_stream)
        torch.cuda.current_stream(device).synchronize()
        self.bytes_loaded = 0

    def set_for(self, i: int) -> _SlotSet:
        return self.sets[i % len(self.sets)]

    def load(self, i: int, store: HostStore, layer: int) -> _SlotSet:
        """Queue the copies of every expert of `layer` into set i % depth (returns at once)."""
        s = self.set_for(i)
        E = self.spec.n_experts
        if store.tensor(layer).shape[0] != E:
            raise ValueError(f"layer {layer} has {store.tensor(layer).shape[0]} experts in the "
                             f"store, the ring holds {E}")
        t = store.tensor(layer)
        per = int(t.shape[1])
        # expert e into slot e: the whole layer in one transfer
        self.bytes_loaded += s.device.write_range(0, t.data_ptr(), E, per, per)
        s.layer = layer
        return s

    def reset(self) -> None:
        """Forget which layer each set holds (the next prefill copies every layer again)."""
        for s in self.sets:
            s.layer = None

    def close(self) -> None:
        for s in self.sets:
            s.device.close()


def prefill(spec: LayerSpec, layers: list, store: HostStore, chunks: list, ring: LayerRing,
            residual: bool = True, read_ahead: bool = True, progress=None) -> list:
    """Run the hidden states `chunks` ([T_j, H] bf16 device tensors, the prompt's chunks in
    order) through the MoE blocks `layers` (MoEWeights, in model order), layer by layer.

    With `residual`, a block's output is added to its input (h <- h + moe(h)); otherwise it
    replaces it. With `read_ahead` (default), layer i + 1's experts are queued for copying
    before layer i's chunks, so the copy overlaps their compute; without it, a layer's copy
    starts only once the previous layer's compute has finished (the serial schedule, for
    comparison). `progress(done, total)` is called after each layer. Returns the chunks after
    the last block (new tensors)."""
    import torch

    from . import layer as ops
    if not layers:
        return list(chunks)
    h = list(chunks)
    n = len(layers)
    for i, lw in enumerate(layers):
        s = ring.set_for(i)
        if s.layer != lw.layer:
            if not read_ahead:
                ring.copy_stream.wait_stream(torch.cuda.current_stream())
            ring.load(i, store, lw.layer)
        if read_ahead and i + 1 < n and ring.set_for(i + 1).layer != layers[i + 1].layer:
            ring.load(i + 1, store, layers[i + 1].layer)
        for j, x in enumerate(h):
            out = ops.moe_block(spec, s, x, lw.router, lw.router_bias, lw.shared_gate_w, lw.shared,
                                flags=ops.path_flag(x.shape[0], spec.top_k))
            h[j] = out + x if residual else out
        if progress is not None:
            progress(i + 1, n)
    return h
