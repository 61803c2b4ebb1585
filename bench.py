#!/usr/bin/env python3
"""MoE-layer throughput on one MI355X: batch-1 decode and 2048-token prefill, with roofline.

Workload (synthetic, seeded; random-init weights of the named architecture):
  a Qwen3-30B-A3B-shaped routed-expert stack, 48 MoE layers: hidden 2048, 128 experts, softmax
  top-8 renormalised, expert intermediate 768, SwiGLU, MLX affine 4-bit g64 bf16 scale/bias.
  Expert weights N(0, 0.02) per (layer, expert, projection), quantized on the GPU; router
  weights N(0, 0.02) bf16 plus a per-layer Zipf(s=1.1) logit bias; layer inputs N(0, 1) bf16.

One step = one decode token through all 48 layers, each layer one brx_moe_block_forward call
(router logits; gate/up + SwiGLU with the top-k ranked inside the kernel; down + router-weighted
combine), every expert resident in HBM (the pool's sync-free path), the step replayed as a HIP
graph. `value` = decode tokens/s of the stack.

Also reported on the same line:
  roofline      the dominant kernel (decode gate/up) timed with HIP events on its stream:
                algorithmic bytes per launch / average launch duration vs 8 TB/s
  prefill       one 2048-token chunk through the 48 layers (bucketing + grouped MFMA GEMMs),
                tokens/s and the gate/up GEMM's TFLOP/s vs 2.5 PFLOP/s dense bf16
  bounded_pool  the same decode with 32 of 128 experts per layer resident, misses refilled
                from pinned host memory over PCIe, one routing read-back per layer (end to end);
                `host_served`: the kernels read misses from pinned host memory and residency
                follows behind the forwards (no read-back wait); `host_served_plan`: the same
                with the whole-layer plan for that memory (some layers whole, the rest smaller)
  layer_major_prefill  a 32768-token prompt through 8 layers layer by layer, each layer's
                experts streamed from pinned host memory into a two-layer HBM ring while the
                previous layer computes (PCIe-inclusive)
  policy_replay the eviction-policy trace replay (host C++, libbrx_replay.so) against the
                Python restatement, requests/s on the shipped Qwen3 routing trace
  cpu_baseline  the fp32 dequant-on-the-fly CPU layer (oracle/cpu_baseline.c, OpenMP) on
                the host cores, on a bounded sample
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE-layer tokens/s at batch 1 and 2048-token prefill; % of HBM/MFMA roofline"
HBM_PEAK_GBS = 8000.0
# the decode kernel the roofline line times: one token, affine 4-bit, routing ranked in-kernel
# for E <= 128 (k_dec_gateup1<MODE, UPL, KP>)
DECODE_GATEUP_KERNEL = "k_dec_gateup1<0, 1, 2>"
BF16_PEAK_TFLOPS = 2500.0


def _r(v, n):
    return None if v is None else round(v, n)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200, help="timed decode steps")
    ap.add_argument("--warmup", type=int, default=20, help="untimed decode steps")
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--prefill-tokens", type=int, default=2048)
    ap.add_argument("--prefill-steps", type=int, default=5)
    ap.add_argument("--pool-capacity", type=int, default=32)
    ap.add_argument("--pool-tokens", type=int, default=64)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--skip", default="", help="comma list of: prefill,pool,layered,replay,cpu,graph,report,widths")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB (--steps times): the "
                         "known-size reference for scaling HBM byte counters")
    return ap.parse_args()


def copy_probe(args) -> None:
    import torch
    n = args.copy_mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    print(json.dumps({"copy_bytes": n, "read_bytes": n, "write_bytes": n, "steps": args.steps,
                      "gbs": round(2 * n / dt / 1e9, 1)}), flush=True)


class Stack:
    """A stack of layers on the GPU: fully resident pools, router weights, the router's Zipf
    bias (None for the configurations that route on plain logits) and input banks."""

    def __init__(self, spec, layers: int, bank: int, keep_host_layers: int = 0,
                 zipf: float | None = 1.1):
        import torch

        from bigrig_amd import synth
        from bigrig_amd.pool import ExpertPool, HostStore
        self.spec = spec
        self.layers = layers
        self.pools, self.routers, self.biases, self.xbank = [], [], [], []
        self.shared, self.shared_gate = [], []   # per layer, when the spec has a shared expert
        self.host = HostStore()
        t0 = time.time()
        for l in range(layers):
            experts = synth.make_layer_experts(spec, seed=1000 + l)
            pool = ExpertPool(l, spec, spec.n_experts).build()
            for e in range(spec.n_experts):
                pool.touch([e], [0])
                pool.admit_device(e, experts[e].data_ptr())
            pool.device.sync()
            if l < keep_host_layers:
                h = torch.empty(experts.shape, dtype=torch.uint8, pin_memory=True)
                h.copy_(experts)
                self.host.add_layer_tensor(l, h)
            del experts
            self.pools.append(pool)
            self.routers.append(synth.router_weights(spec, seed=2000 + l))
            self.biases.append(synth.zipf_bias_torch(spec.n_experts, zipf, seed=3000 + l)
                               if zipf else None)
            self.xbank.append(synth.activations(bank, spec.hidden, seed=4000 + l))
            if spec.shared_inter:
                self.shared.append(synth.make_layer_experts(spec, seed=5000 + l, shared=True)[0].contiguous())
                g = torch.Generator(device="cuda")
                g.manual_seed(5500 + l)
                self.shared_gate.append((torch.randn(spec.hidden, generator=g, device="cuda") * 0.02)
                                        .to(torch.bfloat16))
        torch.cuda.synchronize()
        for p in self.pools:
            p.g2s_device(torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        log(f"built {layers} layers x {spec.n_experts} experts "
            f"({layers * spec.n_experts * spec.bytes_per_expert / 1e9:.1f} GB) in {time.time() - t0:.1f}s")


def decode_bench(args, st: "Stack"):
    """48-layer decode step of one token, each layer one brx_moe_block_forward call (router
    logits, gate/up with the top-k ranked in-kernel, down + combine), replayed as a HIP graph.
    Per-kernel times come from graphs of the block's split steps (PHASE_R, +PHASE_A, +PHASE_B)
    timed with HIP events on the stream the kernels run on."""
    import ctypes as C

    import torch

    from bigrig_amd import lib as L
    spec, Ln = st.spec, st.layers
    G = st.xbank[0].shape[0]
    dev = st.xbank[0].device
    k, H = spec.top_k, spec.hidden
    outs = [torch.empty((1, H), dtype=torch.bfloat16, device=dev) for _ in range(Ln)]
    lib = L.load()
    d = spec.desc()
    dref = C.byref(d)

    def step(g: int, stream: int, phases: int = 0):
        for l in range(Ln):
            x = st.xbank[l][g:g + 1]
            L.check(lib.brx_moe_block_forward(dref, st.pools[l].device.handle, x.data_ptr(),
                                              st.routers[l].data_ptr(), st.biases[l].data_ptr(),
                                              None, None, 1, outs[l].data_ptr(), None, None,
                                              L.FWD_FORCE_DECODE | phases, stream))

    s = torch.cuda.current_stream()
    sp = s.cuda_stream
    for g in range(G):
        step(g, sp)
    torch.cuda.synchronize()

    def capture(g, phases=0):
        cg = torch.cuda.CUDAGraph()
        with torch.cuda.graph(cg):
            step(g, torch.cuda.current_stream().cuda_stream, phases)
        return cg

    use_graph = "graph" not in args.skip
    graphs = []
    if use_graph:
        try:
            graphs = [capture(g) for g in range(G)]
            torch.cuda.synchronize()
        except Exception as ex:   # capture unsupported: time eager launches
            log(f"graph capture failed ({ex}); timing eager launches")
            graphs = []
            torch.cuda.synchronize()

    def run(i):
        if graphs:
            graphs[i % G].replay()
        else:
            step(i % G, sp)

    for i in range(args.warmup):
        run(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        run(i)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    tok_s = args.steps / dt
    t1 = time.perf_counter()
    ne = max(10, args.steps // 5)
    for i in range(ne):
        step(i % G, sp)
    torch.cuda.synchronize()
    eager_tok_s = ne / (time.perf_counter() - t1)

    # per-kernel times: graphs of the split steps over all layers, events on the same stream
    per = {}
    if graphs:
        ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
        reps = 10
        for name, ph in (("r", L.FWD_PHASE_R), ("ra", L.FWD_PHASE_R | L.FWD_PHASE_A),
                         ("rab", L.FWD_PHASE_R | L.FWD_PHASE_A | L.FWD_PHASE_B)):
            gs = [capture(g, ph) for g in range(G)]
            for g in gs:
                g.replay()
            torch.cuda.synchronize()
            e0, e1 = ev(), ev()
            e0.record(s)
            for r in range(reps):
                for g in gs:
                    g.replay()
            e1.record(s)
            torch.cuda.synchronize()
            per[name] = e0.elapsed_time(e1) / (reps * G * Ln) * 1e3   # us per layer
            del gs
    router_us = per.get("r")
    gateup_us = per["ra"] - per["r"] if per else None
    down_us = per["rab"] - per["ra"] if per else None
    spec_e = spec.expert_spec()
    gu = sum(c["nbytes"] for p in ("gate_proj", "up_proj") for c in spec_e[p].values())
    dn = sum(c["nbytes"] for c in spec_e["down_proj"].values())
    E = spec.n_experts
    # per launch: the selected experts' packed bytes + x, logits, slot table and h written
    # (gate/up); + h read, out written and the routing weights (down)
    gu_bytes = k * gu + 2 * H + 4 * (E + 1) + 4 * E + 2 * k * spec.inter
    dn_bytes = k * dn + 2 * k * spec.inter + 2 * H + 4 * k
    layer_bytes = k * spec.bytes_per_expert + spec.router_bytes + 2 * H * 2
    return {
        "tok_s": tok_s, "ms_per_step": dt / args.steps * 1e3, "graph": bool(graphs),
        "eager_tok_s": eager_tok_s, "router_us": router_us,
        "gateup_us": gateup_us, "down_us": down_us,
        "gateup_bytes": gu_bytes, "down_bytes": dn_bytes, "layer_bytes": layer_bytes,
        "gateup_gbs": gu_bytes / (gateup_us * 1e-6) / 1e9 if gateup_us else None,
        "down_gbs": dn_bytes / (down_us * 1e-6) / 1e9 if down_us else None,
        "step_gbs": layer_bytes * Ln * tok_s / 1e9,
    }


def prefill_bench(args, st: "Stack"):
    import ctypes as C

    import torch

    from bigrig_amd import lib as L
    from bigrig_amd import synth
    spec, Ln = st.spec, st.layers
    T, k, H = args.prefill_tokens, spec.top_k, spec.hidden
    dev = st.xbank[0].device
    xs = [synth.activations(T, H, seed=5000 + l) for l in range(Ln)]
    idx = [torch.empty((T, k), dtype=torch.int32, device=dev) for _ in range(Ln)]
    wts = [torch.empty((T, k), dtype=torch.float32, device=dev) for _ in range(Ln)]
    out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    lib = L.load()
    d = spec.desc()
    dref = C.byref(d)
    s = torch.cuda.current_stream()
    sp = s.cuda_stream

    def route(l):
        L.check(lib.brx_router_topk(dref, xs[l].data_ptr(), st.routers[l].data_ptr(),
                                    st.biases[l].data_ptr(), None, T, idx[l].data_ptr(),
                                    wts[l].data_ptr(), None, sp))

    def fwd(l, phases=0):
        L.check(lib.brx_moe_forward(dref, st.pools[l].device.handle, xs[l].data_ptr(),
                                    idx[l].data_ptr(), wts[l].data_ptr(), None, None, T,
                                    out.data_ptr(), None, L.FWD_FORCE_PREFILL | phases, sp))

    def chunk():
        for l in range(Ln):
            route(l)
            fwd(l)

    chunk()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.prefill_steps):
        chunk()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.prefill_steps
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    e0, e1, e2, e3 = ev(), ev(), ev(), ev()
    e0.record(s)
    for l in range(Ln):
        route(l)
    e1.record(s)
    for l in range(Ln):
        fwd(l, L.FWD_PHASE_A)
    e2.record(s)
    for l in range(Ln):
        fwd(l, L.FWD_PHASE_A)
        fwd(l, L.FWD_PHASE_B)
    e3.record(s)
    torch.cuda.synchronize()
    router_ms = e0.elapsed_time(e1) / Ln
    gateup_ms = e1.elapsed_time(e2) / Ln
    down_ms = e2.elapsed_time(e3) / Ln - gateup_ms
    gu_flop = 2.0 * T * k * 2 * spec.inter * H
    dn_flop = 2.0 * T * k * spec.inter * H
    # routing spread: distinct experts hit by the chunk, and the busiest expert's share
    counts = torch.bincount(idx[0].reshape(-1).long(), minlength=spec.n_experts).cpu()
    return {
        "tok_s": T / dt, "ms_per_chunk": dt * 1e3, "layers": Ln, "tokens": T,
        "router_us": router_ms * 1e3, "gateup_us": gateup_ms * 1e3, "down_us": down_ms * 1e3,
        "gateup_tflops": gu_flop / (gateup_ms * 1e-3) / 1e12,
        "down_tflops": dn_flop / (down_ms * 1e-3) / 1e12 if down_ms > 0 else None,
        "layer_tflops": (gu_flop + dn_flop) / (dt / Ln) / 1e12,
        "max_expert_rows": int(counts.max()), "experts_hit": int((counts > 0).sum()),
    }


def _p(t):
    return None if t is None else t.data_ptr()


def decode_report(st: "Stack", T: int, steps: int, per_graph: int = 16, reps: int = 3):
    """Kernel-level decode of T tokens through every layer of `st` (one brx_moe_block_forward
    per layer, all experts resident) for `steps` steps, each with its own input rows (a fresh
    input per step: repeating a few inputs would let a biased router settle on experts the
    last-level cache then holds). Steps are captured `per_graph` at a time as HIP graphs and the
    graphs replayed in order."""
    import ctypes as C

    import torch

    from bigrig_amd import lib as L
    spec, Ln = st.spec, st.layers
    lib = L.load()
    d = spec.desc()
    dref = C.byref(d)
    H, k = spec.hidden, spec.top_k
    assert st.xbank[0].shape[0] >= steps * T, "input bank smaller than steps x T"
    outs = [torch.empty((T, H), dtype=torch.bfloat16, device="cuda") for _ in range(Ln)]
    idx = [[torch.empty((T, k), dtype=torch.int32, device="cuda") for _ in range(Ln)]
           for _ in range(steps)]
    sh = bool(spec.shared_inter)

    def step(i, stream):
        for l in range(Ln):
            x = st.xbank[l][i * T:(i + 1) * T]
            L.check(lib.brx_moe_block_forward(dref, st.pools[l].device.handle, x.data_ptr(),
                                              st.routers[l].data_ptr(), _p(st.biases[l]),
                                              st.shared_gate[l].data_ptr() if sh else None,
                                              st.shared[l].data_ptr() if sh else None, T,
                                              outs[l].data_ptr(), idx[i][l].data_ptr(), None,
                                              L.FWD_FORCE_DECODE, stream))

    # one eager step first: a pool's first forward orders itself after the pool's refills,
    # which a graph capture cannot wait on
    step(0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    gs = []
    for g0 in range(0, steps, per_graph):
        cg = torch.cuda.CUDAGraph()
        with torch.cuda.graph(cg):
            for i in range(g0, min(g0 + per_graph, steps)):
                step(i, torch.cuda.current_stream().cuda_stream)
        gs.append(cg)
    torch.cuda.synchronize()
    for cg in gs:
        cg.replay()
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for r in range(reps):
        for cg in gs:
            cg.replay()
    e1.record(s)
    torch.cuda.synchronize()
    us_layer = e0.elapsed_time(e1) * 1e3 / (reps * steps * Ln)
    distinct = sum(len(torch.unique(i)) for row in idx for i in row) / (steps * Ln)
    router_b = spec.n_experts * H * (4 if spec.router_dtype == "float32" else 2)
    nbytes = distinct * spec.bytes_per_expert + router_b + 2 * T * H * 2
    if spec.shared_inter:
        from bigrig_amd import formats as F
        nbytes += F.spec_bytes(spec.expert_spec(True)) + 2 * H
    del gs
    return {"tokens": T, "layers": Ln, "steps": steps, "us_per_layer": round(us_layer, 3),
            "layer_tokens_per_s": round(T * 1e6 / us_layer, 1),
            "distinct_experts": round(distinct, 2), "bytes_per_layer_step": int(nbytes),
            "hbm_gbs": round(nbytes / (us_layer * 1e-6) / 1e9, 1),
            "hbm_frac": round(nbytes / (us_layer * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def prefill_report(st: "Stack", T: int, reps: int = 3):
    """One T-token chunk through every layer of `st`: router, bucketing, grouped GEMMs, combine."""
    import ctypes as C

    import torch

    from bigrig_amd import lib as L
    from bigrig_amd import synth
    spec, Ln = st.spec, st.layers
    lib = L.load()
    d = spec.desc()
    dref = C.byref(d)
    H, k = spec.hidden, spec.top_k
    xs = [synth.activations(T, H, seed=7000 + l) for l in range(Ln)]
    out = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    idx = [torch.empty((T, k), dtype=torch.int32, device="cuda") for _ in range(Ln)]
    sp = torch.cuda.current_stream().cuda_stream

    def chunk():
        for l in range(Ln):
            sh = bool(spec.shared_inter)
            L.check(lib.brx_moe_block_forward(dref, st.pools[l].device.handle, xs[l].data_ptr(),
                                              st.routers[l].data_ptr(), _p(st.biases[l]),
                                              st.shared_gate[l].data_ptr() if sh else None,
                                              st.shared[l].data_ptr() if sh else None, T,
                                              out.data_ptr(), idx[l].data_ptr(), None,
                                              L.FWD_FORCE_PREFILL, sp))

    chunk()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        chunk()
    torch.cuda.synchronize()
    us_layer = (time.perf_counter() - t0) * 1e6 / (reps * Ln)
    hit = sum(len(torch.unique(i)) for i in idx) / Ln
    nbytes = hit * spec.bytes_per_expert + spec.n_experts * H * 2 + 2 * 2 * T * H
    flops = 2.0 * T * k * 3 * H * spec.inter
    return {"tokens": T, "layers": Ln, "us_per_layer": round(us_layer, 2),
            "tokens_per_s_all_layers": round(T * 1e6 / (us_layer * Ln), 1),
            "experts_hit": round(hit, 1), "bytes_per_layer": int(nbytes),
            "hbm_gbs": round(nbytes / (us_layer * 1e-6) / 1e9, 1),
            "hbm_frac": round(nbytes / (us_layer * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "tflops": round(flops / (us_layer * 1e-6) / 1e12, 1),
            "mfma_frac": round(flops / (us_layer * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4)}


def layered_bench(st: "Stack", n_layers: int = 8, prompt: int = 32768, chunk: int = 2048):
    """Layer-major prefill of a long prompt (bigrig_amd/layered.py) with every layer's experts
    streamed from pinned host memory over PCIe into a ring of two whole layers in HBM: the next
    layer's copy overlapping this layer's chunks (read-ahead) against the serial schedule, and
    the same chunks with the layers already resident (compute alone)."""
    import torch

    from bigrig_amd import layered, synth
    spec = st.spec
    nl = min(n_layers, len(st.host.layers()))
    if nl < 2:
        return None
    ws = [layered.MoEWeights(l, st.routers[l], st.biases[l]) for l in range(nl)]
    chunks = [synth.activations(chunk, spec.hidden, seed=8000 + j) for j in range(prompt // chunk)]
    ring = layered.LayerRing(spec)

    def run(layers, read_ahead, reset=True):
        if reset:
            ring.reset()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        layered.prefill(spec, layers, st.host, chunks, ring, read_ahead=read_ahead)
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    run(ws, True)
    t_ra = min(run(ws, True) for _ in range(2))
    t_ser = min(run(ws, False) for _ in range(2))
    # compute alone: layers 0 and 1 alternate over the two sets, which already hold them
    alt = [ws[i % 2] for i in range(nl)]
    run(alt, True)
    t_cmp = min(run(alt, True, reset=False) for _ in range(2))
    layer_bytes = spec.n_experts * spec.bytes_per_expert
    t_copy = max(t_ser - t_cmp, 1e-9)
    ring.close()
    return {"layers": nl, "prompt_tokens": len(chunks) * chunk, "chunk": chunk,
            "layer_bytes": layer_bytes, "read_ahead_ms": round(t_ra * 1e3, 2),
            "serial_ms": round(t_ser * 1e3, 2), "compute_ms": round(t_cmp * 1e3, 2),
            "tok_s_read_ahead": round(len(chunks) * chunk / t_ra, 1),
            "tok_s_serial": round(len(chunks) * chunk / t_ser, 1),
            "pcie_gbs": round(nl * layer_bytes / t_copy / 1e9, 1),
            "hidden_frac": round((t_ser - t_ra) / max(min(t_copy, t_cmp), 1e-9), 3)}


def config_report(args):
    """The other configurations, each as specified, all experts resident unless stated:
      OLMoE-1B-7B layer, decode batch 1: 256 seeded steps, each with a fresh input, cycled over
        16 distinct weight replicas (3.6 GB, far beyond the 256 MB last-level cache); fp32
        router, softmax top-8 without renormalisation, no router bias;
      256 experts + shared expert, the 40-layer stack (18 GB), Zipf(1.1) router bias: decode at
        batch 1 and batch 8 (64 steps, fresh inputs), and end to end through 38 of 256 slots per
        layer (15% residency), synchronous and host-served (PCIe-inclusive);
      gpt-oss-120b MXFP4, the 36-layer stack (61 GB), plain logits: decode at batch 1 (64 steps,
        fresh inputs) and one 512-token prefill chunk through every layer."""
    import torch

    from bigrig_amd.spec import E256_SHARED, GPT_OSS_120B, OLMOE_1B_7B
    rep = {}
    st = Stack(OLMOE_1B_7B, 16, bank=256, zipf=None)
    rep["olmoe_1b_7b_decode_b1"] = decode_report(st, 1, steps=256)
    del st
    torch.cuda.empty_cache()
    keep = 0 if "pool" in args.skip else 40
    st = Stack(E256_SHARED, 40, bank=64 * 8, keep_host_layers=keep)
    rep["e256_shared_decode_b1"] = decode_report(st, 1, steps=64)
    rep["e256_shared_decode_b8"] = decode_report(st, 8, steps=64, per_graph=8)
    if keep:
        log("256-expert + shared through 38 slots")
        pool = {"synchronous": pool_bench(args, st, capacities=[38] * keep),
                "host_served": pool_bench(args, st, host_served=True, capacities=[38] * keep)}
        rep["e256_shared_pool_c38"] = {
            k2: {k3: (round(v, 4) if isinstance(v, float) else v) for k3, v in d.items()}
            for k2, d in pool.items()}
    del st
    torch.cuda.empty_cache()
    st = Stack(GPT_OSS_120B, 36, bank=64, zipf=None)
    rep["gpt_oss_120b_decode_b1"] = decode_report(st, 1, steps=64)
    rep["gpt_oss_120b_prefill_512"] = prefill_report(st, 512, reps=1)
    del st
    torch.cuda.empty_cache()
    return rep


# affine widths of the reference's per-layer precision candidates (bigrig_engine/precision.py:58),
# and unquantized bf16 experts (16, 0)
WIDTHS = [(2, 128), (2, 64), (3, 128), (3, 64), (4, 128), (4, 64), (6, 64), (8, 64), (16, 0)]


def widths_report():
    """The Qwen3-30B-A3B-shaped layer (Zipf(1.1) router bias, all experts resident) at every
    affine width and group size, and with bf16 experts: 8 layers (1.4-9.7 GB, beyond the
    last-level cache), decode at batch 1 (64 steps, fresh inputs) and 2048-token prefill
    chunks (4-bit g64 is the headline layer, measured here in the same way as the others)."""
    from dataclasses import replace

    import torch

    from bigrig_amd import formats as F
    from bigrig_amd.spec import QWEN3_30B_A3B
    rep = {}
    for b_, g_ in WIDTHS:
        q = F.QuantSpec(16, 0, "none") if b_ == 16 else F.QuantSpec(b_, g_)
        spec = replace(QWEN3_30B_A3B, quant=q)
        st = Stack(spec, 8, bank=64)
        dec = decode_report(st, 1, steps=64)
        pf = prefill_report(st, 2048, reps=3)
        rep["bf16" if b_ == 16 else f"{b_}bit_g{g_}"] = {
            "bytes_per_expert": spec.bytes_per_expert,
            "decode_us_per_layer": dec["us_per_layer"], "decode_hbm_frac": dec["hbm_frac"],
            "prefill_us_per_layer": pf["us_per_layer"], "prefill_mfma_frac": pf["mfma_frac"]}
        log(f"width {b_}-bit g{g_}: decode {dec['us_per_layer']} us, prefill {pf['us_per_layer']} us per layer")
        del st
        torch.cuda.empty_cache()
    return rep


def pool_bench(args, st: "Stack", host_served: bool = False, capacities=None):
    """Bounded pool end to end: C of E experts per layer resident, misses copied from pinned
    host memory. Synchronous: one routing read-back per layer, misses admitted before the layer
    computes. host_served: the kernels read misses from the pinned store themselves and
    residency follows behind the forwards. `capacities` gives each layer its own C (a whole-layer
    plan). PCIe-inclusive; never the headline value."""
    import torch

    from bigrig_amd.layer import MoELayer, StreamingSwitchGLU
    from bigrig_amd.pool import ExpertPool, PinnedFetcher
    spec = st.spec
    layers = st.host.layers()
    fetcher = PinnedFetcher(st.host)
    mods = []
    for i, l in enumerate(layers):
        cap = args.pool_capacity if capacities is None else capacities[i]
        pool = ExpertPool(l, spec, cap).build()
        shared = st.shared[l] if spec.shared_inter else None
        sw = StreamingSwitchGLU(pool, fetcher, shared=shared, host_served=host_served)
        sw.refresh()
        mods.append(MoELayer(spec, st.routers[l], sw, router_bias=st.biases[l],
                             shared_gate_w=st.shared_gate[l] if spec.shared_inter else None))
    from bigrig_amd import synth
    n = args.pool_tokens
    # a fresh activation per (layer, token): repeating a small input bank would let the pool
    # settle on that bank's experts and report no misses
    xs = [synth.activations(8 + n, spec.hidden, seed=6000 + l) for l in layers]

    def token(i):
        for l, m in zip(layers, mods):
            m(xs[l][i:i + 1])

    for i in range(8):            # fill the pools
        token(i)
    torch.cuda.synchronize()
    for m in mods:
        p = m.switch._pool
        p.hits = p.misses = 0
    t0 = time.perf_counter()
    for i in range(n):
        token(8 + i)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    hits = sum(m.switch._pool.hits for m in mods)
    miss = sum(m.switch._pool.misses for m in mods)
    caps = sorted(set(capacities)) if capacities is not None else [args.pool_capacity]
    res = {"capacity": caps[0] if len(caps) == 1 else "per layer",
           "layers": len(layers),
           "tok_s": n / dt,
           "miss_rate": miss / max(1, hits + miss),
           "pcie_inclusive": True}
    if host_served:
        res["host_waits_s"] = sum(m.switch.sync_seconds for m in mods)
        res["admit_gb"] = sum(m.switch._serve.admit_bytes for m in mods) / 1e9
    for m in mods:
        m.switch._pool.close()
    return res


def replay_bench() -> dict:
    """Trace-replay throughput (host CPU): the Python restatement of LFUDA on two layers of the
    shipped Qwen3 routing trace against the native sweep over all 48 layers at three
    capacities, LFUDA and the Belady bound, on 16 threads; miss rates as evaluate() gives them."""
    import numpy as np

    from bigrig_amd import policy as P
    from bigrig_amd import replay as R
    idx = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "tests", "golden",
                               "qwen3_full.npz"))["idx"].astype(np.int32)
    L, T, k = idx.shape
    caps = [16, 32, 64]
    t0 = time.perf_counter()
    for l in range(2):
        seq, ranks = P.layer_sequence(idx, l)
        P.simulate(seq, 32, 128, P.LFUDA, ranks)
    py = 2 * T * k / (time.perf_counter() - t0)
    out = {"trace": f"qwen3 routing, {L} layers x {T} tokens x top-{k}", "capacities": caps,
           "python_lfuda_req_s": round(py)}
    for name in ("lfuda", "belady"):
        t0 = time.perf_counter()
        m = R.trace_misses(name, idx, caps, 128, threads=16)
        dt = time.perf_counter() - t0
        out[f"native_{name}_req_s"] = round(len(caps) * L * T * k / dt)
        out[f"{name}_miss_rate"] = [round(float(v), 4) for v in m.sum(1) / (L * T * k)]
    out["threads"] = 16
    return out


def cpu_bench(args, st: "Stack"):
    """The CPU baseline (oracle/cpu_baseline.c: router, fp32 dequant-on-the-fly GEMVs and the
    combine, OpenMP over output rows) on a bounded sample: decode tokens through two layers of
    the same stack, read from the pinned host copies of their experts, until cpu_seconds of
    work, scaled to the 48-layer stack."""
    import numpy as np
    import torch

    import oracle
    spec = st.spec
    oracle.build(force=False)
    nlay = 2
    blobs, routers, biases = [], [], []
    for l in range(nlay):
        blobs.append(st.host.tensor(l))          # pinned [E, bytes_per_expert] uint8
        routers.append(st.routers[l].view(torch.int16).cpu().numpy().view(np.uint16))
        biases.append(st.biases[l].cpu().numpy())
    xs = [st.xbank[l].view(torch.int16).cpu().numpy().view(np.uint16) for l in range(nlay)]
    G = xs[0].shape[0]
    cores = len(os.sched_getaffinity(0))
    n, t0 = 0, time.perf_counter()
    while True:
        for l in range(nlay):
            oracle.cpu_baseline_decode(spec, xs[l][n % G], routers[l], biases[l],
                                       blobs[l].data_ptr(), blobs[l].shape[1], nthreads=cores)
        n += 1
        el = time.perf_counter() - t0
        if el >= args.cpu_seconds:
            break
    per_layer_tok = el / (n * nlay)
    return {"value": 1.0 / (per_layer_tok * 48), "unit": "tokens/s", "cores": cores,
            "kind": "port",
            "sample": f"{n} decode tokens x {nlay} layers of the same stack (router, 8 experts as "
                      f"fp32 dequant-on-the-fly GEMVs, combine; OpenMP over output rows), "
                      f"{el:.1f}s, scaled to 48 layers"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the library has no multi-GPU path (got --gpus "
              f"{args.gpus}). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch

    from bigrig_amd import lib as L
    from bigrig_amd.spec import QWEN3_30B_A3B
    if not torch.cuda.is_available():
        print("bench.py needs a GPU (no CPU fallback)", file=sys.stderr)
        sys.exit(1)
    L.init(0)
    if args.copy_mib:
        copy_probe(args)
        return
    spec = QWEN3_30B_A3B
    skip = set(filter(None, args.skip.split(",")))
    keep = 0 if "pool" in skip else args.layers
    if "cpu" not in skip:
        keep = max(keep, 2)
    st = Stack(spec, args.layers, bank=8, keep_host_layers=keep)
    log("decode")
    dec = decode_bench(args, st)
    pre = None
    if "prefill" not in skip:
        log("prefill")
        pre = prefill_bench(args, st)
    pool = None
    if "pool" not in skip:
        from bigrig_amd.hostserve import plan_full_layers
        log("bounded pool")
        pool = pool_bench(args, st)
        log("bounded pool, misses served from host memory")
        pool["host_served"] = pool_bench(args, st, host_served=True)
        nl = len(st.host.layers())
        whole, rest = plan_full_layers(48, st.spec.n_experts, st.spec.top_k,
                                       args.pool_capacity)
        if whole:
            caps = [st.spec.n_experts if i < round(whole * nl / 48) else rest
                    for i in range(nl)]
            log(f"bounded pool, host-served, {whole} of 48 layers whole, the rest at {rest}")
            hp = pool_bench(args, st, host_served=True, capacities=caps)
            hp["plan"] = {"whole_of_48": whole, "rest_capacity": rest}
            pool["host_served_plan"] = hp
    lay = None
    if "layered" not in skip and "pool" not in skip:
        log("layer-major prefill, experts streamed from host")
        lay = layered_bench(st)
    rep = None
    if "replay" not in skip:
        log("policy replay (host)")
        rep = replay_bench()
    cpu = None
    if "cpu" not in skip:
        log("cpu baseline")
        cpu = cpu_bench(args, st)
    report = None
    if "report" not in skip:
        log("other shapes")
        del st
        torch.cuda.empty_cache()
        report = config_report(args)
    widths = None
    if "widths" not in skip:
        log("affine widths")
        if "report" in skip:
            del st
            torch.cuda.empty_cache()
        widths = widths_report()
    # HBM bytes per launch of the timed kernel, from the committed FETCH_SIZE / WRITE_SIZE
    # profile; only counters taken on this kernel are reported
    traffic = None
    tp = os.path.join(ROOT, "profiles", "traffic_decode_gateup.json")
    if os.path.exists(tp):
        try:
            tj = json.load(open(tp))
            if tj.get("kernel") == DECODE_GATEUP_KERNEL:
                traffic = tj.get("traffic_bytes")
        except (OSError, ValueError):
            traffic = None
    rec = {
        "metric": METRIC,
        "value": round(dec["tok_s"], 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"qwen3-30b-a3b-shape MoE stack, {args.layers} layers, decode batch 1: "
                        f"hidden 2048, 128 experts, softmax top-8 renorm, inter 768, SwiGLU, "
                        f"MLX affine 4-bit g64 bf16 scale/bias, all experts HBM-resident, "
                        f"Zipf(1.1) router bias, HIP-graph replay" if dec["graph"] else
                        f"qwen3-30b-a3b-shape MoE stack, {args.layers} layers, decode batch 1 "
                        f"(eager launches)",
            "layers": args.layers, "batch": 1, "experts": 128, "top_k": 8,
            "weights": "4-bit affine g64", "layer_gb_per_token": round(dec["layer_bytes"] / 1e9, 5),
        },
        "roofline": {
            "bound": "hbm", "achieved": _r(dec["gateup_gbs"], 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": _r(dec["gateup_gbs"] / HBM_PEAK_GBS if dec["gateup_gbs"] else None, 4),
            "traffic": traffic,
            "kernel": f"{DECODE_GATEUP_KERNEL}: one token's gate/up + SwiGLU, routed in-kernel "
                      f"({spec.top_k} experts x gate+up, {dec['gateup_bytes']:,} B per launch)",
            "avg_us": _r(dec["gateup_us"], 3),
        },
        "decode_kernels": {
            "router_us": _r(dec["router_us"], 3),
            "gateup_us": _r(dec["gateup_us"], 3), "down_us": _r(dec["down_us"], 3),
            "gateup_gbs": _r(dec["gateup_gbs"], 1),
            "down_gbs": _r(dec["down_gbs"], 1),
            "stack_gbs": round(dec["step_gbs"], 1),
            "stack_frac": round(dec["step_gbs"] / HBM_PEAK_GBS, 4),
            "eager_tok_s": round(dec["eager_tok_s"], 1),
        },
        "cpu_baseline": cpu,
    }
    if pre is not None:
        rec["prefill"] = {
            "tokens": pre["tokens"], "layers": pre["layers"], "tok_s": round(pre["tok_s"], 1),
            "ms_per_chunk": round(pre["ms_per_chunk"], 3),
            "router_us": round(pre["router_us"], 2), "gateup_us": round(pre["gateup_us"], 2),
            "down_us": round(pre["down_us"], 2),
            "roofline": {"bound": "mfma", "achieved": round(pre["gateup_tflops"], 1),
                         "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(pre["gateup_tflops"] / BF16_PEAK_TFLOPS, 4),
                         "kernel": "k_pf_gemm gate/up + SwiGLU (+ k_bucket)"},
            "layer_tflops": round(pre["layer_tflops"], 1),
            "max_expert_rows": pre["max_expert_rows"], "experts_hit": pre["experts_hit"],
        }
    if report is not None:
        rec["report"] = report
    if widths is not None:
        rec["widths"] = widths
    if pool is not None:
        def rnd(d):
            return {k2: (rnd(v) if isinstance(v, dict) else round(v, 4) if isinstance(v, float)
                         else v) for k2, v in d.items()}
        rec["bounded_pool"] = rnd(pool)
    if lay is not None:
        rec["layer_major_prefill"] = lay
    if rep is not None:
        rec["policy_replay"] = rep
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
