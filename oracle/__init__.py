"""ORACLE -- test infrastructure only; the product never imports this package.

Only tests/, the smoke check in __graft_entry__.py and bench.py's CPU-baseline leg use it, and
only as the reference result to compare against (or the timed CPU baseline), never as a code
path of the product.

Two restatements of the reference's routed-expert layer (the reference computes it through MLX,
which cannot run here; see moe_oracle.c for the file:line each function follows):

* `moe_oracle.c` (built by `build()` into oracle/_build/liboracle.so): the router in the
  kernels' exact fp32 reduction order (indices bit-exact), dequantization (bit-exact fp32),
  the layer with the kernels' bf16 rounding points, OpenMP-parallel (the CPU baseline), and
  the stable pair bucketing.
* numpy float64 here: `moe_forward_f64`, the "truth" the C layer and the kernels are both
  compared against, and `router_f64` for closed-form pins.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(BUILD, "liboracle.so")
SRC = os.path.join(HERE, "moe_oracle.c")
# the CPU baseline bench.py times (not the oracle: see cpu_baseline.c)
CPB_LIB = os.path.join(BUILD, "libcpu_baseline.so")
CPB_SRC = os.path.join(HERE, "cpu_baseline.c")

_lib = None
_cpb = None


def _gcc(src: str, out: str, flags: list, force: bool) -> str:
    if not force and os.path.exists(out) and os.path.getmtime(out) >= os.path.getmtime(src):
        return out
    tmp = out + ".tmp"
    cmd = ["gcc", *flags, "-fopenmp", "-fPIC", "-shared", src, "-o", tmp, "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build of {os.path.basename(src)} failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, out)
    return out


def build(force: bool = True) -> str:
    """gcc -O3 -fopenmp the C restatement (-ffp-contract=off keeps fmaf() the only fused op),
    and the CPU baseline (vectorized: reassociation allowed, it is timed, not compared bit for
    bit)."""
    os.makedirs(BUILD, exist_ok=True)
    # reassociation (vectorized sums) without -ffast-math, whose startup code would switch the
    # whole process to flush-to-zero when the library loads
    _gcc(CPB_SRC, CPB_LIB, ["-O3", "-march=x86-64-v3", "-fassociative-math", "-fno-signed-zeros",
                            "-fno-trapping-math", "-fno-math-errno"], force)
    return _gcc(SRC, LIB, ["-O3", "-march=x86-64-v3", "-ffp-contract=off", "-fno-fast-math"], force)


class OrcLayer(C.Structure):
    _fields_ = [("H", C.c_int), ("I", C.c_int), ("quant_mode", C.c_int), ("bits", C.c_int),
                ("gs", C.c_int), ("scale_f16", C.c_int), ("has_bias", C.c_int), ("act", C.c_int),
                ("alpha", C.c_float), ("limit", C.c_float)]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        _lib = C.CDLL(LIB)
        vp = C.c_void_p
        _lib.orc_dot_lane_tree.argtypes = [vp, vp, C.c_int, C.c_int]
        _lib.orc_dot_lane_tree.restype = C.c_float
        _lib.orc_exp_rt.argtypes = [C.c_float]
        _lib.orc_exp_rt.restype = C.c_float
        _lib.orc_router.argtypes = [vp, vp, C.c_int, vp, vp, C.c_int, C.c_int, C.c_int, C.c_int,
                                    C.c_int, C.c_int, C.c_int, C.c_float, vp, vp, vp, vp]
        _lib.orc_dequant.argtypes = [C.POINTER(OrcLayer), vp, C.c_int, C.c_int, vp]
        _lib.orc_moe_forward.argtypes = [C.POINTER(OrcLayer), vp, C.c_int, vp, C.c_int, vp, vp, vp,
                                         vp, C.c_int, vp, vp, C.c_int]
        _lib.orc_sort_pairs.argtypes = [vp, C.c_int, C.c_int, vp, vp]
        _lib.orc_num_threads.restype = C.c_int
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def orc_layer(spec) -> OrcLayer:
    """OrcLayer from a bigrig_amd.layer.LayerSpec-like object."""
    q = spec.quant
    # unquantized (bf16) weights: mode 2; the group size only sets the oracle's summation chunks
    return OrcLayer(spec.hidden, spec.inter, {"affine": 0, "mxfp4": 1, "none": 2}[q.mode], q.bits,
                    q.group_size or 64,
                    1 if q.scale_dtype == "float16" else 0, int(spec.has_bias),
                    {"swiglu": 0, "swiglu_clamped": 1, "silu_mlp": 2}[spec.act], spec.alpha,
                    spec.limit)


# ------------------------------------------------------------------ C restatement wrappers
def dot_lane_tree(x_bits: np.ndarray, w, w_f32: bool) -> float:
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.float32 if w_f32 else np.uint16)
    return float(lib().orc_dot_lane_tree(_p(x), _p(w), int(w_f32), x.shape[-1]))


def router(x_bits, w, w_f32: bool, bias, k: int, mode: int, shared_gate_w=None, n_group: int = 0,
           topk_group: int = 0, scale: float = 1.0):
    """(logits [T,E] f32, idx [T,k] i32, w [T,k] f32, sgate [T] f32|None) in the kernels' order.
    mode: 0 softmax-topk, 1 softmax-topk-renorm, 2 topk-softmax, 3 sigmoid-topk (bias enters
    the selection only), 4 sigmoid-topk-renorm; n_group > 1 limits the top-k to the
    topk_group best expert groups; the weights are multiplied by `scale`. Sigmoid modes return
    the raw logits."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    T, H = x.shape
    wr = np.ascontiguousarray(w, dtype=np.float32 if w_f32 else np.uint16)
    E = wr.shape[0]
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    sg = None if shared_gate_w is None else np.ascontiguousarray(shared_gate_w, dtype=np.uint16)
    logits = np.zeros((T, E), np.float32)
    idx = np.zeros((T, k), np.int32)
    wts = np.zeros((T, k), np.float32)
    sgo = np.zeros(T, np.float32) if sg is not None else None
    rc = lib().orc_router(_p(x), _p(wr), int(w_f32), _p(b), _p(sg), T, H, E, k, mode, n_group,
                          topk_group, float(scale), _p(logits), _p(idx), _p(wts), _p(sgo))
    if rc != 0:
        raise ValueError("orc_router rejected its arguments")
    return logits, idx, wts, sgo


def dequant(spec, expert: bytes, proj: int, shared: bool = False) -> np.ndarray:
    L = orc_layer(spec)
    inter = spec.shared_inter if shared else spec.inter
    buf = np.frombuffer(expert, dtype=np.uint8)
    n_out, n_in = (inter, spec.hidden) if proj < 2 else (spec.hidden, inter)
    out = np.zeros((n_out, n_in), np.float32)
    if lib().orc_dequant(C.byref(L), _p(buf), inter, proj, _p(out)) != 0:
        raise ValueError("orc_dequant supports 4-bit layouts only")
    return out


def moe_forward(spec, experts: list, x_bits, idx, w, shared: bytes | None = None, sgate=None,
                nthreads: int = 0, want_unreduced: bool = False):
    """Layer output (out [T,H] bf16 bits, y_unreduced [T,k,H] bf16 bits | None)."""
    L = orc_layer(spec)
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    T = x.shape[0]
    k = spec.top_k
    bufs = [np.frombuffer(b, dtype=np.uint8) for b in experts]
    ptrs = (C.c_void_p * len(bufs))(*[b.ctypes.data for b in bufs])
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    sh = None if shared is None else np.frombuffer(shared, dtype=np.uint8)
    sg = None if sgate is None else np.ascontiguousarray(sgate, dtype=np.float32)
    out = np.zeros((T, spec.hidden), np.uint16)
    yun = np.zeros((T, k, spec.hidden), np.uint16) if want_unreduced else None
    rc = lib().orc_moe_forward(C.byref(L), C.cast(ptrs, C.c_void_p), k, _p(sh),
                               spec.shared_inter if sh is not None else 0, _p(x), _p(idx), _p(w),
                               _p(sg), T, _p(out), _p(yun), nthreads)
    if rc != 0:
        raise ValueError(f"orc_moe_forward failed ({rc})")
    return out, yun


def sort_pairs(idx, E: int):
    flat = np.ascontiguousarray(np.asarray(idx).reshape(-1), dtype=np.int32)
    order = np.zeros(flat.size, np.int32)
    offsets = np.zeros(E + 1, np.int32)
    if lib().orc_sort_pairs(_p(flat), flat.size, E, _p(order), _p(offsets)) != 0:
        raise ValueError("expert id out of range")
    return order, offsets


def num_threads() -> int:
    return int(lib().orc_num_threads())


# ------------------------------------------------------------------ CPU baseline (timed only)
def _cpb_lib():
    global _cpb
    if _cpb is None:
        if not os.path.exists(CPB_LIB):
            build(force=False)
        _cpb = C.CDLL(CPB_LIB)
        vp = C.c_void_p
        _cpb.cpb_decode_layer.argtypes = [vp, vp, vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                          C.c_int, vp, C.c_int64, vp, C.c_int]
        _cpb.cpb_decode_layer.restype = C.c_int
    return _cpb


def cpu_baseline_decode(spec, x_bits, router_bits, bias, experts_ptr: int, stride: int,
                        nthreads: int = 0) -> np.ndarray:
    """One decode token through one layer on the host with cpu_baseline.c (fp32 dequant-on-the-
    fly GEMVs, OpenMP): out [H] bf16 bits. `experts_ptr` is the host address of the layer's
    [E, stride] expert bytes. Only 4-bit affine group-64 SwiGLU layers without biases."""
    q = spec.quant
    if (q.mode != "affine" or q.bits != 4 or q.group_size != 64 or spec.has_bias or
            spec.act != "swiglu" or spec.route_mode not in (0, 1) or
            spec.router_dtype != "bfloat16"):
        raise ValueError("the CPU baseline runs 4-bit affine g64 SwiGLU layers with a bf16 "
                         "softmax router only")
    x = np.ascontiguousarray(x_bits, dtype=np.uint16).reshape(-1)
    wr = np.ascontiguousarray(router_bits, dtype=np.uint16)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    out = np.zeros(spec.hidden, np.uint16)
    rc = _cpb_lib().cpb_decode_layer(_p(x), _p(wr), _p(b), spec.hidden, spec.inter,
                                     spec.n_experts, spec.top_k, int(spec.route_mode == 1),
                                     int(q.scale_dtype == "float16"), experts_ptr, stride,
                                     _p(out), nthreads)
    if rc != 0:
        raise ValueError("cpb_decode_layer rejected its arguments")
    return out


# ------------------------------------------------------------------ float64 truth (numpy)
def _silu(g):
    return g / (1.0 + np.exp(-g))


def act_f64(spec, g, u):
    if spec.act == "swiglu":
        return _silu(g) * u
    if spec.act == "silu_mlp":
        return _silu(g)
    g = np.minimum(g, spec.limit)
    u = np.clip(u, -spec.limit, spec.limit)
    return g / (1.0 + np.exp(-spec.alpha * g)) * (u + 1.0)


def expert_weights_f64(spec, expert: bytes, shared: bool = False):
    """(Wg, Wu, Wd, bg, bu, bd) float64 from packed bytes (biases zero when absent). A plain
    two-layer expert returns (W_fc1, zeros, W_fc2, ...): its up projection contributes nothing."""
    from bigrig_amd import formats as F
    inter = spec.shared_inter if shared else spec.inter
    gated = spec.act != "silu_mlp"
    es = F.expert_spec(spec.hidden, inter, spec.quant, spec.has_bias, gated)
    arrs = F.split_expert(expert, es)
    W = [F.dequantize_projection(arrs, p, spec.quant).astype(np.float64) for p in es]
    if spec.has_bias:
        B = [F.bf16_bits_to_f32(arrs[(p, "bias")]).astype(np.float64) for p in es]
    else:
        B = [np.zeros(m.shape[0]) for m in W]
    if not gated:
        W.insert(1, np.zeros_like(W[0]))
        B.insert(1, np.zeros_like(B[0]))
    return W[0], W[1], W[2], B[0], B[1], B[2]


def moe_forward_f64(spec, experts: list, x_bits, idx, w, shared=None, sgate=None):
    """float64 layer output with no intermediate rounding: (out [T,H], y [T,k,H])."""
    from bigrig_amd import formats as F
    x = F.bf16_bits_to_f32(x_bits).astype(np.float64)
    T = x.shape[0]
    idx = np.asarray(idx)
    cache = {}

    def row(e, xt, sh=False):
        key = ("s" if sh else e)
        if key not in cache:
            cache[key] = expert_weights_f64(spec, shared if sh else experts[e], sh)
        Wg, Wu, Wd, bg, bu, bd = cache[key]
        h = act_f64(spec, Wg @ xt + bg, Wu @ xt + bu)
        return Wd @ h + bd

    y = np.zeros((T, spec.top_k, spec.hidden))
    out = np.zeros((T, spec.hidden))
    for t in range(T):
        for j in range(spec.top_k):
            y[t, j] = row(int(idx[t, j]), x[t])
            out[t] += float(w[t, j]) * y[t, j]
        if shared is not None:
            out[t] += float(sgate[t]) * row(-1, x[t], sh=True)
    return out, y


def exp_rt(x) -> np.ndarray:
    """The routing exponential (orc_exp_rt) over an array of float32 inputs."""
    xs = np.asarray(x, np.float32).reshape(-1)
    f = lib().orc_exp_rt
    return np.array([f(float(v)) for v in xs], np.float32).reshape(np.shape(x))


def router_f64(x_bits, w, w_f32: bool, bias, k: int, mode: int, n_group: int = 0,
               topk_group: int = 0, scale: float = 1.0):
    """float64 logits and the top-k set/weights from them (closed form, by sorting): sigmoid
    modes select on sigmoid + bias and weigh the sigmoid; groups score by their largest logit
    (softmax) or the sum of their two largest selection values (sigmoid, the two last entries
    of the group's sorted values), the topk_group best stay eligible."""
    from bigrig_amd import formats as F
    x = F.bf16_bits_to_f32(x_bits).astype(np.float64)
    W = (np.asarray(w, np.float64) if w_f32 else F.bf16_bits_to_f32(w).astype(np.float64))
    lg = x @ W.T
    sig = mode >= 3
    b = None if bias is None else np.asarray(bias, np.float64)
    if b is not None and not sig:
        lg = lg + b
    s = 1.0 / (1.0 + np.exp(-lg)) if sig else None
    c = (s + (0.0 if b is None else b)) if sig else lg.copy()
    if n_group > 1:
        T, E = c.shape
        g = c.reshape(T, n_group, E // n_group)
        gscore = np.sort(g, -1)[..., -2:].sum(-1) if sig else g.max(-1)
        best = np.argsort(-gscore, axis=-1, kind="stable")[:, :topk_group]
        keep = np.zeros((T, n_group), bool)
        np.put_along_axis(keep, best, True, -1)
        c = np.where(np.repeat(keep, E // n_group, axis=1), c, 0.0 if sig else -np.inf)
    order = np.argsort(-c, axis=-1, kind="stable")[:, :k]
    if sig:
        wts = np.take_along_axis(s, order, -1)
        if mode == 4:
            wts = wts / wts.sum(-1, keepdims=True)
        return lg, order, wts * scale
    sel = np.take_along_axis(lg, order, -1)
    if mode == 2:
        ex = np.exp(sel - sel[:, :1])
        wts = ex / ex.sum(-1, keepdims=True)
    else:
        p = np.exp(lg - lg.max(-1, keepdims=True))
        p = p / p.sum(-1, keepdims=True)
        wts = np.take_along_axis(p, order, -1)
        if mode == 1:
            wts = wts / wts.sum(-1, keepdims=True)
    return lg, order, wts * scale


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))
