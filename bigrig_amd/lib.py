"""ctypes binding of libbrx.so (include/brx.h).

Loading fails loudly: there is no CPU fallback for any entry point. `load()` raises if the
library has not been built (`python -m bigrig_amd.build`) or cannot be opened.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

from .build import LIB

# ------------------------------------------------------------------ constants (brx.h)
BRX_OK, BRX_EINVAL, BRX_ESTATE, BRX_EHIP, BRX_ENOMEM, BRX_ERANGE = 0, -1, -2, -3, -4, -5
QUANT_AFFINE, QUANT_MXFP4, QUANT_NONE = 0, 1, 2
SCALE_BF16, SCALE_F16 = 0, 1
ACT_SWIGLU, ACT_SWIGLU_CLAMPED = 0, 1
ROUTE_SOFTMAX_TOPK, ROUTE_SOFTMAX_TOPK_RENORM, ROUTE_TOPK_SOFTMAX = 0, 1, 2
ROUTE_SIGMOID_TOPK, ROUTE_SIGMOID_TOPK_RENORM = 3, 4
DT_F32, DT_BF16 = 0, 1
FWD_FORCE_DECODE, FWD_FORCE_PREFILL, FWD_PHASE_A, FWD_PHASE_B, FWD_PHASE_R = 1, 2, 4, 8, 16
ABI_VERSION = 2         # brx_abi_version() of the library this binding matches (BRX_ABI_VERSION)
NOALLOC_SCRATCH_BYTES = 16 << 20

EXPORTS = (
    "brx_abi_version", "brx_last_error", "brx_init", "brx_expert_layout_get",
    "brx_pool_create", "brx_pool_destroy", "brx_pool_capacity", "brx_pool_slot_ptr",
    "brx_pool_g2s_ptr", "brx_pool_refill_async", "brx_pool_refill_from_device_async",
    "brx_pool_set_g2s", "brx_pool_sync", "brx_router_topk", "brx_moe_forward",
    "brx_moe_forward_pairs", "brx_moe_block_forward", "brx_combine", "brx_dequant",
    "brx_sort_pairs", "brx_pool_set_host_backing", "brx_pool_publish_async",
    "brx_pool_admit_async", "brx_pool_refill_range_async", "brx_pool_check",
    "brx_moe_block_forward_noalloc",
)


class LayerDesc(C.Structure):
    _fields_ = [("hidden", C.c_int32), ("inter", C.c_int32), ("n_experts", C.c_int32),
                ("top_k", C.c_int32), ("quant_mode", C.c_int32), ("bits", C.c_int32),
                ("group_size", C.c_int32), ("scale_dtype", C.c_int32), ("has_bias", C.c_int32),
                ("act", C.c_int32), ("alpha", C.c_float), ("limit", C.c_float),
                ("route_mode", C.c_int32), ("router_dtype", C.c_int32),
                ("shared_inter", C.c_int32), ("n_group", C.c_int32), ("topk_group", C.c_int32),
                ("route_scale", C.c_float), ("reserved", C.c_int32 * 2)]


class ExpertLayout(C.Structure):
    _fields_ = [("weight", C.c_int64 * 3), ("scales", C.c_int64 * 3), ("biases", C.c_int64 * 3),
                ("bias", C.c_int64 * 3), ("bytes_per_expert", C.c_int64)]


class BrxError(RuntimeError):
    """A libbrx entry point returned an error code."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"libbrx error {code}: {msg}")
        self.code = code


_lib = None
_lock = threading.Lock()
_init_device = None

_vp, _i32p, _f32p = C.c_void_p, C.POINTER(C.c_int32), C.POINTER(C.c_float)
_SIGS = {
    "brx_abi_version": ([], C.c_int),
    "brx_last_error": ([], C.c_char_p),
    "brx_init": ([C.c_int], C.c_int),
    "brx_expert_layout_get": ([C.POINTER(LayerDesc), C.c_int, C.POINTER(ExpertLayout)], C.c_int),
    "brx_pool_create": ([C.POINTER(LayerDesc), C.c_int, C.POINTER(_vp)], C.c_int),
    "brx_pool_destroy": ([_vp], C.c_int),
    "brx_pool_capacity": ([_vp], C.c_int),
    "brx_pool_slot_ptr": ([_vp, C.c_int, C.POINTER(_vp)], C.c_int),
    "brx_pool_g2s_ptr": ([_vp, C.POINTER(_vp)], C.c_int),
    "brx_pool_refill_async": ([_vp, C.c_int, _vp, C.c_size_t, _vp], C.c_int),
    "brx_pool_refill_from_device_async": ([_vp, C.c_int, _vp, C.c_size_t, _vp], C.c_int),
    "brx_pool_set_g2s": ([_vp, _i32p, C.c_int, _vp], C.c_int),
    "brx_pool_sync": ([_vp], C.c_int),
    "brx_pool_check": ([_vp], C.c_int),
    "brx_pool_set_host_backing": ([_vp, _vp, C.c_int64, C.c_size_t], C.c_int),
    "brx_pool_publish_async": ([_vp, C.c_int, _i32p, _i32p, _vp], C.c_int),
    "brx_pool_admit_async": ([_vp, C.c_int, C.c_int, _vp, C.c_size_t, _vp], C.c_int),
    "brx_pool_refill_range_async": ([_vp, C.c_int, C.c_int, _vp, C.c_int64, C.c_size_t, _vp],
                                    C.c_int),
    "brx_router_topk": ([C.POINTER(LayerDesc), _vp, _vp, _vp, _vp, C.c_int, _vp, _vp, _vp, _vp],
                        C.c_int),
    "brx_moe_forward": ([C.POINTER(LayerDesc), _vp, _vp, _vp, _vp, _vp, _vp, C.c_int, _vp, _vp,
                         C.c_uint, _vp], C.c_int),
    "brx_moe_forward_pairs": ([C.POINTER(LayerDesc), _vp, _vp, C.c_int, _vp, _vp, _vp, C.c_int,
                               C.c_int, _vp, _vp, C.c_uint, _vp], C.c_int),
    "brx_moe_block_forward": ([C.POINTER(LayerDesc), _vp, _vp, _vp, _vp, _vp, _vp, C.c_int, _vp,
                               _vp, _vp, C.c_uint, _vp], C.c_int),
    "brx_moe_block_forward_noalloc": ([C.POINTER(LayerDesc), _vp, _vp, _vp, _vp, _vp, _vp, C.c_int,
                                       _vp, _vp, _vp, C.c_uint, _vp], C.c_int),
    "brx_combine": ([C.POINTER(LayerDesc), _vp, _vp, _vp, _vp, C.c_int, _vp, _vp], C.c_int),
    "brx_dequant": ([C.POINTER(LayerDesc), _vp, C.c_int, C.c_int, _vp, _vp], C.c_int),
    "brx_sort_pairs": ([C.POINTER(LayerDesc), _vp, C.c_int, _vp, _vp, _vp], C.c_int),
}


def load(path: str | None = None):
    """Open libbrx.so and declare its signatures (no GPU call is made)."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or LIB
        if not os.path.exists(p):
            raise RuntimeError(f"{p} is missing: build it with `python -m bigrig_amd.build` "
                               f"(there is no CPU fallback)")
        lib = C.CDLL(p)
        for name, (args, res) in _SIGS.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        if lib.brx_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{p} has ABI {lib.brx_abi_version()}, this binding expects "
                               f"{ABI_VERSION}: rebuild the library")
        if path is None:
            _lib = lib
        return lib


def check(rc: int) -> None:
    if rc != BRX_OK:
        msg = load().brx_last_error()
        raise BrxError(rc, msg.decode() if msg else "")


def init(device: int = 0) -> None:
    """brx_init(device) once per process (idempotent for the same device)."""
    global _init_device
    if _init_device == device:
        return
    check(load().brx_init(device))
    _init_device = device


def ptr(t) -> int | None:
    """Device/host address of a torch tensor (or None)."""
    if t is None:
        return None
    return t.data_ptr()


def stream_ptr(stream=None) -> int | None:
    """hipStream_t of a torch stream (default: torch's current stream)."""
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream or None
