"""ctypes binding of libmer_hip.so (the C ABI declared in include/mer_hip.h).

The library is the only compute path: if it is missing this module raises
instead of falling back to anything else.
"""
from __future__ import annotations

import ctypes
import enum
import os
import threading

from .build import LIB_PATH

c_size = ctypes.c_size_t
c_void = ctypes.c_void_p
c_int = ctypes.c_int
c_u64 = ctypes.c_uint64
c_float = ctypes.c_float


class MerLayerArgs(ctypes.Structure):
    _fields_ = [
        ("expert_table", c_void),
        ("table_len", c_size),
        ("expert_ids", c_void),
        ("weights", c_void),
        ("x", c_void),
        ("out", c_void),
    ]


class MerGateOptions(ctypes.Structure):
    """mer_gate_options (LinearGate::with_routing, gating.rs:207-268)."""
    _fields_ = [
        ("scoring", ctypes.c_int32),
        ("normalise_topk", ctypes.c_int32),
        ("correction_bias", ctypes.c_void_p),
        ("n_group", ctypes.c_uint32),
        ("topk_group", ctypes.c_uint32),
        ("routed_scaling_factor", ctypes.c_float),
    ]


class MerSlotStats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in
                ("hits", "misses", "prefetches", "evictions", "stale_retirements", "bytes_uploaded", "resident")]


class MerErrorInfo(ctypes.Structure):
    _fields_ = [
        ("status", ctypes.c_int32),
        ("have", ctypes.c_uint64),
        ("need", ctypes.c_uint64),
        ("d_model", ctypes.c_uint64),
        ("d_ff", ctypes.c_uint64),
    ]


class MerUthProjection(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int32), ("weights", ctypes.c_uint32), ("offset", c_u64), ("len", c_u64)]


class MerUthInfo(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32), ("dtype", ctypes.c_int32), ("version", ctypes.c_uint32),
                ("flags", ctypes.c_uint32), ("shape_rank", ctypes.c_uint32), ("shape", ctypes.c_uint32 * 4),
                ("quant_scale_offset", ctypes.c_uint32), ("quant_scale_count", ctypes.c_uint32),
                ("d_model", ctypes.c_uint32), ("d_ff", ctypes.c_uint32), ("proj", MerUthProjection * 3),
                ("payload_offset", c_u64), ("payload_len", c_u64)]


class MerGgufMoeInfo(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int32), ("layout", ctypes.c_int32), ("d_model", c_u64), ("d_ff", c_u64),
                ("n_experts", c_u64), ("expert_bytes", c_u64)]


class Status(enum.IntEnum):
    OK = 0
    BUFFER_TOO_SMALL = 1
    MISALIGNED = 2
    COMPUTE = 3
    INVALID_LAYOUT = 4
    TRUNCATED_PAYLOAD = 5
    RESIDENCY_MISS = 16
    PHYSICAL_CAPACITY = 17
    UPLOAD = 18
    VALIDATION_DISPATCH = 19
    SUBMISSION = 20
    READBACK_CHANNEL = 21
    READBACK_MAP = 22
    DEVICE_LOST = 23
    RUNTIME_INVARIANT = 24
    UNSUPPORTED_DTYPE = 32
    SHAPE_EXCEEDS_WORKSPACE = 33
    NOT_INITIALIZED = 48
    WRONG_DEVICE = 49
    IO = 50


# name -> (restype, argtypes); exactly the symbols include/mer_hip.h declares.
SIGNATURES = {
    "mer_hip_abi_version": (c_int, []),
    "mer_hip_init": (c_int, [c_int]),
    "mer_hip_shutdown": (c_int, []),
    "mer_hip_stream_release": (c_int, [c_void]),
    "mer_set_swiglu_limit": (c_int, [c_float]),
    "mer_get_swiglu_limit": (c_float, []),
    "mer_last_error": (ctypes.c_char_p, []),
    "mer_last_error_info": (c_int, [ctypes.POINTER(MerErrorInfo)]),
    "mer_hip_take_device_status": (c_int, []),
    "mer_hip_stage_timing_enable": (c_int, [c_int]),
    "mer_hip_stage_timing_read": (c_int, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(c_u64)]),
    "mer_hip_decode_trace": (c_int, [c_void, c_size, ctypes.POINTER(c_u64)]),
    "mer_expert_weight_bytes": (c_size, [c_int, c_size, c_size]),
    "mer_output_digest": (c_int, [c_u64, ctypes.c_uint32, c_void, c_size, ctypes.POINTER(c_u64),
                                  ctypes.POINTER(c_float)]),
    "mer_validate_expert": (c_int, [c_int, c_size, c_size, c_size, c_size, c_size, c_size]),
    "mer_routed_expert_gpu_compatibility": (c_int, [c_int, c_size, c_size]),
    "mer_hip_dequantize": (c_int, [c_int, c_void, c_size, c_size, c_void, c_void]),
    "mer_hip_q4_0_matvec": (c_int, [c_void, c_size, c_size, c_size, c_size, c_void, c_void, c_void]),
    "mer_hip_expert_forward": (
        c_int, [c_int, c_void, c_size, c_void, c_size, c_size, c_size, c_void, c_size, c_void]),
    "mer_hip_expert_forward_qmm": (
        c_int, [c_void, c_size, c_void, c_size, c_size, c_size, c_void, c_size, c_void]),
    "mer_hip_expert_forward_host": (
        c_int, [c_int, c_void, c_size, c_void, c_size, c_size, c_size, c_void, c_size]),
    "mer_hip_moe_forward": (
        c_int, [c_int, c_size, c_size, c_size, c_size, c_void, c_size, c_void, c_void, c_void, c_void,
                ctypes.c_uint, c_void]),
    "mer_hip_moe_forward_noalloc": (
        c_int, [c_int, c_size, c_size, c_size, c_size, c_void, c_size, c_void, c_void, c_void, c_void,
                ctypes.c_uint, c_void]),
    "mer_hip_moe_grouped": (
        c_int, [c_int, c_size, c_size, c_size, c_size, c_void, c_size, c_void, c_void, c_void, c_void,
                ctypes.c_uint, c_void]),
    "mer_hip_expert_batch_f16": (
        c_int, [c_int, c_size, c_size, c_size, c_void, c_size, c_void, c_void, c_void, c_void]),
    "mer_hip_moe_forward_layers": (
        c_int, [c_int, c_size, c_size, c_size, c_size, c_size, ctypes.POINTER(MerLayerArgs), ctypes.c_uint, c_void]),
    "mer_hip_route_linear_gate": (
        c_int, [c_void, c_size, c_size, c_void, c_size, c_size, ctypes.POINTER(MerGateOptions), c_void, c_void, c_void,
                c_void]),
    "mer_slot_cache_create": (c_int, [c_int, c_size, c_size, c_size, c_size, ctypes.POINTER(c_void)]),
    "mer_slot_cache_destroy": (c_int, [c_void]),
    "mer_slot_cache_table": (c_void, [c_void]),
    "mer_slot_cache_prepare": (c_int, [c_void, c_void, c_void, c_void, c_size, c_void]),
    "mer_slot_cache_prefetch": (c_int, [c_void, c_void, c_void, c_void, c_size, c_void]),
    "mer_slot_cache_release": (c_int, [c_void, c_void]),
    "mer_slot_cache_stats": (c_int, [c_void, ctypes.POINTER(MerSlotStats)]),
    "mer_hip_host_alloc": (c_int, [c_size, ctypes.POINTER(c_void)]),
    "mer_hip_host_free": (c_int, [c_void]),
    "mer_hip_fill_synthetic": (
        c_int, [c_int, c_u64, c_u64, c_u64, c_u64, c_float, c_float, c_void, c_void]),
    "mer_uth_probe": (c_int, [c_void, c_size, c_size, ctypes.POINTER(MerUthInfo)]),
    "mer_uth_write_expert_header": (c_int, [c_int, c_size, c_size, c_size, c_void, c_size, ctypes.POINTER(c_size)]),
    "mer_gguf_open": (c_int, [ctypes.c_char_p, ctypes.POINTER(c_void)]),
    "mer_gguf_close": (c_int, [c_void]),
    "mer_gguf_moe_layer": (c_int, [c_void, c_size, ctypes.POINTER(MerGgufMoeInfo)]),
    "mer_gguf_read_expert": (c_int, [c_void, c_size, c_size, c_void, c_size]),
}

_lock = threading.Lock()
_lib = None
_initialised_device = None


def lib() -> ctypes.CDLL:
    """Load libmer_hip.so (raises if it has not been built)."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: the HIP extension must be built "
                    "(python __graft_entry__.py build) -- there is no CPU fallback")
            handle = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
        return _lib


def last_error() -> tuple[int, str, MerErrorInfo]:
    l = lib()
    info = MerErrorInfo()
    l.mer_last_error_info(ctypes.byref(info))
    msg = l.mer_last_error()
    return info.status, (msg.decode() if msg else ""), info


def ensure_init(device: int) -> None:
    """mer_hip_init once per process for the given device."""
    global _initialised_device
    if _initialised_device == device:
        return
    rc = lib().mer_hip_init(device)
    if rc != 0:
        from .errors import raise_for_status
        raise_for_status(rc)
    _initialised_device = device
