"""ctypes binding of libmoe_stream.so (the C ABI in include/moe_stream.h).

The library must exist: there is no fallback path.  torch is imported first
so that the library binds to the HIP runtime torch already loaded (both
carry the soname libamdhip64.so.7).
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import torch  # noqa: F401  (load torch's HIP runtime before ours)

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libmoe_stream.so"

MOE_OK = 0
MOE_ERR_INVALID = -1
MOE_ERR_UNSUPPORTED = -2
MOE_ERR_HIP = -3
MOE_ERR_EXHAUSTED = -4
MOE_ERR_DEVICE = -5
MOE_ERR_TIMEOUT = -6

MOE_STACK_COOPERATIVE = 0
MOE_STACK_ORDINARY = 1

MOE_ACT_SWIGLU = 0
MOE_ACT_SWIGLU_CLAMP = 1
MOE_ROUTE_SOFTMAX_TOPK = 0
MOE_ROUTE_TOPK_SOFTMAX = 1
MAX_COMPONENTS = 12
MAX_TOPK = 16

# Every symbol declared in include/moe_stream.h.
EXPORTS = (
    "moe_version", "moe_last_error", "moe_component_bytes",
    "moe_ffn_decode_workspace", "moe_ffn_decode",
    "moe_ffn_decode_up", "moe_ffn_decode_down",
    "moe_ffn_decode_static_bytes", "moe_ffn_decode_static",
    "moe_ffn_grouped_workspace", "moe_ffn_grouped",
    "moe_route_workspace", "moe_route", "moe_slot_lookup",
    "moe_stack_workspace", "moe_stack_decode", "moe_stack_trace",
    "moe_fill_slots", "moe_host_alloc", "moe_host_free",
    "moe_event_create", "moe_event_destroy", "moe_event_record",
    "moe_event_query", "moe_stream_wait_event", "moe_event_elapsed_ms",
    "moe_check_device_error",
    "moe_policy_create", "moe_policy_destroy", "moe_policy_prefetch",
    "moe_policy_acquire", "moe_policy_complete", "moe_policy_cancel", "moe_policy_lookup",
    "moe_policy_is_pending", "moe_policy_table", "moe_policy_stats",
    "moe_engine_create", "moe_engine_destroy", "moe_engine_layer", "moe_engine_layer_depths",
    "moe_engine_counters",
)

MOE_EVICT_LFU = 0
MOE_EVICT_LRU = 1
MOE_EVICT_ASIS = 2


class MoeError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class Geom(C.Structure):
    _fields_ = [("d_model", C.c_int32), ("d_ff", C.c_int32),
                ("group_size", C.c_int32), ("bits", C.c_int32),
                ("has_proj_bias", C.c_int32), ("act", C.c_int32),
                ("alpha", C.c_float), ("limit", C.c_float)]


class PoolView(C.Structure):
    _fields_ = [("n_components", C.c_int32), ("n_slots", C.c_int32),
                ("base", C.c_void_p * MAX_COMPONENTS),
                ("slot_bytes", C.c_int64 * MAX_COMPONENTS),
                ("store", C.c_void_p), ("record_bytes", C.c_int64),
                ("n_records", C.c_int64),
                ("comp_offset", C.c_int64 * MAX_COMPONENTS)]


_lib = None


def _declare(lib):
    P, I32, I64, SZ, F = C.c_void_p, C.c_int32, C.c_int64, C.c_size_t, C.c_float
    sig = {
        "moe_version": (C.c_int, []),
        "moe_last_error": (C.c_char_p, []),
        "moe_component_bytes": (C.c_int, [C.POINTER(Geom), P]),
        "moe_ffn_decode_workspace": (SZ, [C.POINTER(Geom), I32, I32]),
        "moe_ffn_decode": (C.c_int, [C.POINTER(PoolView), C.POINTER(Geom), P, P, P,
                                     I32, I32, P, P, P, SZ, P]),
        "moe_ffn_decode_static_bytes": (SZ, []),
        "moe_ffn_decode_static": (C.c_int, [C.POINTER(PoolView), C.POINTER(Geom), P, P, P,
                                            I32, I32, P, P, P]),
        "moe_ffn_decode_up": (C.c_int, [C.POINTER(PoolView), C.POINTER(Geom), P, P,
                                        I32, I32, P, SZ, P]),
        "moe_ffn_decode_down": (C.c_int, [C.POINTER(PoolView), C.POINTER(Geom), P, P,
                                          I32, I32, P, P, P, SZ, P]),
        "moe_ffn_grouped_workspace": (SZ, [C.POINTER(Geom), I32, I32]),
        "moe_ffn_grouped": (C.c_int, [C.POINTER(PoolView), C.POINTER(Geom), P, P, P,
                                      I32, I32, P, P, P, SZ, P]),
        "moe_route_workspace": (SZ, [I32, I32]),
        "moe_route": (C.c_int, [P, I32, I32, P, P, I32, I32, I32, I32, P, P,
                                P, P, I32, P, P, P, P, P, SZ, P]),
        "moe_slot_lookup": (C.c_int, [P, I32, P, I32, P, P, P]),
        "moe_stack_workspace": (SZ, [C.POINTER(Geom), I32, I32, I32]),
        "moe_stack_trace": (C.c_int, [P, SZ]),
        "moe_stack_decode": (C.c_int, [C.POINTER(PoolView), C.POINTER(Geom), I32, I32, I32,
                                       P, P, P, I32, I32, I32, P, P, P, P, P, P, P,
                                       C.c_uint32, I32, P, SZ, P]),
        "moe_fill_slots": (C.c_int, [C.POINTER(PoolView), P, I64, I64, P, P, I32, P]),
        "moe_host_alloc": (C.c_int, [SZ, C.POINTER(C.c_void_p)]),
        "moe_host_free": (C.c_int, [P]),
        "moe_event_create": (C.c_int, [C.POINTER(C.c_void_p)]),
        "moe_event_destroy": (C.c_int, [P]),
        "moe_event_record": (C.c_int, [P, P]),
        "moe_event_query": (C.c_int, [P]),
        "moe_stream_wait_event": (C.c_int, [P, P]),
        "moe_event_elapsed_ms": (C.c_int, [P, P, C.POINTER(F)]),
        "moe_check_device_error": (C.c_int, [P]),
        "moe_policy_create": (C.c_int, [I32, I32, I32, I32, I32, C.POINTER(C.c_void_p)]),
        "moe_policy_destroy": (C.c_int, [P]),
        "moe_policy_prefetch": (C.c_int, [P, I32, P, I32, P, P, P]),
        "moe_policy_acquire": (C.c_int, [P, I32, P, I32, P, P, P, P, P]),
        "moe_policy_complete": (C.c_int, [P, I32, I32]),
        "moe_policy_cancel": (C.c_int, [P, I32, I32]),
        "moe_policy_lookup": (C.c_int, [P, I32, I32]),
        "moe_policy_is_pending": (C.c_int, [P, I32, I32]),
        "moe_policy_table": (C.c_int, [P, P]),
        "moe_policy_stats": (C.c_int, [P, P]),
        "moe_engine_create": (C.c_int, [C.POINTER(PoolView), C.POINTER(Geom), I32, I32, I32,
                                        I32, P, P, I64, I64, P, P, C.POINTER(C.c_void_p)]),
        "moe_engine_destroy": (C.c_int, [P]),
        "moe_engine_layer": (C.c_int, [P, I32, P, P, P, I32, I32, P, P, P]),
        "moe_engine_layer_depths": (C.c_int, [P, I32, P, P, P, I32, I32, P, I32, P, P, P]),
        "moe_engine_counters": (C.c_int, [P, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m moe_stream_amd.build` "
                "(there is no CPU fallback for the expert hot path)")
        l = C.CDLL(str(LIB_PATH))
        _declare(l)
        _lib = l
    return _lib


def check(rc: int) -> int:
    if rc < 0:
        raise MoeError(rc, lib().moe_last_error().decode(errors="replace"))
    return rc


def stream_ptr(stream=None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)
