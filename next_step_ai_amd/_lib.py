"""ctypes binding of ``libnsmlp.so`` (declared in include/nsmlp.h).

The library is built in-tree by ``python -m next_step_ai_amd.build_lib``.
There is no fallback: if the library is missing or fails to load, every
entry point raises ``RuntimeError``.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libnsmlp.so")

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

P = ctypes.c_void_p
I32 = ctypes.c_int
I64 = ctypes.c_longlong
U64 = ctypes.c_uint64
F32 = ctypes.c_float
SZ = ctypes.c_size_t

NSMLP_ROUTE_SORTED = 1
NSMLP_ROUTE_LEGACY_ABS = 2
NSMLP_DOWN_BLOCK_MAJOR = 0
NSMLP_DOWN_GATHERED = 1
NSMLP_CACHE_GROW_ONLY = 1
NSMLP_STATUS_BLOCK_UNAVAILABLE = 1
NSMLP_STATUS_FIXED_RANGE = 2


class SlotTable(ctypes.Structure):
    """Mirror of ``nsmlp_slot_table``."""

    _fields_ = [
        ("H", I32), ("I", I32), ("qbs", I32), ("n_slots", I32),
        ("lookup", P),
        ("gate_packed", P), ("gate_absmax", P),
        ("up_packed", P), ("up_absmax", P),
        ("down_packed", P), ("down_absmax", P),
        ("host_gate_packed", P), ("host_gate_absmax", P),
        ("host_up_packed", P), ("host_up_absmax", P),
        ("host_down_packed", P), ("host_down_absmax", P),
        ("code", P),
        ("down_bias", P),
        ("dq_block", I32),
        ("gate_qabsmax", P), ("up_qabsmax", P), ("down_qabsmax", P),
        ("host_gate_qabsmax", P), ("host_up_qabsmax", P), ("host_down_qabsmax", P),
        ("gate_absmax2", P), ("up_absmax2", P), ("down_absmax2", P),
        ("gate_code2", P), ("up_code2", P), ("down_code2", P),
        ("gate_offset", F32), ("up_offset", F32), ("down_offset", F32),
    ]


class Router(ctypes.Structure):
    """Mirror of ``nsmlp_router``."""

    _fields_ = [
        ("R", I32), ("basis_top_k", I32), ("NB", I32), ("flags", I32),
        ("enc_w", P), ("enc_b", P), ("score_w", P), ("score_b", P), ("down_block_norm", P),
    ]


class Nf4Matrix(ctypes.Structure):
    """Mirror of ``nsmlp_nf4_matrix``."""

    _fields_ = [
        ("out_features", I32), ("in_features", I32), ("qbs", I32), ("packed", P), ("absmax", P), ("code", P),
        ("dq_block", I32), ("qabsmax", P), ("absmax2", P), ("code2", P), ("offset", F32),
    ]


class CacheState(ctypes.Structure):
    """Mirror of ``nsmlp_cache_state``."""

    _fields_ = [("capacity", I32), ("lookup", P), ("slot_block", P), ("slot_score", P), ("active_count", P)]


# name -> (restype, argtypes)
SIGNATURES: dict[str, tuple] = {
    "nsmlp_last_error": (ctypes.c_char_p, []),
    "nsmlp_version": (I32, []),
    "nsmlp_device_supported": (I32, [I32]),
    "nsmlp_fault_inject": (I32, [ctypes.c_char_p]),
    "nsmlp_workspace_init": (I32, [P, SZ, P]),
    "nsmlp_workspace_take_status": (I32, [P, P, P]),
    "nsmlp_workspace_take_block_counts": (I32, [P, P, P]),
    "nsmlp_route_workspace_bytes": (SZ, [I32, I32, I32, I32, I32]),
    "nsmlp_route_f16": (I32, [P, I32, I32, P, P, I32, I32, P, P, P, I32, I32, I32, P, P, P, P, SZ, P]),
    "nsmlp_decode_workspace_bytes": (SZ, [I32, I32]),
    "nsmlp_decode_slots_f16": (I32, [ctypes.POINTER(SlotTable), P, P, I32, P, P, SZ, P]),
    "nsmlp_decode_slots_add_f16": (I32, [ctypes.POINTER(SlotTable), P, P, P, I32, P, P, SZ, P]),
    "nsmlp_layer_workspace_bytes": (SZ, [I32, I32, I32, I32]),
    "nsmlp_decode_layer_f16": (I32, [ctypes.POINTER(Router), ctypes.POINTER(SlotTable), P, I32, P, P, P, SZ, P]),
    "nsmlp_decode_layer_add_f16": (I32, [ctypes.POINTER(Router), ctypes.POINTER(SlotTable), P, P, I32, P, P, P, SZ,
                                         P]),
    "nsmlp_decode_layer_noalloc_f16": (I32, [ctypes.POINTER(Router), ctypes.POINTER(SlotTable), P, P, I32, P, P, P,
                                             P]),
    "nsmlp_prefill_workspace_bytes": (SZ, [I32, I32, I32, I32]),
    "nsmlp_prefill_slots_f16": (I32, [ctypes.POINTER(SlotTable), P, I32, P, I32, P, P, SZ, P]),
    "nsmlp_dense_mlp_workspace_bytes": (SZ, [I32, I32, I32]),
    "nsmlp_dense_mlp_slots_f16": (I32, [ctypes.POINTER(SlotTable), P, I32, P, P, P, SZ, P]),
    "nsmlp_single_kernel_workspace_bytes": (SZ, [I32, I32]),
    "nsmlp_single_kernel_decode_f16": (I32, [P, P, P, P, P, P, P, P, P, P, P, P, I32, I32, I32, I32, P, SZ, P]),
    "nsmlp_fused_decode_workspace_bytes": (SZ, [I32, I32]),
    "nsmlp_fused_decode_gathered_f16": (I32, [P, I32, P, I32, I32, P, P, P, P, P, P, P, P, P, P, P, P, P, I32, P, P, SZ, P]),
    "nsmlp_output_linear_workspace_bytes": (SZ, [I32, I32, I32]),
    "nsmlp_output_linear_nf4_f16": (I32, [P, I32, I32, P, I32, I32, P, P, P, P, I32, P, I32, P, P, SZ, P]),
    "nsmlp_input_linear_nf4_f16": (I32, [P, I32, I32, P, I32, P, P, P, I32, I32, P, I32, P, P]),
    "nsmlp_dense_linear_nf4_f16": (I32, [ctypes.POINTER(Nf4Matrix), P, I32, P, P, P]),
    "nsmlp_silu_mul_f16": (I32, [P, P, P, I64, P]),
    "nsmlp_gather_row_blocks": (I32, [P, P, I32, P, I32, I32, I32, P, P, P]),
    "nsmlp_gather_down_columns": (I32, [P, P, P, I32, I32, I32, I32, I32, P, P, P]),
    "nsmlp_gather_row_blocks_q8": (I32, [P, P, I32, P, I32, I32, I32, P, P, P]),
    "nsmlp_gather_down_columns_q8": (I32, [P, P, P, I32, I32, I32, I32, I32, P, P, P]),
    "nsmlp_absmax_dq_quantize": (I32, [P, I64, I32, P, F32, P, P, P]),
    "nsmlp_absmax_dq_dequantize": (I32, [P, I64, I32, P, P, F32, P, P]),
    "nsmlp_cache_workspace_bytes": (SZ, [I32]),
    "nsmlp_cache_promote": (I32, [ctypes.POINTER(SlotTable), ctypes.POINTER(CacheState), P, I32, I32, P, P, SZ, P]),
    "nsmlp_cache_record_f32": (I32, [P, I32, P, I32, I32, P, P]),
    "nsmlp_host_device_pointer": (I32, [P, ctypes.POINTER(P)]),
    "nsmlp_synth_normal_f16": (I32, [U64, I64, F32, P, P]),
    "nsmlp_synth_normal_f32": (I32, [U64, I64, F32, P, P]),
    "nsmlp_synth_nf4": (I32, [U64, I64, I32, F32, P, P, P]),
    "nsmlp_nf4_quantize_f32": (I32, [P, I64, I32, P, P, P]),
}


def lib() -> ctypes.CDLL:
    """Load the library once; raise RuntimeError when it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m next_step_ai_amd.build_lib` "
                "(there is no CPU fallback)"
            )
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def last_error() -> str:
    msg = lib().nsmlp_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed (status {rc}): {last_error()}")


def call(name: str, *args) -> None:
    """Call a status-returning entry point; raise RuntimeError on failure."""
    rc = getattr(lib(), name)(*args)
    check(int(rc), name)


def fault_inject(spec: str | None) -> None:
    """Arm (or, with None or "", disarm) the library's fault injection: the
    compute entry points named in ``spec`` ("name=kind[:count],...", names
    without the nsmlp_ prefix or ``*``; kind oom, hip, inval, nospc or nodev)
    fail before they touch the device, so the drop-ins raise RuntimeError as
    on a real failure.  Process-wide; see nsmlp_fault_inject in nsmlp.h."""
    check(int(lib().nsmlp_fault_inject(None if not spec else spec.encode())), "nsmlp_fault_inject")


class injected_faults:
    """Context manager: ``with injected_faults("single_kernel_decode_f16=hip:3"):``
    arms the spec and disarms it on exit."""

    def __init__(self, spec: str):
        self.spec = spec

    def __enter__(self):
        fault_inject(self.spec)
        return self

    def __exit__(self, *exc):
        fault_inject(None)
        return False
