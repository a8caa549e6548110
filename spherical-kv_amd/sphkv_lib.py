"""ctypes binding of libsphkv.so (the C ABI declared in include/sphkv.h).

Loads the in-tree library built by `make -C spherical-kv_amd`.  There is no
fallback: if the library is missing or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libsphkv.so")
_lib = None
_lock = threading.Lock()

P = ctypes.c_void_p
I32 = ctypes.c_int32
I64 = ctypes.c_int64
F32 = ctypes.c_float
F64 = ctypes.c_double

# name -> (restype, argtypes); must match include/sphkv.h
SIGNATURES = {
    "sphkv_last_error": (ctypes.c_char_p, []),
    "sphkv_version": (ctypes.c_char_p, []),
    "sphkv_encode_pages": (ctypes.c_int, [P, I32, P, I64, P, P, P, P, P, P, I32, I32, P, P, P,
                                          P, I64, P, I64, P, P, I32, I32, P]),
    "sphkv_encode_codes": (ctypes.c_int, [P, I32, I64, P, P, P, P, P, I32, I32, P, P, P, P, P, I32, I32, P]),
    "sphkv_decode_paged_workspace_bytes": (I64, [I32, I32, I32]),
    "sphkv_decode_paged": (ctypes.c_int, [P, I64, P, P, P, I32, P, I64, P, P, P, P, I32, P,
                                          I32, I32, I32, P, P, P, I64, I32, I32, F32, F64, P]),
    "sphkv_decode_paged_partials": (ctypes.c_int, [P, I64, P, P, P, I32, P, I64, P, P, P, P, I32, P,
                                                   I32, I32, I32, P, P, I64, I32, I32, F32, F64, P]),
    "sphkv_decode_merge_partials": (ctypes.c_int, [P, I64, I32, P, I32, I32, I32, I32, P, P]),
    "sphkv_decode_paged_status": (ctypes.c_int, [P, I64, I32, I32, I32, P, P]),
    "sphkv_decode_paged_noalloc": (ctypes.c_int, [P, I64, P, P, P, I32, P, I64, P, P, P, P, I32, P,
                                                  I32, I32, I32, P, P, I32, I32, F32, F64, P]),
    "sphkv_decode_paged_checked": (ctypes.c_int, [P, I64, P, P, P, I32, P, I64, P, P, P, P, I32, P,
                                                  I32, I32, I32, P, P, P, I64, I32, I32, F32, F64, P]),
    "sphkv_time_next_decode_kernel": (ctypes.c_int, [P, P]),
    "sphkv_step_plan_create": (ctypes.c_int, [P, I64, P, P, P, I32, P, I64, P, P, P, P, I32, P, I32, I32, I32,
                                              P, P, P, P, P, I64, I32, I32, I32, I32, I32, P, I64, I32, I32, F32,
                                              F64, P]),
    "sphkv_step_plan_run": (ctypes.c_int, [P, P, P, I32, P, P, P, I32, P]),
    "sphkv_step_plan_counts": (ctypes.c_int, [P, P, P, P]),
    "sphkv_step_plan_destroy": (None, [P]),
    "sphkv_tail_relayout": (ctypes.c_int, [P, I32, I32, P, P, P, I32, I64, I32, I32, P, P, P, P]),
    "sphkv_decode_step": (ctypes.c_int, [P, I64, P, P, P, I32, P, I64, P, P, P, P, I32, P, I32, I32, I32,
                                         P, P, I32, P, P, P, P, P, P, P, I64, I32, I32, I32, I32, P, P, I64,
                                         I32, I32, F32, F64, P]),
    "sphkv_decode_append": (ctypes.c_int, [P, I64, P, I32, P, I64, P, P, I32, P, I32, I32, P, I32, P, P,
                                           P, P, P, P, P, I64, I32, I32, I32, I32, I32, P]),
    "sphkv_fused_decode_ragged": (ctypes.c_int, [P, I64, P, P, P, I32, P, P, I32, P, I32, I32, P,
                                                 I32, I32, I32, I32, I32, P, P]),
    "sphkv_fused_decode_ragged_fitted": (ctypes.c_int, [P, I64, P, P, P, I32, P, P, I32, P, I32, I32, P,
                                                        I32, I32, I32, I32, I32, P, I32, P, P]),
    "sphkv_rope_table_fit": (ctypes.c_int, [P, P, I32, I32, P, P, P, P]),
    "sphkv_decode_plan_create": (ctypes.c_int, [P, I64, P, P, P, I32, P, I64, P, P, P, P, I32, P, I32, I32, I32,
                                                P, I64, I32, I32, F32, F64, P]),
    "sphkv_decode_plan_run": (ctypes.c_int, [P, P, P, P]),
    "sphkv_decode_plan_destroy": (None, [P]),
    "sphkv_encode_append": (ctypes.c_int, [P, P, P, P, P, P, P, P, I32, I64, I32, I32, I32, I32, I32,
                                           I32, I32, I32, P]),
    "sphkv_decode_modea": (ctypes.c_int, [P, P, P, P, P, P, P, P, I64, P, P, P, P, P, I32, I32, I32, I32,
                                          I32, I32, I32, I32, I32, I32, F32, I32, P]),
    "sphkv_q_lut": (ctypes.c_int, [P, P, P, P, I32, I32, I32, I32, I32, I32, I32, I32, P, P]),
    "sphkv_logits_lut": (ctypes.c_int, [P, P, P, P, I64, P, P, P, P, I32, I32, I32, I32, I32, I32, I32,
                                        I32, F32, I32, P]),
    "sphkv_omega_ema": (ctypes.c_int, [P, P, I64, I64, P, P, I32, I32, I32, F32, P]),
    "sphkv_plan_pages_work_ints": (I64, [I32, I32, I32]),
    "sphkv_plan_pages_count": (ctypes.c_int, [P, I64, P, I32, I32, I32, I32, P, I64, P, P, P]),
    "sphkv_plan_pages_fill": (ctypes.c_int, [P, I64, P, P, I64, P, I32, I32, I32, I32, P, I32, P, P, P, P, P, P, P,
                                             P, P]),
    "sphkv_build_layer_pool": (ctypes.c_int, [P, P, I64, P, I64, P, I32, I32, P, P, P, P, I64, I32, I32, I32,
                                              P]),
    "sphkv_work_rows_per_item": (I32, [P, I32, I32, I32]),
    "sphkv_work_fill": (I64, [P, I32, I32, I32, P, I64, P]),
}


class SphkvError(RuntimeError):
    pass


def load():
    """Return the loaded library; raise SphkvError if it is not there."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise SphkvError(f"libsphkv.so not found at {LIB_PATH}; build it with "
                                 f"`make -C {_HERE}` (or __graft_entry__.build())")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


_raw_stream = None


def current_stream() -> int:
    """Raw handle of torch's current stream on the current device: every
    launch of this package goes to it.  Uses torch's raw accessor where this
    torch build has it (no Stream object built per launch)."""
    global _raw_stream
    import torch
    if _raw_stream is None:
        _raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", False)
    if _raw_stream:
        return _raw_stream(torch.cuda.current_device())
    return torch.cuda.current_stream().cuda_stream


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().sphkv_last_error().decode(errors="replace")
        raise SphkvError(f"{what} failed ({rc}): {msg}")


def version() -> str:
    return load().sphkv_version().decode()
