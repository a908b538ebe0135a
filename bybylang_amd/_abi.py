"""ctypes declarations of libbybyhip.so (include/byhip.h).

Loading fails loudly: there is no other implementation of these entry points to fall back to.
"""
from __future__ import annotations

import ctypes as C
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libbybyhip.so")

BYHIP_OK = 0
BYHIP_UNSUPPORTED = 1
BYHIP_ERROR = -1

F32, F16, BF16, MXFP4_KM = 0, 1, 2, 3


class HipBackendError(RuntimeError):
    """A failure reported by libbybyhip.so (its byhip_last_error text)."""


class HipUnsupported(HipBackendError):
    """BYHIP_UNSUPPORTED: the entry point does not handle this shape or device."""


class DeviceInfo(C.Structure):
    _fields_ = [("device", C.c_int), ("compute_units", C.c_int), ("wavefront_size", C.c_int),
                ("clock_khz", C.c_int), ("memory_clock_khz", C.c_int),
                ("memory_bus_width", C.c_int), ("total_global_mem", C.c_size_t),
                ("lds_bytes_per_block", C.c_size_t), ("arch_name", C.c_char * 64),
                ("name", C.c_char * 128)]


class Q4WInfo(C.Structure):
    _fields_ = [("K", C.c_int), ("N", C.c_int), ("group_size", C.c_int),
                ("groups_per_row", C.c_int), ("scale_is_f16", C.c_int),
                ("zero_uniform", C.c_int), ("zero_value", C.c_float),
                ("device_bytes", C.c_size_t), ("f16_safe", C.c_int)]


_VP, _SZ, _I, _U8P, _FP = C.c_void_p, C.c_size_t, C.c_int, C.c_void_p, C.c_void_p

# name: (restype, argtypes), in the order of include/byhip.h
SIGNATURES = {
    "byhip_init": (_I, [_I]),
    "byhip_device_info_get": (_I, [C.POINTER(DeviceInfo)]),
    "byhip_last_error": (C.c_char_p, []),
    "byhip_clear_error": (None, []),
    "byhip_fault_inject": (None, [_I]),
    "byhip_version": (_I, []),
    "byhip_alloc": (_I, [_SZ, C.POINTER(_VP)]),
    "byhip_free": (_I, [_VP]),
    "byhip_upload": (_I, [_VP, _SZ, _VP, _SZ]),
    "byhip_read": (_I, [_VP, _SZ, _VP, _SZ]),
    "byhip_memset": (_I, [_VP, _I, _SZ]),
    "byhip_synchronize": (_I, []),
    "byhip_stream": (_VP, []),
    "byhip_session_begin": (_I, []),
    "byhip_session_upload": (_I, [_FP, _SZ, C.POINTER(_VP)]),
    "byhip_session_upload_bytes": (_I, [_VP, _SZ, C.POINTER(_VP)]),
    "byhip_session_alloc_scratch": (_I, [_SZ, C.POINTER(_VP)]),
    "byhip_session_end": (_I, []),
    "byhip_session_commit_continue": (_I, []),
    "byhip_session_recover": (_I, []),
    "byhip_session_read": (_I, [_VP, _FP, _SZ]),
    "byhip_session_free": (_I, [_VP]),
    "byhip_session_set_gpu_timing": (_I, [_I]),
    "byhip_session_gpu_seconds": (C.c_double, []),
    "byhip_session_can_record": (_I, []),
    "byhip_session_begin_recording": (_I, []),
    "byhip_session_last_recording": (_I, []),
    "byhip_session_replay": (_I, [_I, _I]),
    "byhip_session_replay_after": (_I, [_I, _I, _I, _I]),
    "byhip_session_mark": (_I, [_I]),
    "byhip_session_replay_marked": (_I, [_I]),
    "byhip_session_take_marks": (_I, []),
    "byhip_session_free_recording": (_I, [_I]),
    "byhip_session_set_direct_replay": (_I, [_I]),
    "byhip_debug_alloc_count": (C.c_ulonglong, []),
    "byhip_q4_resident_upload": (_I, [_U8P, _SZ, _SZ, _FP, _FP, _I, _I, _I, _I, C.POINTER(_VP)]),
    "byhip_q4_resident_from_device": (_I, [_VP, _SZ, _VP, _VP, _I, _I, _I, _I, C.POINTER(_VP)]),
    "byhip_q4_resident_free": (_I, [_VP]),
    "byhip_q4_resident_info": (_I, [_VP, C.POINTER(Q4WInfo)]),
    "byhip_q4_matmul": (_I, [_VP, _I, _VP, _VP, _I, _I]),
    "byhip_q4_matmul_static": (_I, [_VP, _I, _VP, _VP, _I, _I]),
    "byhip_q4_matmul_fused": (_I, [_I, _FP, _VP, _I, _VP, _I, _FP, _I, _FP, C.c_float, _I]),
    "byhip_q4_prepare": (_I, [_VP, _I, _I]),
    "byhip_q4_plan_info": (_I, [_VP, _I, _I, C.c_char_p, _I, C.POINTER(_I)]),
    "byhip_q4_plans_reset": (_I, []),
    "byhip_gpu_matmul_q4": (_I, [_FP, _U8P, _FP, _FP, _FP, _I, _I, _I, _I, _I]),
    "byhip_fp4km_tile_gemm": (_I, [_VP, _I, _U8P, _SZ, _SZ, _FP, _SZ, _SZ, _VP, _I, _I, _I, _I]),
    "byhip_mxfp4_gemm": (_I, [_U8P, _U8P, _VP, _I, _I, _I, _I]),
    "byhip_f16_tile_gemm": (_I, [_VP, _I, _VP, _SZ, _VP, _I, _I, _I, _I]),
    "byhip_tile_gemm_ready": (_I, [_I, _I]),
    "byhip_program_dispatch": (_I, [C.POINTER(C.c_uint32), _I, _VP, _SZ, _VP, _SZ, _VP, _SZ,
                                    _VP, _SZ, _I]),
    "byhip_debug_unpack_q4": (_I, [_VP, _U8P, _FP, _FP]),
    "byhip_debug_unpack_fp4km": (_I, [_U8P, _SZ, _FP, _SZ, _I, _I, _U8P, _FP]),
    "byhip_debug_copy": (_I, [_VP, _VP, _SZ]),
    "byhip_debug_read": (_I, [_VP, _SZ, _VP, _SZ]),
}

_lib = None


def load(path: str = LIB_PATH) -> C.CDLL:
    """Loads libbybyhip.so once; raises HipBackendError when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise HipBackendError(
            f"{path} is missing: build it with `python -m bybylang_amd.build` (hipcc, gfx950). "
            "The HIP backend has no other implementation to fall back to.")
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    return (load().byhip_last_error() or b"").decode(errors="replace")


def check(rc: int, what: str = "") -> int:
    """Raises on BYHIP_ERROR / BYHIP_UNSUPPORTED with the library's message."""
    if rc == BYHIP_OK:
        return rc
    msg = last_error() or f"{what} failed with {rc}"
    if rc == BYHIP_UNSUPPORTED:
        raise HipUnsupported(msg)
    raise HipBackendError(msg)
