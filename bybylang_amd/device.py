"""Device buffers and typed entry points of libbybyhip.so for numpy callers (tests, bench).

Thin plumbing over the C ABI: every array goes to device memory the library allocates, every
compute call is one C entry point, and failures raise HipBackendError with the library's message.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _abi
from ._abi import BF16, F16, F32, MXFP4_KM, HipBackendError, HipUnsupported, check, load

__all__ = ["DeviceBuffer", "Q4Weights", "init", "device_info", "synchronize", "stream",
           "q4_matmul", "fp4km_tile_gemm", "mxfp4_gemm", "f16_tile_gemm", "program_dispatch",
           "tile_gemm_ready", "F32", "F16", "BF16", "MXFP4_KM", "HipBackendError",
           "HipUnsupported", "dtype_code", "np_dtype"]

_NP = {F32: np.float32, F16: np.float16, BF16: np.uint16}


def np_dtype(code: int):
    return _NP[code]


def dtype_code(dt) -> int:
    dt = np.dtype(dt)
    if dt == np.float32:
        return F32
    if dt == np.float16:
        return F16
    raise ValueError(f"no byhip dtype for {dt}")


def init(device: int = 0) -> None:
    check(load().byhip_init(device), "byhip_init")


def device_info() -> dict:
    info = _abi.DeviceInfo()
    check(load().byhip_device_info_get(C.byref(info)))
    return {f: (getattr(info, f).decode() if isinstance(getattr(info, f), bytes) else getattr(info, f))
            for f, _ in _abi.DeviceInfo._fields_}


def synchronize() -> None:
    check(load().byhip_synchronize())


def stream() -> int:
    return load().byhip_stream() or 0


class DeviceBuffer:
    """A device allocation of `nbytes` owned by the library (freed on close / garbage collection)."""

    def __init__(self, nbytes: int):
        p = C.c_void_p()
        check(load().byhip_alloc(int(nbytes), C.byref(p)), "byhip_alloc")
        self.ptr = p.value
        self.nbytes = int(nbytes)

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        buf = cls(max(a.nbytes, 1))
        buf.upload(a)
        return buf

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        if a.nbytes:
            check(load().byhip_upload(self.ptr, offset, a.ctypes.data, a.nbytes), "byhip_upload")

    def read(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        count = (self.nbytes - offset) // dtype.itemsize if count is None else int(count)
        out = np.empty(count, dtype=dtype)
        if out.nbytes:
            check(load().byhip_read(self.ptr, offset, out.ctypes.data, out.nbytes), "byhip_read")
        return out

    def zero(self) -> None:
        check(load().byhip_memset(self.ptr, 0, self.nbytes))

    def close(self) -> None:
        if self.ptr:
            lib = load()
            lib.byhip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Q4Weights:
    """Resident Q4 weights (residentUploadQ4, gpubackend.nim:2883-2919)."""

    def __init__(self, wq: np.ndarray, scales: np.ndarray, zeros: np.ndarray, K: int, N: int,
                 group_size: int, groups_per_row: int, wq_off: int = 0):
        wq = np.ascontiguousarray(wq, dtype=np.uint8)
        scales = np.ascontiguousarray(scales, dtype=np.float32)
        zeros = np.ascontiguousarray(zeros, dtype=np.float32)
        h = C.c_void_p()
        check(load().byhip_q4_resident_upload(wq.ctypes.data, wq.nbytes, wq_off, scales.ctypes.data,
                                              zeros.ctypes.data, K, N, group_size, groups_per_row,
                                              C.byref(h)), "byhip_q4_resident_upload")
        self.handle = h.value
        self.K, self.N, self.group_size, self.groups_per_row = K, N, group_size, groups_per_row

    def info(self) -> dict:
        i = _abi.Q4WInfo()
        check(load().byhip_q4_resident_info(self.handle, C.byref(i)))
        return {f: getattr(i, f) for f, _ in _abi.Q4WInfo._fields_}

    def unpack(self):
        codes = np.empty(self.N * self.K, dtype=np.uint8)
        ng = self.N * self.groups_per_row
        sc = np.empty(ng, dtype=np.float32)
        ze = np.empty(ng, dtype=np.float32)
        check(load().byhip_debug_unpack_q4(self.handle, codes.ctypes.data, sc.ctypes.data,
                                           ze.ctypes.data))
        return codes.reshape(self.N, self.K), sc, ze

    def close(self) -> None:
        if self.handle:
            load().byhip_q4_resident_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def q4_matmul(x: DeviceBuffer, x_dtype: int, w: Q4Weights, y: DeviceBuffer, y_dtype: int, M: int) -> None:
    check(load().byhip_q4_matmul(x.ptr, x_dtype, w.handle, y.ptr, y_dtype, M), "byhip_q4_matmul")


def q4_prepare(w: Q4Weights, M: int, x_dtype: int = F32) -> int:
    """byhip_q4_prepare: BYHIP_OK when a plan is in place, BYHIP_UNSUPPORTED when tuning is off or
    a session is open."""
    rc = load().byhip_q4_prepare(w.handle, M, x_dtype)
    if rc == _abi.BYHIP_UNSUPPORTED:
        return rc
    check(rc, "byhip_q4_prepare")
    return rc


def q4_plan_info(w: Q4Weights, M: int, x_dtype: int = F32):
    """(plan name, from the plan file) for these weights, or None when there is no plan."""
    name = C.create_string_buffer(64)
    cached = C.c_int(0)
    rc = load().byhip_q4_plan_info(w.handle, M, x_dtype, name, 64, C.byref(cached))
    if rc == _abi.BYHIP_UNSUPPORTED:
        return None
    check(rc, "byhip_q4_plan_info")
    return name.value.decode(), bool(cached.value)


def q4_plans_reset() -> None:
    check(load().byhip_q4_plans_reset(), "byhip_q4_plans_reset")


def q4_matmul_fused(mode: int, a: DeviceBuffer, ws, outs, res: DeviceBuffer = None,
                    gamma: DeviceBuffer = None, eps: float = 0.0) -> int:
    """The fused decode GEMV (byhip_q4_matmul_fused): returns BYHIP_OK, or BYHIP_UNSUPPORTED when
    the library does not take the combination (the caller then runs the unfused sequence)."""
    wp = (C.c_void_p * max(1, len(ws)))(*[w.handle for w in ws])
    op = (C.c_void_p * max(1, len(outs)))(*[o.ptr for o in outs])
    rc = load().byhip_q4_matmul_fused(mode, a.ptr, C.cast(wp, C.c_void_p), len(ws), C.cast(op, C.c_void_p),
                                      len(outs), res.ptr if res is not None else None, int(res is not None),
                                      gamma.ptr if gamma is not None else None, eps, int(gamma is not None))
    if rc == _abi.BYHIP_UNSUPPORTED:
        return rc
    check(rc, "byhip_q4_matmul_fused")
    return rc


def fp4km_tile_gemm(x: DeviceBuffer, x_dtype: int, blob: DeviceBuffer, scale_base: int,
                    lut: DeviceBuffer, lut_base: int, y: DeviceBuffer, y_dtype: int,
                    M: int, K: int, N: int) -> None:
    check(load().byhip_fp4km_tile_gemm(x.ptr, x_dtype, blob.ptr, blob.nbytes, scale_base, lut.ptr,
                                       lut.nbytes // 4, lut_base, y.ptr, y_dtype, M, K, N),
          "byhip_fp4km_tile_gemm")


def mxfp4_gemm(x: DeviceBuffer, w: DeviceBuffer, y: DeviceBuffer, y_dtype: int, M: int, K: int,
               N: int) -> None:
    check(load().byhip_mxfp4_gemm(x.ptr, w.ptr, y.ptr, y_dtype, M, K, N), "byhip_mxfp4_gemm")


def f16_tile_gemm(x: DeviceBuffer, x_dtype: int, w: DeviceBuffer, y: DeviceBuffer, y_dtype: int,
                  M: int, K: int, N: int) -> None:
    check(load().byhip_f16_tile_gemm(x.ptr, x_dtype, w.ptr, w.nbytes // 2, y.ptr, y_dtype, M, K, N),
          "byhip_f16_tile_gemm")


def program_dispatch(words, mem: DeviceBuffer, u8: DeviceBuffer | None, lut: DeviceBuffer | None,
                     inp: DeviceBuffer | None, rows: int = 0, mem_len: int | None = None) -> None:
    w = np.ascontiguousarray(words, dtype=np.uint32)
    wp = w.ctypes.data_as(C.POINTER(C.c_uint32))
    check(load().byhip_program_dispatch(
        wp, len(w), mem.ptr, mem.nbytes // 4 if mem_len is None else mem_len,
        u8.ptr if u8 else None, u8.nbytes if u8 else 0, lut.ptr if lut else None,
        lut.nbytes // 4 if lut else 0, inp.ptr if inp else None, inp.nbytes // 4 if inp else 0,
        rows), "byhip_program_dispatch")


def tile_gemm_ready(f16: bool, tensor_core: bool = True) -> bool:
    rc = load().byhip_tile_gemm_ready(int(f16), int(tensor_core))
    if rc < 0:
        check(rc, "byhip_tile_gemm_ready")
    return rc == 1
