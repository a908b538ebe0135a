"""The reference's GPU dispatch / session API for the quantized tile-GEMM path, on the HIP backend.

Same names, argument meaning and error behaviour as bobbyshop-vui/bybylang's gpubackend.nim for the
procs on this path, with `gbHip` added to GpuBackend. Every call goes to libbybyhip.so through its C
ABI; nothing here computes on the CPU. Where the reference falls back to CPU after a GPU failure
(handleGpuFailure, gpubackend.nim:80-105), this module raises when CPU fallback is forbidden and
otherwise calls the fallback the caller passes in (the reference's own CPU path), never one of its
own.
"""
from __future__ import annotations

import ctypes as C
import enum
import os
import sys
from dataclasses import dataclass, field

import numpy as np

from . import _abi
from ._abi import HipBackendError, HipUnsupported, check, load

# ── backend selection (gpubackend.nim:55-57, 75-78, 107-129) ─────────────────────────────────


class GpuBackend(enum.Enum):
    gbAuto = "auto"
    gbCpu = "cpu"
    gbCuda = "cuda"
    gbMetal = "metal"
    gbVulkan = "vulkan"
    gbHip = "hip"

    def __str__(self) -> str:
        return self.value


gbAuto, gbCpu, gbCuda, gbMetal, gbVulkan, gbHip = (GpuBackend.gbAuto, GpuBackend.gbCpu,
                                                   GpuBackend.gbCuda, GpuBackend.gbMetal,
                                                   GpuBackend.gbVulkan, GpuBackend.gbHip)

gForbidCpuFallback = False


def setForbidCpuFallback(forbid: bool) -> None:
    """setForbidCpuFallback, gpubackend.nim:77-78."""
    global gForbidCpuFallback
    gForbidCpuFallback = bool(forbid)


def parseBackend(s: str) -> GpuBackend:
    """parseBackend, gpubackend.nim:107-114, with "hip" added."""
    v = s.strip().lower()
    table = {"cuda": gbVulkan, "metal": gbMetal, "cpu": gbCpu, "vulkan": gbVulkan,
             "auto": gbAuto, "hip": gbHip}
    if v not in table:
        raise ValueError("unknown BybyLang backend: " + s)
    return table[v]


def _require_hip(backend: GpuBackend) -> None:
    if backend != gbHip:
        raise ValueError(f"this module drives the hip backend only, not '{backend}'")


_device_ready = False


def ensureGpuInit(backend: GpuBackend = gbHip, device: int = 0) -> bool:
    """Initialises the HIP device once (the reference's ensureGpuInit); False if unavailable."""
    global _device_ready
    _require_hip(backend)
    if _device_ready:
        return True
    rc = load().byhip_init(device)
    _device_ready = rc == _abi.BYHIP_OK
    return _device_ready


def handleGpuFailure(backend: GpuBackend, opName: str, e: Exception) -> None:
    """handleGpuFailure, gpubackend.nim:80-105: report, then raise under forbid."""
    msg = f"[GPU] backend '{backend}' failed during '{opName}' ({e})"
    sys.stderr.write(msg + "\n")
    if gForbidCpuFallback:
        raise HipBackendError(msg + ". CPU fallback is forbidden (gForbidCpuFallback=true). "
                              "Call setForbidCpuFallback(false) to allow automatic CPU fallback.") from e
    sys.stderr.write("[GPU] falling back to CPU for this operation. Will retry GPU on next operation.\n")


# ── session (gpubackend.nim:894-903 and the lifecycle procs) ───────────────────────────────


@dataclass
class SessionHandle:
    kind: GpuBackend = gbCpu
    hipHandle: int | None = None      # device pointer owned by libbybyhip.so
    probeBytes: int = 0
    extra: dict = field(default_factory=dict)


def sessionBegin(backend: GpuBackend) -> bool:
    """sessionBegin, gpubackend.nim:1042: False when a session is already open or on failure."""
    _require_hip(backend)
    return ensureGpuInit(backend) and load().byhip_session_begin() == _abi.BYHIP_OK


def sessionUpload(backend: GpuBackend, data) -> SessionHandle:
    """sessionUpload, gpubackend.nim:1133 (fp32 data; packed bytes travel as float bit copies)."""
    _require_hip(backend)
    a = np.ascontiguousarray(data, dtype=np.float32)
    p = C.c_void_p()
    check(load().byhip_session_upload(a.ctypes.data, a.size, C.byref(p)), "sessionUpload")
    return SessionHandle(gbHip, p.value, a.nbytes)


def sessionUploadBytes(backend: GpuBackend, data) -> SessionHandle:
    _require_hip(backend)
    a = np.ascontiguousarray(data, dtype=np.uint8)
    p = C.c_void_p()
    check(load().byhip_session_upload_bytes(a.ctypes.data, a.nbytes, C.byref(p)), "sessionUploadBytes")
    return SessionHandle(gbHip, p.value, a.nbytes)


def sessionAllocScratch(backend: GpuBackend, n: int) -> SessionHandle:
    """sessionAllocScratch, gpubackend.nim:1295: `n` floats, zeroed."""
    _require_hip(backend)
    p = C.c_void_p()
    check(load().byhip_session_alloc_scratch(int(n), C.byref(p)), "sessionAllocScratch")
    return SessionHandle(gbHip, p.value, int(n) * 4)


def sessionEnd(backend: GpuBackend) -> bool:
    """sessionEnd, gpubackend.nim:2422: waits; False on a device error (see sessionGetLastError)."""
    _require_hip(backend)
    return load().byhip_session_end() == _abi.BYHIP_OK


def sessionCommitContinue(backend: GpuBackend) -> bool:
    _require_hip(backend)
    return load().byhip_session_commit_continue() == _abi.BYHIP_OK


def sessionRecoverQueue(backend: GpuBackend) -> bool:
    _require_hip(backend)
    return load().byhip_session_recover() == _abi.BYHIP_OK


def sessionGetLastError(backend: GpuBackend) -> str:
    _require_hip(backend)
    return _abi.last_error()


def sessionRead(backend: GpuBackend, h: SessionHandle, n: int) -> np.ndarray:
    """sessionRead, gpubackend.nim:2669: `n` floats."""
    _require_hip(backend)
    out = np.empty(int(n), dtype=np.float32)
    check(load().byhip_session_read(h.hipHandle, out.ctypes.data, out.size), "sessionRead")
    return out


def sessionFree(backend: GpuBackend, h: SessionHandle) -> None:
    """sessionFree, gpubackend.nim:2694 (deferred while a session is open)."""
    _require_hip(backend)
    if h.hipHandle:
        check(load().byhip_session_free(h.hipHandle), "sessionFree")
    h.kind, h.hipHandle = gbCpu, None


def sessionSetGpuTiming(backend: GpuBackend, on: bool) -> bool:
    _require_hip(backend)
    return load().byhip_session_set_gpu_timing(int(on)) == _abi.BYHIP_OK


def sessionGpuSeconds(backend: GpuBackend) -> float:
    _require_hip(backend)
    return float(load().byhip_session_gpu_seconds())


# ── record / replay (gpubackend.nim:2502-2552), kept as HIP graphs ──────────────────────────


def sessionCanRecord(backend: GpuBackend) -> bool:
    _require_hip(backend)
    return load().byhip_session_can_record() == 1


def sessionBeginRecording(backend: GpuBackend) -> bool:
    _require_hip(backend)
    return ensureGpuInit(backend) and load().byhip_session_begin_recording() == _abi.BYHIP_OK


def sessionLastRecording(backend: GpuBackend) -> int:
    _require_hip(backend)
    return int(load().byhip_session_last_recording())


def sessionReplay(backend: GpuBackend, id: int, times: int = 1) -> bool:
    """Submits a kept recording again (`times` back to back) and waits for it."""
    _require_hip(backend)
    return load().byhip_session_replay(int(id), int(times)) == _abi.BYHIP_OK


def sessionFreeRecording(backend: GpuBackend, id: int) -> None:
    _require_hip(backend)
    load().byhip_session_free_recording(int(id))


# ── resident Q4 weights and Q4 ops ──────────────────────────────────────────────────────────


@dataclass
class ResidentWeightHandle:
    """ResidentWeightHandle, gpubackend.nim:2813-2825 (hip fields)."""
    kind: GpuBackend
    k: int
    n: int
    groupSize: int
    nGroupsPerRow: int
    wqOffset: int = 0
    hipWeights: int | None = None


def residentUploadQ4(backend: GpuBackend, wq, scales, zeros, k: int, n: int, groupSize: int,
                     nGroupsPerRow: int, wqOffset: int = 0) -> ResidentWeightHandle:
    """residentUploadQ4, gpubackend.nim:2883-2919."""
    _require_hip(backend)
    ensureGpuInit(backend)
    wq = np.ascontiguousarray(wq, dtype=np.uint8)
    sc = np.ascontiguousarray(scales, dtype=np.float32)
    ze = np.ascontiguousarray(zeros, dtype=np.float32)
    h = C.c_void_p()
    check(load().byhip_q4_resident_upload(wq.ctypes.data, wq.nbytes, wqOffset, sc.ctypes.data,
                                          ze.ctypes.data, k, n, groupSize, nGroupsPerRow,
                                          C.byref(h)), "residentUploadQ4")
    return ResidentWeightHandle(gbHip, k, n, groupSize, nGroupsPerRow, wqOffset, h.value)


@dataclass
class MappedReadOnlyFile:
    """MappedReadOnlyFile, mapped_file.nim:5-8: a read-only mapping of a checkpoint; `data` is the
    host address of its first byte."""
    data: int = 0
    size: int = 0
    backing: object = None


def openReadOnlyMapping(path: str) -> MappedReadOnlyFile:
    """openReadOnlyMapping, mapped_file.nim:9-13."""
    import mmap
    with open(path, "rb") as f:
        size = os.fstat(f.fileno()).st_size
        m = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) if size else None
    if m is None:
        return MappedReadOnlyFile(0, 0, None)
    view = np.frombuffer(m, dtype=np.uint8)
    return MappedReadOnlyFile(view.ctypes.data, size, (m, view))


def unmapReadOnlyFile(mapping: MappedReadOnlyFile) -> None:
    """unmapReadOnlyFile, mapped_file.nim:15-20."""
    if mapping.backing is not None:
        m, view = mapping.backing
        del view
        mapping.backing = None
        m.close()
    mapping.data = 0
    mapping.size = 0


def residentUploadQ4Mapped(backend: GpuBackend, wq: int, wqBytes: int, scales, zeros, k: int, n: int,
                           groupSize: int, nGroupsPerRow: int) -> tuple[ResidentWeightHandle, bool]:
    """residentUploadQ4Mapped, gpubackend.nim:2961-2998: packed weights at host address `wq` (for
    example inside a MappedReadOnlyFile) are copied straight from the mapping into device memory,
    never through an intermediate host copy; scales and zeros are small and always copied.

    Returns (weights, zeroCopy). zeroCopy is False: the MI355X keeps weights in its own HBM, and
    the GPU does not wrap pageable host pages in place here (that would need the pages
    registered with the runtime), so the copy is the dGPU branch of the reference. The caller may
    unmap once this returns (the library has its own copy)."""
    _require_hip(backend)
    ensureGpuInit(backend)
    sc = np.ascontiguousarray(scales, dtype=np.float32)
    ze = np.ascontiguousarray(zeros, dtype=np.float32)
    h = C.c_void_p()
    check(load().byhip_q4_resident_upload(C.c_void_p(wq), wqBytes, 0, sc.ctypes.data, ze.ctypes.data,
                                          k, n, groupSize, nGroupsPerRow, C.byref(h)),
          "residentUploadQ4Mapped")
    return ResidentWeightHandle(gbHip, k, n, groupSize, nGroupsPerRow, 0, h.value), False


def residentPrepareQ4(w: ResidentWeightHandle, M: int = 1) -> bool:
    """residentPrepareQ4, gpubackend.nim:2871-2880: opt-in plan selection for these weights at
    this M (fp32 activations, the session API's dtype); the ordinary Q4 session calls then use
    the plan. False when tuning is off or a session is open."""
    if w.hipWeights is None:
        return False
    rc = load().byhip_q4_prepare(w.hipWeights, M, _abi.F32)
    if rc == _abi.BYHIP_UNSUPPORTED:
        return False
    check(rc, "residentPrepareQ4")
    return True


def residentFreeQ4(w: ResidentWeightHandle) -> None:
    """residentFreeQ4, gpubackend.nim:3233-3253."""
    if w.hipWeights:
        check(load().byhip_q4_resident_free(w.hipWeights), "residentFreeQ4")
    w.hipWeights = None


def sessionMatmulQ4(backend: GpuBackend, a: SessionHandle, w: ResidentWeightHandle,
                    c: SessionHandle, M: int) -> bool:
    """sessionMatmulQ4, gpubackend.nim:3000-3061: c (M x N) = a (M x K) . Wq^T, fp32 handles; c is
    allocated when it has no buffer. Returns False when the op cannot be encoded."""
    _require_hip(backend)
    if w.hipWeights is None or a.hipHandle is None:
        return False
    if c.hipHandle is None:
        c.__dict__.update(sessionAllocScratch(gbHip, M * w.n).__dict__)
    rc = load().byhip_q4_matmul(a.hipHandle, _abi.F32, w.hipWeights, c.hipHandle, _abi.F32, M)
    if rc == _abi.BYHIP_UNSUPPORTED:
        return False
    check(rc, "sessionMatmulQ4")
    return True


def sessionMatmulQ4Fused(backend: GpuBackend, mode: int, a: SessionHandle, ws, outs,
                         res: SessionHandle, hasRes: bool, gamma: SessionHandle = None,
                         eps: float = 0.0, hasNorm: bool = False) -> bool:
    """sessionMatmulQ4Fused, gpubackend.nim:3185-3231: the fused decode GEMV (M = 1). mode 0: ws
    (1..3 resident weights) share a, outs[i] receives ws[i]; mode 1: ws = [gate, up], outs[0] =
    silu(gate . x) * (up . x). res is added when hasRes; with hasNorm, a is the raw vector and
    RMSNorm (gamma, eps) is applied inside the kernel. Output handles must already be allocated.
    Returns False when unsupported, so callers run the unfused sequence."""
    import ctypes as C
    _require_hip(backend)
    if a.hipHandle is None or len(ws) < 1 or len(ws) > 3 or len(outs) < len(ws) or \
            (mode == 1 and len(ws) != 2):
        return False
    if hasRes and (res is None or res.hipHandle is None):
        return False
    if hasNorm and (gamma is None or gamma.hipHandle is None):
        return False
    if any(w.hipWeights is None for w in ws) or any(o.hipHandle is None for o in outs[:len(ws)]):
        return False
    wp = (C.c_void_p * len(ws))(*[w.hipWeights for w in ws])
    op = (C.c_void_p * len(outs))(*[o.hipHandle for o in outs])
    rc = load().byhip_q4_matmul_fused(mode, a.hipHandle, C.cast(wp, C.c_void_p), len(ws),
                                      C.cast(op, C.c_void_p), len(outs),
                                      res.hipHandle if hasRes else None, int(hasRes),
                                      gamma.hipHandle if hasNorm else None, eps, int(hasNorm))
    if rc == _abi.BYHIP_UNSUPPORTED:
        return False
    check(rc, "sessionMatmulQ4Fused")
    return True


def gpuMatmulQ4(backend: GpuBackend, a, wq, scales, zeros, m: int, k: int, n: int, groupSize: int,
                nGroupsPerRow: int, cpuFallback=None) -> np.ndarray:
    """gpuMatmulQ4, gpubackend.nim:806-843: host fp32 in and out, weights uploaded per call.

    On a device failure: raises when CPU fallback is forbidden; otherwise returns
    cpuFallback(...) when the caller supplies one (the reference uses
    cpuDequantMatmulQ4Fallback, gpubackend.nim:779-804) and raises when it does not."""
    _require_hip(backend)
    a = np.ascontiguousarray(a, dtype=np.float32)
    wq = np.ascontiguousarray(wq, dtype=np.uint8)
    sc = np.ascontiguousarray(scales, dtype=np.float32)
    ze = np.ascontiguousarray(zeros, dtype=np.float32)
    c = np.empty(m * n, dtype=np.float32)
    try:
        if not ensureGpuInit(backend):
            raise HipBackendError(_abi.last_error() or "no HIP device")
        check(load().byhip_gpu_matmul_q4(a.ctypes.data, wq.ctypes.data, sc.ctypes.data, ze.ctypes.data,
                                         c.ctypes.data, m, k, n, groupSize, nGroupsPerRow),
              "matmul_q4")
        return c
    except HipBackendError as e:
        handleGpuFailure(backend, "matmul_q4", e)
        if cpuFallback is None:
            raise
        return cpuFallback(a, wq, sc, ze, m, k, n, groupSize, nGroupsPerRow)


# ── FP4-KM / FP16 tile GEMM (gpubackend.nim:1442-1488) ───────────────────────────────────────


def _tile(a: SessionHandle, w: SessionHandle, lut: SessionHandle, c: SessionHandle, M, K, N) -> bool:
    if c.hipHandle is None:
        c.__dict__.update(sessionAllocScratch(gbHip, M * N).__dict__)
    rc = load().byhip_fp4km_tile_gemm(a.hipHandle, _abi.F32, w.hipHandle, w.probeBytes, N * (K // 2),
                                      lut.hipHandle, lut.probeBytes // 4, 0, c.hipHandle, _abi.F32,
                                      M, K, N)
    if rc == _abi.BYHIP_UNSUPPORTED:
        return False
    check(rc, "sessionFp4Gemm")
    return True


def sessionFp4GemmTensorCore(backend, a, w, lut, c, M, K, N) -> bool:
    """sessionFp4GemmTensorCore, gpubackend.nim:1442-1449 (MFMA on the hip backend)."""
    _require_hip(backend)
    return _tile(a, w, lut, c, M, K, N)


def sessionFp4GemmTiledEnc(backend, a, w, lut, c, M, K, N) -> bool:
    """sessionFp4GemmTiledEnc, gpubackend.nim:1465-1472."""
    _require_hip(backend)
    return _tile(a, w, lut, c, M, K, N)


def sessionF16GemmTile(backend, a, w, c, M, K, N, tensorCore=True) -> bool:
    """sessionF16GemmTile, gpubackend.nim:1474-1481."""
    _require_hip(backend)
    if c.hipHandle is None:
        c.__dict__.update(sessionAllocScratch(gbHip, M * N).__dict__)
    rc = load().byhip_f16_tile_gemm(a.hipHandle, _abi.F32, w.hipHandle, w.probeBytes // 2, c.hipHandle,
                                    _abi.F32, M, K, N)
    if rc == _abi.BYHIP_UNSUPPORTED:
        return False
    check(rc, "sessionF16GemmTile")
    return True


def sessionTileGemmReady(backend, f16: bool, tensorCore: bool) -> bool:
    """sessionTileGemmReady, gpubackend.nim:1483-1488."""
    _require_hip(backend)
    if not ensureGpuInit(backend):
        return False
    rc = load().byhip_tile_gemm_ready(int(f16), int(tensorCore))
    return rc == 1


# ── micro-VM route (session_vm_dispatch.nim:128-158) ─────────────────────────────────────────


def sessionEncTileProgram(backend, words, mem: SessionHandle, u8: SessionHandle | None,
                          lut: SessionHandle | None, inp: SessionHandle | None, rows: int = 0) -> bool:
    """Encodes a shape-op micro-kernel (tile GEMM, FP4 / Q4 shape ops) over the slots the reference
    binds (mem, u8, lut, input; slot_layout.nim:23-37). False when the program has no HIP route."""
    _require_hip(backend)
    w = np.ascontiguousarray(words, dtype=np.uint32)
    rc = load().byhip_program_dispatch(
        w.ctypes.data_as(C.POINTER(C.c_uint32)), len(w), mem.hipHandle, mem.probeBytes // 4,
        u8.hipHandle if u8 else None, u8.probeBytes if u8 else 0,
        lut.hipHandle if lut else None, lut.probeBytes // 4 if lut else 0,
        inp.hipHandle if inp else None, inp.probeBytes // 4 if inp else 0, rows)
    if rc == _abi.BYHIP_UNSUPPORTED:
        return False
    check(rc, "sessionEncTileProgram")
    return True


__all__ = [n for n in dir() if not n.startswith("_") and n not in ("C", "enum", "sys", "np",
                                                                    "dataclass", "field",
                                                                    "annotations")]
