## backends/hip/hip_backend.nim - the MI355X (gfx950) backend of BybyLang's quantized tile-GEMM path.
##
## NOT COMPILED: no Nim toolchain exists where this file was written. It is the binding a maintainer
## adds beside backends/cpu, backends/metal and backends/vulkan; the C ABI it binds
## (include/byhip.h, libbybyhip.so) is what this repository builds and tests.
##
## The binding follows backends/cpu/cpu_backend.nim:22-26,102-160 (importc, cdecl over a native
## ABI), here from a shared library. The `hip*` procs below are the bodies of the `of gbHip:`
## branches that gpubackend.nim gains (INTEGRATION.md section 3 lists each proc and line); they take
## the reference's handle types, whose HIP fields are added by that patch:
##   SessionHandle.hipHandle: pointer          (gpubackend.nim:894-903)
##   ResidentWeightHandle.hipWeights: pointer  (gpubackend.nim:2813-2825)

import std/[os, strutils]

const HipLib* = "libbybyhip.so"

const
  BYHIP_OK* = 0.cint
  BYHIP_UNSUPPORTED* = 1.cint
  BYHIP_ERROR* = -1.cint
  BYHIP_F32* = 0.cint
  BYHIP_F16* = 1.cint
  BYHIP_BF16* = 2.cint
  BYHIP_MXFP4_KM* = 3.cint

{.push importc, cdecl, dynlib: HipLib.}
proc byhip_init*(device: cint): cint
proc byhip_last_error*(): cstring
proc byhip_clear_error*()
proc byhip_fault_inject*(count: cint)
proc byhip_alloc*(bytes: csize_t, dptr: ptr pointer): cint
proc byhip_free*(dptr: pointer): cint
proc byhip_upload*(dptr: pointer, dstOff: csize_t, src: pointer, bytes: csize_t): cint
proc byhip_read*(dptr: pointer, srcOff: csize_t, dst: pointer, bytes: csize_t): cint
proc byhip_synchronize*(): cint
proc byhip_session_begin*(): cint
proc byhip_session_upload*(data: ptr float32, n: csize_t, outp: ptr pointer): cint
proc byhip_session_upload_bytes*(data: pointer, bytes: csize_t, outp: ptr pointer): cint
proc byhip_session_alloc_scratch*(n: csize_t, outp: ptr pointer): cint
proc byhip_session_end*(): cint
proc byhip_session_commit_continue*(): cint
proc byhip_session_recover*(): cint
proc byhip_session_read*(h: pointer, dst: ptr float32, n: csize_t): cint
proc byhip_session_free*(h: pointer): cint
proc byhip_session_set_gpu_timing*(on: cint): cint
proc byhip_session_gpu_seconds*(): cdouble
proc byhip_session_can_record*(): cint
proc byhip_session_begin_recording*(): cint
proc byhip_session_last_recording*(): cint
proc byhip_session_replay*(id, times: cint): cint
proc byhip_session_free_recording*(id: cint): cint
proc byhip_q4_resident_upload*(wq: pointer, wqBytes, wqOff: csize_t, scales, zeros: ptr float32,
                               K, N, groupSize, groupsPerRow: cint, outp: ptr pointer): cint
proc byhip_q4_resident_from_device*(dWq: pointer, wqOff: csize_t, dScales, dZeros: pointer,
                                    K, N, groupSize, groupsPerRow: cint, outp: ptr pointer): cint
proc byhip_q4_resident_free*(w: pointer): cint
proc byhip_q4_matmul*(x: pointer, xDtype: cint, w: pointer, y: pointer, yDtype, M: cint): cint
proc byhip_q4_matmul_static*(x: pointer, xDtype: cint, w: pointer, y: pointer, yDtype, M: cint): cint
proc byhip_q4_prepare*(w: pointer, M, xDtype: cint): cint
proc byhip_q4_plan_info*(w: pointer, M, xDtype: cint, name: cstring, nameLen: cint,
                         fromCache: ptr cint): cint
proc byhip_q4_plans_reset*(): cint
proc byhip_q4_matmul_fused*(mode: cint, a: pointer, ws: ptr pointer, nWs: cint, outs: ptr pointer,
                            nOuts: cint, res: pointer, hasRes: cint, gamma: pointer, eps: cfloat,
                            hasNorm: cint): cint
proc byhip_gpu_matmul_q4*(a: ptr float32, wq: ptr uint8, scales, zeros: ptr float32, c: ptr float32,
                          M, K, N, groupSize, groupsPerRow: cint): cint
proc byhip_fp4km_tile_gemm*(x: pointer, xDtype: cint, blob: pointer, blobBytes, scaleBase: csize_t,
                            lut: pointer, lutFloats, lutBase: csize_t, y: pointer, yDtype,
                            M, K, N: cint): cint
proc byhip_mxfp4_gemm*(x, w: pointer, y: pointer, yDtype, M, K, N: cint): cint
proc byhip_f16_tile_gemm*(x: pointer, xDtype: cint, w: pointer, wHalves: csize_t, y: pointer,
                          yDtype, M, K, N: cint): cint
proc byhip_tile_gemm_ready*(f16, tensorCore: cint): cint
proc byhip_program_dispatch*(words: ptr uint32, nWords: cint, mem: pointer, memLen: csize_t,
                             u8: pointer, u8Len: csize_t, lut: pointer, lutLen: csize_t,
                             input: pointer, inputLen: csize_t, rows: cint): cint
{.pop.}

proc hipCheck*(rc: cint, what: string) =
  ## BYHIP_ERROR becomes a CatchableError, so handleGpuFailure (gpubackend.nim:80-105) applies the
  ## forbid-fallback policy; BYHIP_UNSUPPORTED is left to the caller, which returns `false`.
  if rc == BYHIP_ERROR:
    raise newException(CatchableError, what & ": " & $byhip_last_error())

var hipReady = false

proc hipEnsureInit*(): bool =
  ## ensureGpuInit for gbHip; the device ordinal follows BYBY_HIP_DEVICE (as BYBY_VULKAN_DEVICE,
  ## distributed.nim:144-145).
  if hipReady: return true
  let dev = try: parseInt(getEnv("BYBY_HIP_DEVICE", "0")) except ValueError: 0
  hipReady = byhip_init(dev.cint) == BYHIP_OK
  hipReady

# ── session lifecycle (gpubackend.nim:1042-2721) ─────────────────────────────────────────────

proc hipSessionBegin*(): bool = hipEnsureInit() and byhip_session_begin() == BYHIP_OK

proc hipSessionUpload*(data: seq[float32]): pointer =
  var p: pointer
  hipCheck(byhip_session_upload(if data.len > 0: unsafeAddr data[0] else: nil,
                                csize_t(data.len), addr p), "sessionUpload")
  p

proc hipSessionAllocScratch*(n: int): pointer =
  var p: pointer
  hipCheck(byhip_session_alloc_scratch(csize_t(n), addr p), "sessionAllocScratch")
  p

proc hipSessionEnd*(): bool = byhip_session_end() == BYHIP_OK
proc hipSessionCommitContinue*(): bool = byhip_session_commit_continue() == BYHIP_OK
proc hipSessionRecoverQueue*(): bool = byhip_session_recover() == BYHIP_OK
proc hipSessionGetLastError*(): string = $byhip_last_error()

proc hipSessionRead*(h: pointer, n: int): seq[float32] =
  result = newSeq[float32](n)
  if n > 0:
    hipCheck(byhip_session_read(h, addr result[0], csize_t(n)), "sessionRead")

proc hipSessionFree*(h: pointer) =
  ## deferred to the end of an open session (vulkan_driver.nim:1192,1817-1819)
  if h != nil: hipCheck(byhip_session_free(h), "sessionFree")

proc hipSessionSetGpuTiming*(on: bool): bool = byhip_session_set_gpu_timing(on.cint) == BYHIP_OK
proc hipSessionGpuSeconds*(): float = float(byhip_session_gpu_seconds())
proc hipSessionCanRecord*(): bool = byhip_session_can_record() == 1
proc hipSessionBeginRecording*(): bool = hipEnsureInit() and byhip_session_begin_recording() == BYHIP_OK
proc hipSessionLastRecording*(): int = int(byhip_session_last_recording())
proc hipSessionReplay*(id: int): bool = byhip_session_replay(id.cint, 1) == BYHIP_OK
proc hipSessionFreeRecording*(id: int) = discard byhip_session_free_recording(id.cint)

# ── resident Q4 weights and Q4 ops (gpubackend.nim:2813-3253) ───────────────────────────────

proc hipResidentUploadQ4*(wq: pointer, wqBytes, wqOffset: int, scales, zeros: seq[float32],
                          k, n, groupSize, nGroupsPerRow: int): pointer =
  ## residentUploadQ4 and residentUploadQ4Mapped (the mapping's pointer, offset 0): the packed rows
  ## are copied once into HBM in the library's layout.
  doAssert hipEnsureInit(), "HIP backend unavailable"
  var w: pointer
  hipCheck(byhip_q4_resident_upload(wq, csize_t(wqBytes), csize_t(wqOffset),
                                    unsafeAddr scales[0], unsafeAddr zeros[0], k.cint, n.cint,
                                    groupSize.cint, nGroupsPerRow.cint, addr w), "residentUploadQ4")
  w

proc hipResidentFreeQ4*(w: pointer) =
  if w != nil: hipCheck(byhip_q4_resident_free(w), "residentFreeQ4")

proc hipResidentPrepareQ4*(w: pointer, M: int): bool =
  ## residentPrepareQ4 (2871-2880): false when tuning is off or a session is open
  let rc = byhip_q4_prepare(w, M.cint, BYHIP_F32)
  hipCheck(rc, "residentPrepareQ4")
  rc == BYHIP_OK

proc hipSessionMatmulQ4*(a, w: pointer, c: var pointer, M, n: int): bool =
  ## sessionMatmulQ4 (3000-3061): a nil output is allocated by the encoder (3029-3030)
  if c == nil: c = hipSessionAllocScratch(M * n)
  let rc = byhip_q4_matmul(a, BYHIP_F32, w, c, BYHIP_F32, M.cint)
  hipCheck(rc, "sessionMatmulQ4")
  rc == BYHIP_OK

proc hipSessionMatmulQ4Fused*(mode: int, a: pointer, ws: openArray[pointer], outs: openArray[pointer],
                              res: pointer, hasRes: bool, gamma: pointer, eps: float32,
                              hasNorm: bool): bool =
  ## sessionMatmulQ4Fused (3185-3231), with the reference's early returns
  if ws.len < 1 or ws.len > 3 or outs.len < ws.len or (mode == 1 and ws.len != 2): return false
  var hw: array[3, pointer]
  var ho: array[3, pointer]
  for i in 0 ..< ws.len:
    if outs[i] == nil: return false
    hw[i] = ws[i]
    ho[i] = outs[i]
  let rc = byhip_q4_matmul_fused(mode.cint, a, addr hw[0], ws.len.cint, addr ho[0], ws.len.cint,
                                 (if hasRes: res else: nil), hasRes.cint,
                                 (if hasNorm: gamma else: nil), eps.cfloat, hasNorm.cint)
  hipCheck(rc, "sessionMatmulQ4Fused")
  rc == BYHIP_OK

proc hipGpuMatmulQ4*(a: seq[float32], wq: seq[uint8], scales, zeros: seq[float32],
                     m, k, n, groupSize, nGroupsPerRow: int): seq[float32] =
  ## gpuMatmulQ4 (806-843): a raise reaches handleGpuFailure; the library never computes on the CPU
  doAssert hipEnsureInit(), "HIP backend unavailable"
  result = newSeq[float32](m * n)
  hipCheck(byhip_gpu_matmul_q4(unsafeAddr a[0], unsafeAddr wq[0], unsafeAddr scales[0],
                               unsafeAddr zeros[0], addr result[0], m.cint, k.cint, n.cint,
                               groupSize.cint, nGroupsPerRow.cint), "gpuMatmulQ4")

# ── FP4-KM and F16 tile GEMM (gpubackend.nim:1442-1488) ─────────────────────────────────────

proc hipSessionFp4Gemm*(a, w, lut: pointer, wBytes, lutFloats: int, c: pointer, M, K, N: int): bool =
  ## sessionFp4GemmTensorCore / sessionFp4GemmTiledEnc / sessionFp4GemmMetal: the blob's scale
  ## bytes follow the nibbles (scale base N * K / 2), the table at float 0 of `lut`
  let rc = byhip_fp4km_tile_gemm(a, BYHIP_F32, w, csize_t(wBytes), csize_t(N * (K div 2)), lut,
                                 csize_t(lutFloats), 0, c, BYHIP_F32, M.cint, K.cint, N.cint)
  hipCheck(rc, "sessionFp4Gemm")
  rc == BYHIP_OK

proc hipSessionF16GemmTile*(a, w: pointer, wHalves: int, c: pointer, M, K, N: int): bool =
  let rc = byhip_f16_tile_gemm(a, BYHIP_F32, w, csize_t(wHalves), c, BYHIP_F32, M.cint, K.cint, N.cint)
  hipCheck(rc, "sessionF16GemmTile")
  rc == BYHIP_OK

proc hipSessionTileGemmReady*(f16, tensorCore: bool): bool =
  byhip_tile_gemm_ready(f16.cint, tensorCore.cint) == 1
