## micro_kernel/session_vm_dispatch_hip.nim - the HIP branch of the micro-VM encode bridge.
##
## NOT COMPILED: no Nim toolchain exists where this file was written. It is the proc a maintainer
## adds beside the shared encode API of micro_kernel/session_vm_dispatch.nim (sessionEncPipeline ..
## sessionEncDispatch, 128-158), imported from there. The caller (encodeVm) takes this route when
## the session's backend is gbHip and the program is a shape-op program (isTileGemmProgram,
## tile_gemm.nim:52; isQ4GemvProgram / isQ4CoopProgram / isFp4CoopProgram, jit_vm.nim:567-793):
## instead of compiling a shader and dispatching it, the whole program goes to
## byhip_program_dispatch with the five slots the reference binds (slot_layout.nim:23-37). The slot
## layout is unchanged, so .bybylang programs run unmodified.

import ../backends/hip/hip_backend

proc sessionEncShapeProgramHip*(words: openArray[uint32]; mem, u8, lut, input: pointer;
                                memFloats, u8Bytes, lutFloats, inputFloats, rows: int): bool =
  ## Runs a tile GEMM / Q4 / FP4 shape-op program on the HIP device. `rows` > 0 gives an M = 0
  ## header its row count (the dispatch's). Returns false for a program the library has no route
  ## for (BYHIP_UNSUPPORTED: the caller keeps its other routes); a rejected program raises with
  ## the reference's own CPU VM message ("CPU VM unsupported tile GEMM (format 0 K 48 N 16)", ...).
  if words.len == 0: return false
  let rc = byhip_program_dispatch(unsafeAddr words[0], words.len.cint, mem, csize_t(memFloats),
                                  u8, csize_t(u8Bytes), lut, csize_t(lutFloats), input,
                                  csize_t(inputFloats), rows.cint)
  hipCheck(rc, "shape-op program")
  rc == BYHIP_OK
