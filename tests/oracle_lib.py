"""ctypes bindings of the checker libraries under oracle/ (test infrastructure only).

`Oracle` wraps oracle/liboracle.so, the C restatement of the reference's CPU arithmetic.
`Reference` wraps oracle/_ref/libbybyref.so, the reference's own CPU backend C
(backends/cpu/cpu_vm.c, cpu_kernels.c) compiled from its sources; it exists only where
/root/reference was present at build time, so tests that need it skip without it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_SO = os.path.join(ORACLE_DIR, "liboracle.so")
REF_SO = os.path.join(ORACLE_DIR, "_ref", "libbybyref.so")

OP_HALT = 0x01
OP_BARRIER_TG = 0x50
OP_Q4_COOP_GEMM = 0xAA
OP_Q4_GEMV = 0xAB
OP_FP4_COOP_GEMM = 0xAC
OP_TILE_GEMM = 0xB0
OP_TILE_ZERO, OP_TILE_K_BEGIN, OP_TILE_K_END = 0xB1, 0xB2, 0xB3
OP_TILE_LOAD_A, OP_TILE_DECODE_FP4, OP_TILE_MMA, OP_TILE_STORE = 0xB4, 0xB5, 0xB6, 0xB7
OP_TILE_LOAD_B_F16 = 0xB8

FP4_VALUES = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6],
                      dtype=np.float32)

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")


def ensure_built() -> None:
    """Build the checker libraries if they are missing (gcc only, a second or two)."""
    if not os.path.exists(ORACLE_SO):
        subprocess.run(["make", "-s", "-C", ORACLE_DIR, "liboracle.so"], check=True)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ── program builders (session_vm.nim:379-416, 418-420, 369-371) ─────────────────────────────

def pack1(op: int, a: int) -> int:
    """pack1 of session_vm.nim:210-211: register a in bits 8..12 and 23..25."""
    return (op & 0xFF) | ((a & 0x1F) << 8) | (((a >> 5) & 0x7) << 23)


def fp4_tile_program(M, K, N, scale_base, lut_base):
    """buildFp4TileGemmProgram, session_vm.nim:383-399."""
    return np.array([pack1(OP_TILE_GEMM, 0), M, K, N, scale_base, lut_base, OP_TILE_ZERO,
                     OP_TILE_K_BEGIN, OP_TILE_LOAD_A, OP_TILE_DECODE_FP4, OP_BARRIER_TG,
                     OP_TILE_MMA, OP_BARRIER_TG, OP_TILE_K_END, OP_TILE_STORE, OP_HALT],
                    dtype=np.uint32)


def f16_tile_program(M, K, N):
    """buildF16TileGemmProgram, session_vm.nim:401-416."""
    return np.array([pack1(OP_TILE_GEMM, 1), M, K, N, 0, 0, OP_TILE_ZERO, OP_TILE_K_BEGIN,
                     OP_TILE_LOAD_A, OP_TILE_LOAD_B_F16, OP_BARRIER_TG, OP_TILE_MMA,
                     OP_BARRIER_TG, OP_TILE_K_END, OP_TILE_STORE, OP_HALT], dtype=np.uint32)


def shape_op_program(op, M, K, N, group, n_groups):
    """emitQ4Gemv / emitQ4CoopGemm / emitFp4CoopGemm + HALT (session_vm.nim:369-377, 418-420)."""
    return np.array([op, M, K, N, group, n_groups, OP_HALT], dtype=np.uint32)


def fp4_coop_lut_word(K, N):
    """fp4CoopLutWord, session_vm.nim:447-450."""
    return (N * (K // 2) + N * (K // 32) + 3) // 4


def q4_blob(wq, scales, zeros, K, N, n_groups):
    """The one-blob slot layout of the Q4 shape ops (cpu_vm.c:446-450): nibbles [N, K/2], word
    pad, fp32 scales [N, n_groups] at float (N*K/2+3)/4, fp32 zeros after them. Returns the
    blob as bytes (u8 slot) and as floats (lut slot)."""
    row_bytes = K // 2
    scale_base = (N * row_bytes + 3) // 4
    blob = np.zeros(scale_base + 2 * N * n_groups, dtype=np.float32)
    blob.view(np.uint8)[: N * row_bytes] = wq.reshape(-1)[: N * row_bytes]
    blob[scale_base: scale_base + N * n_groups] = scales.reshape(-1)
    blob[scale_base + N * n_groups:] = zeros.reshape(-1)
    return blob.view(np.uint8).copy(), blob


class Oracle:
    """oracle/liboracle.so."""

    def __init__(self, path: str = ORACLE_SO):
        ensure_built()
        L = C.CDLL(path)
        self.L = L
        L.orc_half_to_float.restype = C.c_float
        L.orc_half_to_float.argtypes = [C.c_uint16]
        L.orc_float_to_half.restype = C.c_uint16
        L.orc_float_to_half.argtypes = [C.c_float]
        L.orc_q4_shape_op.restype = C.c_int
        L.orc_q4_shape_op.argtypes = [C.c_int] + [C.c_uint32] * 5 + [
            C.c_void_p, C.c_int64, C.c_void_p, C.c_int64, C.c_void_p, C.c_int64, C.c_void_p,
            C.c_int64, C.c_uint32, C.c_uint32, C.c_char_p, C.c_int]
        L.orc_tile_gemm.restype = C.c_int
        L.orc_tile_gemm.argtypes = [C.c_uint32] * 4 + [C.c_uint64] * 2 + [
            C.c_void_p, C.c_int64, C.c_void_p, C.c_int64, C.c_void_p, C.c_int64, C.c_void_p,
            C.c_int64, C.c_uint32, C.c_uint32, C.c_char_p, C.c_int]
        L.orc_tile_gemm_reference.restype = None
        L.orc_tile_gemm_reference.argtypes = [C.c_void_p] * 3 + [C.c_int] * 3 + [
            C.c_int64, C.c_int64, C.c_void_p]
        L.orc_matmul_q4.restype = None
        L.orc_matmul_q4.argtypes = [C.c_void_p] * 5 + [C.c_int] * 7
        L.orc_matmul_q4_ref.restype = None
        L.orc_matmul_q4_ref.argtypes = [C.c_void_p] * 5 + [C.c_int] * 5
        L.orc_run_shape_program.restype = C.c_int
        L.orc_run_shape_program.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int,
                                            C.c_void_p, C.c_int, C.c_void_p, C.c_int,
                                            C.c_void_p, C.c_int, C.c_char_p, C.c_int]
        L.orc_unpack_q4.restype = None
        L.orc_unpack_q4.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p]
        L.orc_unpack_fp4km.restype = None
        L.orc_unpack_fp4km.argtypes = [C.c_void_p, C.c_int64, C.c_int, C.c_int, C.c_void_p,
                                       C.c_void_p]
        L.orc_xorshift32.restype = C.c_uint32
        L.orc_xorshift32.argtypes = [C.POINTER(C.c_uint32)]
        L.orc_make_fp4_case.restype = None
        L.orc_make_fp4_case.argtypes = [C.POINTER(C.c_uint32), C.c_int, C.c_int, C.c_int,
                                        C.c_void_p, C.c_void_p, C.c_void_p]
        L.orc_make_f16_case.restype = None
        L.orc_make_f16_case.argtypes = [C.POINTER(C.c_uint32), C.c_int, C.c_int, C.c_int,
                                        C.c_void_p, C.c_void_p, C.c_void_p]
        L.orc_q4_fused.restype = C.c_int
        L.orc_q4_fused.argtypes = [C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                   C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                   C.c_void_p, C.c_void_p, C.c_float]

    # -- conversions
    def half_to_float(self, h: int) -> float:
        return self.L.orc_half_to_float(h)

    def float_to_half(self, f: float) -> int:
        return self.L.orc_float_to_half(f)

    # -- arithmetic
    def run_program(self, code, mem_len, packed=None, lut=None, x=None):
        code = np.ascontiguousarray(code, dtype=np.uint32)
        mem = np.zeros(mem_len, dtype=np.float32)
        err = C.create_string_buffer(256)
        rc = self.L.orc_run_shape_program(
            _ptr(code), len(code), _ptr(mem), mem_len, _ptr(packed),
            0 if packed is None else packed.size, _ptr(lut), 0 if lut is None else lut.size,
            _ptr(x), 0 if x is None else x.size, err, 256)
        return rc, mem, err.value.decode()

    def q4_shape_op(self, coop, M, K, N, group, n_groups, blob_u8, blob_f32, x, rows=None):
        out = np.zeros(M * N, dtype=np.float32)
        err = C.create_string_buffer(256)
        r0, r1 = rows if rows else (0, M)
        rc = self.L.orc_q4_shape_op(int(coop), M, K, N, group, n_groups, _ptr(blob_u8),
                                    blob_u8.size, _ptr(blob_f32), blob_f32.size, _ptr(x), x.size,
                                    _ptr(out), out.size, r0, r1, err, 256)
        if rc != 0:
            raise ValueError(err.value.decode())
        return out.reshape(M, N)

    def tile_gemm(self, fmt, M, K, N, scale_base, lut_base, packed, lut, x, rows=None):
        Mr = M if M else x.size // K
        out = np.zeros(Mr * N, dtype=np.float32)
        err = C.create_string_buffer(256)
        r0, r1 = rows if rows else (0, 0xFFFFFFFF)
        rc = self.L.orc_tile_gemm(fmt, M, K, N, scale_base, lut_base, _ptr(packed), packed.size,
                                  _ptr(lut), 0 if lut is None else lut.size, _ptr(x), x.size,
                                  _ptr(out), out.size, r0, r1, err, 256)
        if rc != 0:
            raise ValueError(err.value.decode())
        return out.reshape(Mr, N)

    def tile_gemm_reference(self, x, packed, table, rows, K, N, scale_base, lut_base):
        out = np.zeros(rows * N, dtype=np.float32)
        self.L.orc_tile_gemm_reference(_ptr(x), _ptr(packed), _ptr(table), rows, K, N,
                                       scale_base, lut_base, _ptr(out))
        return out.reshape(rows, N)

    def matmul_q4(self, a, wq, scales, zeros, M, K, N, group, groups_per_row, rows=None):
        c = np.zeros(M * N, dtype=np.float32)
        r0, r1 = rows if rows else (0, M)
        self.L.orc_matmul_q4(_ptr(a), _ptr(wq), _ptr(scales), _ptr(zeros), _ptr(c), M, K, N,
                             group, groups_per_row, r0, r1)
        return c.reshape(M, N)

    def matmul_q4_ref(self, a, wq, scales, zeros, M, K, N, group, groups_per_row):
        c = np.zeros(M * N, dtype=np.float32)
        self.L.orc_matmul_q4_ref(_ptr(a), _ptr(wq), _ptr(scales), _ptr(zeros), _ptr(c), M, K, N,
                                 group, groups_per_row)
        return c.reshape(M, N)

    def q4_fused(self, mode, a, mats, K, group, groups_per_row, residual=None, gamma=None, eps=0.0):
        """mats: list of (wq, scales, zeros, N). Returns the list of outputs (one in mode 1), or
        None when the reference rejects the combination."""
        n = len(mats)
        keep = [np.ascontiguousarray(m[0]) for m in mats] + [np.ascontiguousarray(m[1], np.float32) for m in mats] + \
            [np.ascontiguousarray(m[2], np.float32) for m in mats]
        wq = (C.c_void_p * max(n, 1))(*[_ptr(keep[i]) for i in range(n)])
        sc = (C.c_void_p * max(n, 1))(*[_ptr(keep[n + i]) for i in range(n)])
        ze = (C.c_void_p * max(n, 1))(*[_ptr(keep[2 * n + i]) for i in range(n)])
        Ns = (C.c_int * max(n, 1))(*[int(m[3]) for m in mats])
        outs = [np.zeros(int(m[3]), dtype=np.float32) for m in mats]
        op = (C.c_void_p * max(n, 1))(*[_ptr(o) for o in outs])
        a = np.ascontiguousarray(a, np.float32)
        res = None if residual is None else np.ascontiguousarray(residual, np.float32)
        gam = None if gamma is None else np.ascontiguousarray(gamma, np.float32)
        rc = self.L.orc_q4_fused(mode, n, _ptr(a), K, group, groups_per_row, C.cast(wq, C.c_void_p),
                                 C.cast(sc, C.c_void_p), C.cast(ze, C.c_void_p), C.cast(Ns, C.c_void_p),
                                 C.cast(op, C.c_void_p), _ptr(res), _ptr(gam), eps)
        if rc != 0:
            return None
        return outs[:1] if mode == 1 else outs

    def unpack_q4(self, wq, K, N):
        codes = np.zeros(N * K, dtype=np.uint8)
        self.L.orc_unpack_q4(_ptr(wq), K, N, _ptr(codes))
        return codes.reshape(N, K)

    def unpack_fp4km(self, packed, scale_base, K, N):
        codes = np.zeros(N * K, dtype=np.uint8)
        sb = np.zeros(N * (K // 32), dtype=np.uint8)
        self.L.orc_unpack_fp4km(_ptr(packed), scale_base, K, N, _ptr(codes), _ptr(sb))
        return codes.reshape(N, K), sb.reshape(N, K // 32)

    # -- generators of tests/t_fp4_tile_gemm.nim
    def make_fp4_case(self, state, M, K, N):
        x = np.zeros(M * K, dtype=np.float32)
        packed = np.zeros(N * (K // 2) + N * (K // 32), dtype=np.uint8)
        table = np.zeros(272, dtype=np.float32)
        self.L.orc_make_fp4_case(C.byref(state), M, K, N, _ptr(x), _ptr(packed), _ptr(table))
        return x, packed, table

    def make_f16_case(self, state, M, K, N):
        x = np.zeros(M * K, dtype=np.float32)
        w = np.zeros(N * K, dtype=np.float32)
        halves = np.zeros(N * K * 2, dtype=np.uint8)
        self.L.orc_make_f16_case(C.byref(state), M, K, N, _ptr(x), _ptr(w), _ptr(halves))
        return x, w, halves


class Reference:
    """oracle/_ref/libbybyref.so: nimf_cpu_vm_run_slots, nimf_cpu_matmul_q4 and nimf_cpu_rmsnorm of
    the reference."""

    def __init__(self, path: str = REF_SO):
        L = C.CDLL(path)
        self.L = L
        L.refshim_vm_run_slots.restype = C.c_int
        L.refshim_vm_run_slots.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p,
                                           C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_int,
                                           C.c_int, C.c_int, C.c_int, C.c_char_p, C.c_int]
        L.refshim_matmul_q4.restype = None
        L.refshim_matmul_q4.argtypes = [C.c_void_p] * 5 + [C.c_int] * 5
        L.refshim_rmsnorm.restype = None
        L.refshim_rmsnorm.argtypes = [C.c_void_p] * 3 + [C.c_int] * 2 + [C.c_float]

    @staticmethod
    def available() -> bool:
        return os.path.exists(REF_SO)

    def run_program(self, code, mem_len, packed=None, lut=None, x=None, n_threads=128,
                    tg_floats=64, tg_size=128):
        """The reference test's call shape (t_fp4_tile_gemm.nim:69-80): 128 threads, tg 128."""
        code = np.array(code, dtype=np.uint32)  # the interpreter takes a mutable pointer
        mem = np.zeros(mem_len, dtype=np.float32)
        err = C.create_string_buffer(512)
        rc = self.L.refshim_vm_run_slots(
            _ptr(code), len(code), _ptr(mem), mem_len, _ptr(packed),
            0 if packed is None else packed.size, _ptr(lut), 0 if lut is None else lut.size,
            _ptr(x), 0 if x is None else x.size, n_threads, tg_floats, tg_size, err, 512)
        return rc, mem, err.value.decode()

    def matmul_q4(self, a, wq, scales, zeros, M, K, N, group, groups_per_row):
        c = np.zeros(M * N, dtype=np.float32)
        self.L.refshim_matmul_q4(_ptr(a), _ptr(wq), _ptr(scales), _ptr(zeros), _ptr(c), M, K, N,
                                 group, groups_per_row)
        return c.reshape(M, N)


    def rmsnorm(self, x, gamma, rows, cols, eps):
        x = np.ascontiguousarray(x, np.float32).copy()  # the reference takes mutable pointers
        gamma = np.ascontiguousarray(gamma, np.float32).copy()
        out = np.zeros(rows * cols, dtype=np.float32)
        self.L.refshim_rmsnorm(_ptr(x), _ptr(gamma), _ptr(out), rows, cols, eps)
        return out


def fp4_cases(oracle: Oracle):
    """The five FP4-KM cases of t_fp4_tile_gemm.nim:147-148, made in order from one seed, then
    the five FP16 cases of 265-266 (same generator state, as the reference test runs them)."""
    state = C.c_uint32(2463534242)
    cases = []
    for (M, K, N) in [(1, 64, 16), (5, 128, 96), (20, 64, 72), (37, 128, 130), (70, 96, 64)]:
        x, packed, table = oracle.make_fp4_case(state, M, K, N)
        cases.append(dict(M=M, K=K, N=N, x=x, packed=packed, table=table))
    f16 = []
    for (M, K, N) in [(1, 64, 16), (5, 128, 96), (20, 64, 72), (37, 128, 130), (70, 192, 64)]:
        x, w, halves = oracle.make_f16_case(state, M, K, N)
        f16.append(dict(M=M, K=K, N=N, x=x, w=w, halves=halves))
    return cases, f16
