"""The micro-VM route's rejections through the C ABI: the reference's return code and message, and
the outputs it writes before it stops.

tests/golden/errors.json holds what the reference's own build (backends/cpu/cpu_vm.c) returned
for rejected programs, with the slots it was run on: mem 64 floats, a 4096-float blob in the u8
and lut slots, 1024 input floats. The out-of-range cases below (slot-domain checks,
slot_layout.nim:11-73, cpu_vm.c:168-175 and 420-628) are compared with the oracle's restatement of
the same loops (orc_run_shape_program), including the outputs it writes before the failing one.
"""
import ctypes as C
import json
import os

import numpy as np
import pytest

from bybylang_amd import _abi, synth
from oracle_lib import (OP_FP4_COOP_GEMM, OP_Q4_COOP_GEMM, OP_Q4_GEMV, f16_tile_program, fp4_coop_lut_word,
                        fp4_tile_program, q4_blob, shape_op_program)
from parity import ref_check

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def dispatch_raw(hip, words, mem, mem_len, u8, u8_len, lut, lut_len, x, x_len, rows=0):
    """byhip_program_dispatch with explicit slot lengths: (return code, message)."""
    w = np.ascontiguousarray(words, dtype=np.uint32)
    lib = _abi.load()
    lib.byhip_clear_error()
    rc = lib.byhip_program_dispatch(w.ctypes.data_as(C.POINTER(C.c_uint32)), len(w), mem.ptr, mem_len,
                                    u8.ptr if u8 else None, u8_len, lut.ptr if lut else None, lut_len,
                                    x.ptr if x else None, x_len, rows)
    return rc, _abi.last_error()


@pytest.mark.parametrize("name", sorted(json.load(open(os.path.join(GOLDEN, "errors.json")))))
def test_reference_error_programs(hip, name):
    """Every rejected program of the golden file gives the reference's code and text."""
    case = json.load(open(os.path.join(GOLDEN, "errors.json")))[name]
    blob = hip.DeviceBuffer.from_array(np.zeros(4096, np.float32))
    x = hip.DeviceBuffer.from_array(np.zeros(1024, np.float32))
    mem = hip.DeviceBuffer.from_array(np.zeros(64, np.float32))
    rc, err = dispatch_raw(hip, case["program"], mem, 64, blob, 4096 * 4, blob, 4096, x, 1024)
    print(f"{name}: rc={rc} err={err!r}", flush=True)
    assert rc == case["rc"] and err == case["err"]


def q4_slots(g, K, N, grp):
    ng = K // grp
    q = g.integers(0, 16, size=(N, K), dtype=np.uint8)
    wq = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8).reshape(-1)
    sc = (np.abs(g.normal(0, 0.05, N * ng)) + 1e-3).astype(np.float32)
    ze = g.uniform(4, 11, N * ng).astype(np.float32)
    return q4_blob(wq, sc, ze, K, N, ng)


def compare_with_oracle(hip, oracle, prog, mem_len, u8, lut, x):
    """Runs `prog` on both sides with the same slot lengths: same code, same text, same outputs
    (the written ones within the reference's tolerance, the rest untouched)."""
    orc_rc, orc_mem, orc_err = oracle.run_program(prog, mem_len, u8, lut, x)
    mem = hip.DeviceBuffer.from_array(np.zeros(mem_len, np.float32))
    du8 = hip.DeviceBuffer.from_array(u8) if u8 is not None else None
    dlut = hip.DeviceBuffer.from_array(lut) if lut is not None else None
    dx = hip.DeviceBuffer.from_array(x)
    rc, err = dispatch_raw(hip, prog, mem, mem_len, du8, 0 if u8 is None else u8.size, dlut,
                           0 if lut is None else lut.size, dx, x.size)
    print(f"program {list(prog[:6])}: rc={rc} err={err!r} oracle rc={orc_rc} err={orc_err!r}", flush=True)
    assert rc == (0 if orc_rc == 0 else -1)
    assert err == orc_err
    got = mem.read(np.float32)
    written = orc_mem != 0
    if written.any():
        ref_check(got[written], orc_mem[written])
    assert np.all(got[~written] == 0)


@pytest.mark.parametrize("op", [OP_Q4_GEMV, OP_Q4_COOP_GEMM])
@pytest.mark.parametrize("short", ["mem", "mem_mid_row", "x", "u8", "lut", "none"])
def test_q4_out_of_range(hip, oracle, op, short):
    """Q4 shape ops with one slot too short: the reference stops at the first output whose inputs
    or store fall outside its slots, after writing the ones before it."""
    g = synth.rng(8100 + op)
    M, K, N, grp = 6, 256, 48, 32
    u8, f32 = q4_slots(g, K, N, grp)
    x = synth.activations(g, M, K, np.float32).reshape(-1)
    mem_len = M * N
    if short == "mem":
        mem_len = 3 * N
    elif short == "mem_mid_row":
        mem_len = 2 * N + 17
    elif short == "x":
        x = x[: 4 * K + 100]
    elif short == "u8":
        u8 = u8[: 20 * (K // 2) + 5]
    elif short == "lut":
        f32 = f32[: f32.size - (N - 30) * (K // grp)]
    compare_with_oracle(hip, oracle, shape_op_program(op, M, K, N, grp, K // grp), mem_len, u8, f32, x)


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("short", ["mem", "x", "none"])
def test_tile_gemm_out_of_range(hip, oracle, fmt, short):
    """OP_TILE_GEMM formats 0 and 1 with too small an output or input slot."""
    g = synth.rng(8200 + fmt)
    M, K, N = 5, 128, 40
    x = synth.activations(g, M, K, np.float32).reshape(-1)
    if fmt == 0:
        codes = g.integers(0, 16, size=(N, K), dtype=np.uint8)
        sb = g.integers(120, 132, size=(N, K // 32), dtype=np.uint8)
        u8 = np.concatenate([synth.fp4km_pack(codes).reshape(-1), sb.reshape(-1)])
        lut = synth.mx_table()
        lut[16 + 255] = 0.0  # the golden table's NaN byte is never used here
        prog = fp4_tile_program(M, K, N, N * (K // 2), 0)
    else:
        u8 = (g.standard_normal((N, K)) * 2).astype(np.float16).view(np.uint8).reshape(-1)
        lut = None
        prog = f16_tile_program(M, K, N)
    mem_len = M * N
    if short == "mem":
        mem_len = 2 * N + 7
    elif short == "x":
        x = x[: 3 * K]
    compare_with_oracle(hip, oracle, prog, mem_len, u8, lut, x)


@pytest.mark.parametrize("short", ["mem", "lut", "none"])
def test_fp4_coop_out_of_range(hip, oracle, short):
    """The legacy OP_FP4_COOP_GEMM one-blob op with a short output or blob."""
    g = synth.rng(8300)
    M, K, N = 4, 128, 32
    codes = g.integers(0, 16, size=(N, K), dtype=np.uint8)
    sb = g.integers(120, 132, size=(N, K // 32), dtype=np.uint8)
    packed = np.concatenate([synth.fp4km_pack(codes).reshape(-1), sb.reshape(-1)])
    words = np.zeros((packed.size + 3) // 4, np.float32)
    words.view(np.uint8)[: packed.size] = packed
    lw = fp4_coop_lut_word(K, N)
    blob = np.zeros(lw + 272, np.float32)
    blob[: min(lw, words.size)] = words[:lw]
    table = synth.mx_table()
    table[16 + 255] = 0.0
    blob[lw:] = table
    x = synth.activations(g, M, K, np.float32).reshape(-1)
    mem_len = M * N if short != "mem" else N + 5
    if short == "lut":
        blob = blob[:-1]
    u8 = blob.view(np.uint8).copy()
    compare_with_oracle(hip, oracle, shape_op_program(OP_FP4_COOP_GEMM, M, K, N, 32, K // 32), mem_len, u8, blob, x)


def test_missing_slots_and_trailing_ops(hip):
    """A missing weight slot is the reference's 'slot is missing'; an op after the shape op that is
    not a tile op has no HIP route (BYHIP_UNSUPPORTED, nothing written)."""
    x = hip.DeviceBuffer.from_array(np.ones(256, np.float32))
    mem = hip.DeviceBuffer.from_array(np.zeros(64, np.float32))
    rc, err = dispatch_raw(hip, shape_op_program(OP_Q4_GEMV, 1, 64, 16, 32, 2), mem, 64, None, 0, None, 0, x, 256)
    assert rc == -1 and err == "CPU VM Q4 cooperative slot is missing"
    rc, err = dispatch_raw(hip, fp4_tile_program(1, 64, 16, 512, 0), mem, 64, None, 0, None, 0, x, 256)
    assert rc == -1 and err == "CPU VM tile GEMM slot is missing"
    g = synth.rng(8400)
    u8, f32 = q4_slots(g, 64, 16, 32)
    prog = list(shape_op_program(OP_Q4_GEMV, 1, 64, 16, 32, 2))
    prog = prog[:6] + [0x20, 1]  # an arithmetic op, then HALT
    rc, err = dispatch_raw(hip, prog, mem, 64, hip.DeviceBuffer.from_array(u8), u8.size,
                           hip.DeviceBuffer.from_array(f32), f32.size, x, 256)
    assert rc == _abi.BYHIP_UNSUPPORTED
    assert np.all(mem.read(np.float32) == 0)
