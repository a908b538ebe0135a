"""Writes the golden fixtures of the quantized tile-GEMM path from the reference's own C.

Run in a container where /root/reference exists (`make -C oracle` builds oracle/_ref first):

    python tests/golden/make_golden.py

Every expected output here comes from the reference's CPU backend compiled from its sources
(backends/cpu/cpu_vm.c nimf_cpu_vm_run_slots, backends/cpu/cpu_kernels.c nimf_cpu_matmul_q4)
through oracle/_ref/libbybyref.so, called the way tests/t_fp4_tile_gemm.nim:69-80 calls it
(128 threads, threadgroups of 128, 64 threadgroup floats). The inputs are stored beside the
outputs so the fixtures stand alone; the FP4-KM and FP16 inputs are the reference test's own
(xorshift32 seed 2463534242, t_fp4_tile_gemm.nim:30-51, 198-223).

Files (numpy .npz, no pickles):
  fp4km_cases.npz  the five FP4-KM cases: inputs, OP_TILE_GEMM output (dynamic rows), the
                   legacy OP_FP4_COOP_GEMM output on the one-blob layout
  f16_cases.npz    the five FP16 tile-GEMM cases: inputs and outputs
  q4_cases.npz     Q4 shape ops (OP_Q4_GEMV, OP_Q4_COOP_GEMM) and matmul_q4 on asymmetric
                   reference-format weights and on the symmetric block-32 fp16-scale format
  errors.json      the reference's error text for rejected programs
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

from oracle_lib import (OP_FP4_COOP_GEMM, OP_Q4_COOP_GEMM, OP_Q4_GEMV, Oracle, Reference,  # noqa: E402
                        f16_tile_program, fp4_cases, fp4_coop_lut_word, fp4_tile_program,
                        q4_blob, shape_op_program)


def legacy_blob(packed, table, K, N):
    """The legacy shape op's one blob (t_fp4_tile_gemm.nim:89-95): packed bytes as words,
    padded to fp4CoopLutWord, then the 272-float table."""
    words = np.zeros((packed.size + 3) // 4, dtype=np.float32)
    words.view(np.uint8)[: packed.size] = packed
    lut_word = fp4_coop_lut_word(K, N)
    blob = np.zeros(lut_word + 272, dtype=np.float32)
    blob[: min(lut_word, words.size)] = words[:lut_word]
    blob[lut_word:] = table
    return blob


def q4_case(rng, M, K, N, group, symmetric):
    ng = K // group
    if symmetric:
        codes = rng.integers(-8, 8, size=(N, K))
        q = (codes + 8).astype(np.uint8)
        scales = (np.abs(rng.normal(0.0, 0.02, size=(N, ng))) + 1e-4).astype(np.float16)
        scales = scales.astype(np.float32)
        zeros = np.full((N, ng), 8.0, dtype=np.float32)
    else:
        q = rng.integers(0, 16, size=(N, K)).astype(np.uint8)
        scales = (rng.random((N, ng)) * 0.05 + 1e-3).astype(np.float32)
        zeros = (rng.random((N, ng)) * 15.0).astype(np.float32)
    wq = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8).reshape(-1)
    x = rng.standard_normal(M * K).astype(np.float32)
    return x, wq, scales.reshape(-1), zeros.reshape(-1)


def main() -> None:
    if not Reference.available():
        raise SystemExit("oracle/_ref/libbybyref.so is missing: run `make -C oracle` where "
                         "/root/reference exists")
    ref = Reference()
    orc = Oracle()
    cases, f16 = fp4_cases(orc)

    out = {}
    for i, c in enumerate(cases):
        M, K, N = c["M"], c["K"], c["N"]
        rc, mem, err = ref.run_program(fp4_tile_program(0, K, N, N * (K // 2), 0), M * N,
                                       c["packed"], c["table"], c["x"])
        assert rc == 0, err
        out[f"shape_{i}"] = np.array([M, K, N], dtype=np.int64)
        out[f"x_{i}"] = c["x"]
        out[f"packed_{i}"] = c["packed"]
        out[f"out_{i}"] = mem
        if K % 64 == 0 and N >= 16:
            blob = legacy_blob(c["packed"], c["table"], K, N)
            prog = shape_op_program(OP_FP4_COOP_GEMM, M, K, N, 32, K // 32)
            rc, mem2, err = ref.run_program(prog, M * N, blob.view(np.uint8).copy(), blob, c["x"])
            assert rc == 0, err
            out[f"legacy_{i}"] = mem2
    out["table"] = cases[0]["table"]
    np.savez_compressed(os.path.join(HERE, "fp4km_cases.npz"), **out)

    out = {}
    for i, c in enumerate(f16):
        M, K, N = c["M"], c["K"], c["N"]
        rc, mem, err = ref.run_program(f16_tile_program(0, K, N), M * N, c["halves"],
                                       np.zeros(1, np.float32), c["x"])
        assert rc == 0, err
        out[f"shape_{i}"] = np.array([M, K, N], dtype=np.int64)
        out[f"x_{i}"] = c["x"]
        out[f"halves_{i}"] = c["halves"]
        out[f"out_{i}"] = mem
    np.savez_compressed(os.path.join(HERE, "f16_cases.npz"), **out)

    # Q4: (M, K, N, group, symmetric). Symmetric = the block-32 fp16-scale format of the
    # benchmark configurations (q = code + 8, zero 8.0, scale = float(fp16)).
    shapes = [(1, 64, 16, 32, True), (1, 4096, 16, 32, True), (3, 256, 40, 32, True),
              (16, 128, 64, 32, True), (1, 64, 16, 32, False), (5, 128, 24, 16, False),
              (17, 256, 48, 64, False), (2, 192, 33, 64, False), (1, 40, 9, 8, False),
              (33, 128, 20, 128, True)]
    rng = np.random.default_rng(20240607)
    out = {}
    for i, (M, K, N, g, sym) in enumerate(shapes):
        ng = K // g
        x, wq, sc, ze = q4_case(rng, M, K, N, g, sym)
        u8, f32 = q4_blob(wq, sc, ze, K, N, ng)
        out[f"shape_{i}"] = np.array([M, K, N, g, int(sym)], dtype=np.int64)
        out[f"x_{i}"], out[f"wq_{i}"], out[f"scales_{i}"], out[f"zeros_{i}"] = x, wq, sc, ze
        rc, mem, err = ref.run_program(shape_op_program(OP_Q4_GEMV, M, K, N, g, ng), M * N,
                                       u8, f32, x)
        assert rc == 0, err
        out[f"gemv_{i}"] = mem
        if N >= 16 and K % 64 == 0 and g % 2 == 0:
            rc, mem, err = ref.run_program(shape_op_program(OP_Q4_COOP_GEMM, M, K, N, g, ng),
                                           M * N, u8, f32, x)
            assert rc == 0, err
            out[f"coop_{i}"] = mem
        out[f"matmul_{i}"] = ref.matmul_q4(x, wq, sc, ze, M, K, N, g, ng).reshape(-1)
    np.savez_compressed(os.path.join(HERE, "q4_cases.npz"), **out)

    # Rejected programs: the reference's messages (error behaviour of the drop-in boundary).
    errors = {}
    blob = np.zeros(4096, dtype=np.float32)
    x = np.zeros(1024, dtype=np.float32)
    probes = {
        "q4_coop_narrow": shape_op_program(OP_Q4_COOP_GEMM, 1, 64, 8, 32, 2),
        "q4_gemv_group": shape_op_program(OP_Q4_GEMV, 1, 64, 16, 12, 5),
        "q4_gemv_range": shape_op_program(OP_Q4_GEMV, 4, 256, 64, 32, 8),
        "fp4_coop_shape": shape_op_program(OP_FP4_COOP_GEMM, 1, 96, 16, 32, 3),
        "tile_bad_k": fp4_tile_program(1, 48, 16, 0, 0),
        "tile_range": fp4_tile_program(4, 256, 64, 64 * 128, 0),
        "tile_truncated": np.array([0xB0, 1, 64], dtype=np.uint32),
    }
    for name, prog in probes.items():
        rc, _, err = ref.run_program(prog, 64, blob.view(np.uint8).copy(), blob, x)
        errors[name] = {"rc": rc, "err": err, "program": [int(w) for w in prog]}
    with open(os.path.join(HERE, "errors.json"), "w") as f:
        json.dump(errors, f, indent=1)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
