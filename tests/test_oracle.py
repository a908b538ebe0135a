"""The oracle (oracle/byby_oracle.c) pinned against the reference and against closed forms.

- Golden fixtures (tests/golden/, written from the reference's own compiled C): bit-exact.
- oracle/_ref (the reference's C compiled from its sources), when present: bit-exact on random
  shapes, including the CPU benchmark configuration in full.
- Closed forms: data whose sums are exact in fp32 (the reference's parity-gate data), fp64 brute
  force within the accumulated-rounding bound, IEEE binary16 conversions against numpy, and planted
  mistakes that these checks must catch.
"""
import json
import os

import numpy as np
import pytest

from oracle_lib import (FP4_VALUES, OP_FP4_COOP_GEMM, OP_Q4_COOP_GEMM, OP_Q4_GEMV, Oracle,
                        Reference, f16_tile_program, fp4_cases, fp4_coop_lut_word,
                        fp4_tile_program, q4_blob, shape_op_program)

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).reshape(-1).view(np.uint32)


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def legacy_blob(packed, table, K, N):
    words = np.zeros((packed.size + 3) // 4, dtype=np.float32)
    words.view(np.uint8)[: packed.size] = packed
    lw = fp4_coop_lut_word(K, N)
    blob = np.zeros(lw + 272, dtype=np.float32)
    blob[: min(lw, words.size)] = words[:lw]
    blob[lw:] = table
    return blob


# ── generators: the reference test's inputs, reproduced bit for bit ─────────────────────────

def test_generators_reproduce_reference_inputs(oracle):
    g = load("fp4km_cases.npz")
    cases, f16 = fp4_cases(oracle)
    for i, c in enumerate(cases):
        assert np.array_equal(bits(c["x"]), bits(g[f"x_{i}"]))
        assert np.array_equal(c["packed"], g[f"packed_{i}"])
    assert np.array_equal(bits(cases[0]["table"]), bits(g["table"]))
    h = load("f16_cases.npz")
    for i, c in enumerate(f16):
        assert np.array_equal(bits(c["x"]), bits(h[f"x_{i}"]))
        assert np.array_equal(c["halves"], h[f"halves_{i}"])


# ── FP4-KM tile GEMM (cpu_vm.c:583-628) ───────────────────────────────────────────────────────

@pytest.mark.parametrize("i", range(5))
def test_fp4km_tile_gemm_golden(oracle, i):
    g = load("fp4km_cases.npz")
    M, K, N = (int(v) for v in g[f"shape_{i}"])
    x, packed, table = g[f"x_{i}"], g[f"packed_{i}"], g["table"]
    for Mh in (0, M):  # dynamic and fixed rows (t_fp4_tile_gemm.nim:84-87)
        rc, mem, err = oracle.run_program(fp4_tile_program(Mh, K, N, N * (K // 2), 0), M * N,
                                          packed, table, x)
        assert rc == 0, err
        assert np.array_equal(bits(mem), bits(g[f"out_{i}"]))
    if f"legacy_{i}" in g:
        blob = legacy_blob(packed, table, K, N)
        prog = shape_op_program(OP_FP4_COOP_GEMM, M, K, N, 32, K // 32)
        rc, mem, err = oracle.run_program(prog, M * N, blob.view(np.uint8).copy(), blob, x)
        assert rc == 0, err
        assert np.array_equal(bits(mem), bits(g[f"legacy_{i}"]))


@pytest.mark.parametrize("i", range(5))
def test_fp4km_host_reference_within_rounding(oracle, i):
    """tileGemmReference (unfused, tile_gemm.nim:663-677) against the fused VM loop: the two
    differ only by fp32 rounding, bounded by K * 2^-24 * sum |x * w|."""
    g = load("fp4km_cases.npz")
    M, K, N = (int(v) for v in g[f"shape_{i}"])
    x, packed, table = g[f"x_{i}"], g[f"packed_{i}"], g["table"]
    ref = oracle.tile_gemm_reference(x, packed, table, M, K, N, N * (K // 2), 0)
    codes, sb = oracle.unpack_fp4km(packed, N * (K // 2), K, N)
    w = table[codes] * np.repeat(table[16 + sb.astype(np.int64)], 32, axis=1)
    absdot = np.abs(x.reshape(M, K)).astype(np.float64) @ np.abs(w).astype(np.float64).T
    bound = 2 * K * 2.0 ** -24 * absdot + 1e-30
    assert np.all(np.abs(ref.astype(np.float64) - g[f"out_{i}"].reshape(M, N)) <= bound)


def test_fp4km_closed_form_ready_gate_data(oracle):
    """vulkanTileGemmReady's data (vulkan_driver.nim:2697-2731): every product and partial sum is
    exact in fp32, so any summation order must give the exact fp64 value."""
    M, K, N = 37, 128, 80
    x = (((np.arange(M * K) * 7 + 3) % 33) - 16).astype(np.float32) / 64
    table = np.zeros(272, np.float32)
    table[:16] = FP4_VALUES
    table[16:] = np.ldexp(np.float32(1), (np.arange(256) % 5) - 3).astype(np.float32)
    groups = K // 32
    packed = np.zeros(N * (K // 2) + N * groups, np.uint8)
    packed[: N * (K // 2)] = (np.arange(N * (K // 2)) * 37 + 11) % 256
    packed[N * (K // 2):] = (np.arange(N * groups) * 13 + 5) % 256
    codes, sb = oracle.unpack_fp4km(packed, N * (K // 2), K, N)
    w = table[codes].astype(np.float64) * np.repeat(table[16 + sb.astype(np.int64)], 32, axis=1)
    exact = x.reshape(M, K).astype(np.float64) @ w.T
    got = oracle.tile_gemm(0, M, K, N, N * (K // 2), 0, packed, table, x)
    assert np.array_equal(got.astype(np.float64), exact)
    ref = oracle.tile_gemm_reference(x, packed, table, M, K, N, N * (K // 2), 0)
    assert np.array_equal(ref.astype(np.float64), exact)


def test_fp4km_unpack_matches_layout(oracle):
    """Byte j of a 32-value group holds element j (low) and j+16 (high): session_vm.nim:384-388."""
    K, N = 64, 3
    packed = np.arange(N * K // 2 + N * K // 32, dtype=np.int64).astype(np.uint8)
    codes, sb = oracle.unpack_fp4km(packed, N * K // 2, K, N)
    for n in range(N):
        for k in range(K):
            b = packed[n * K // 2 + (k // 32) * 16 + (k % 16)]
            assert codes[n, k] == ((b & 15) if (k % 32) < 16 else (b >> 4))
    assert np.array_equal(sb.reshape(-1), packed[N * K // 2:])


def test_fp4km_planted_mistakes_are_caught(oracle):
    """Swapped nibbles, a wrong table entry or a transposed operand must break parity."""
    g = load("fp4km_cases.npz")
    M, K, N = (int(v) for v in g["shape_3"])
    x, packed, table = g["x_3"], g["packed_3"].copy(), g["table"].copy()
    want = g["out_3"]
    swapped = packed.copy()
    nb = N * (K // 2)
    swapped[:nb] = ((packed[:nb] & 15) << 4) | (packed[:nb] >> 4)
    assert not np.array_equal(bits(oracle.tile_gemm(0, M, K, N, nb, 0, swapped, table, x)), bits(want))
    bad = table.copy()
    bad[3] = -bad[3]
    assert not np.array_equal(bits(oracle.tile_gemm(0, M, K, N, nb, 0, packed, bad, x)), bits(want))
    shifted_scale = oracle.tile_gemm(0, M, K, N, nb, 1, packed, np.concatenate([[0], table]).astype(np.float32), x)
    assert np.array_equal(bits(shifted_scale).reshape(-1), bits(want))  # lut_base is honoured


# ── FP16 tile GEMM (cpu_vm.c:550-582) ────────────────────────────────────────────────────────

@pytest.mark.parametrize("i", range(5))
def test_f16_tile_gemm_golden(oracle, i):
    g = load("f16_cases.npz")
    M, K, N = (int(v) for v in g[f"shape_{i}"])
    for Mh in (0, M):
        rc, mem, err = oracle.run_program(f16_tile_program(Mh, K, N), M * N, g[f"halves_{i}"],
                                          np.zeros(1, np.float32), g[f"x_{i}"])
        assert rc == 0, err
        assert np.array_equal(bits(mem), bits(g[f"out_{i}"]))


def test_half_to_float_all_halves(oracle):
    """cpu_vm.c:53-69 against IEEE binary16 (numpy) for all 65536 bit patterns."""
    hb = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = hb.view(np.float16).astype(np.float32)
    got = np.array([oracle.half_to_float(int(h)) for h in hb], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got[~nan]), bits(want[~nan]))


def test_float_to_half_round_to_nearest_even(oracle):
    r = np.random.default_rng(3)
    f = np.concatenate([r.standard_normal(3000).astype(np.float32) * 10.0 ** r.integers(-8, 6, 3000),
                        np.array([65504, 65519.99, 65520, 6.0e-8, 2.98e-8, 2.9802322e-08, -0.0, 1e-45],
                                 dtype=np.float32)]).astype(np.float32)
    got = np.array([oracle.float_to_half(float(v)) for v in f], dtype=np.uint16)
    assert np.array_equal(got, f.astype(np.float16).view(np.uint16))


# ── Q4 (cpu_vm.c:420-482, cpu_kernels_impl.inc:293-319, gpubackend.nim:288-311) ──────────────

def q4_case(g, i):
    M, K, N, grp, sym = (int(v) for v in g[f"shape_{i}"])
    return M, K, N, grp, g[f"x_{i}"], g[f"wq_{i}"], g[f"scales_{i}"], g[f"zeros_{i}"]


@pytest.mark.parametrize("i", range(10))
def test_q4_golden(oracle, i):
    g = load("q4_cases.npz")
    M, K, N, grp, x, wq, sc, ze = q4_case(g, i)
    ng = K // grp
    u8, f32 = q4_blob(wq, sc, ze, K, N, ng)
    rc, mem, err = oracle.run_program(shape_op_program(OP_Q4_GEMV, M, K, N, grp, ng), M * N, u8, f32, x)
    assert rc == 0, err
    assert np.array_equal(bits(mem), bits(g[f"gemv_{i}"]))
    if f"coop_{i}" in g:
        rc, mem, err = oracle.run_program(shape_op_program(OP_Q4_COOP_GEMM, M, K, N, grp, ng), M * N,
                                          u8, f32, x)
        assert rc == 0, err
        assert np.array_equal(bits(mem), bits(g[f"coop_{i}"]))
    mm = oracle.matmul_q4(x, wq, sc, ze, M, K, N, grp, ng)
    assert np.array_equal(bits(mm), bits(g[f"matmul_{i}"]))


@pytest.mark.parametrize("i", range(10))
def test_q4_fp64_bound(oracle, i):
    """The serial chain is within its rounding bound of the exact (fp64) dot product, and the two
    reference formulas (fused VM loop, unfused matmul_q4) agree to that bound."""
    g = load("q4_cases.npz")
    M, K, N, grp, x, wq, sc, ze = q4_case(g, i)
    codes = oracle.unpack_q4(wq, K, N).astype(np.float32)
    gi = np.arange(K) // grp
    w = (codes - ze.reshape(N, -1)[:, gi]) * sc.reshape(N, -1)[:, gi]  # fp32, as the reference
    X = x.reshape(M, K).astype(np.float64)
    exact = X @ w.astype(np.float64).T
    bound = 2 * K * 2.0 ** -24 * (np.abs(X) @ np.abs(w).astype(np.float64).T) + 1e-30
    assert np.all(np.abs(g[f"gemv_{i}"].reshape(M, N) - exact) <= bound)
    assert np.all(np.abs(g[f"matmul_{i}"].reshape(M, N) - exact) <= bound)
    ref = oracle.matmul_q4_ref(x, wq, sc, ze, M, K, N, grp, K // grp)
    assert np.all(np.abs(ref - exact) <= bound)


def test_q4_unpack_layout(oracle):
    wq = np.array([0x21, 0x43, 0xF0], dtype=np.uint8)
    assert oracle.unpack_q4(wq, 6, 1).tolist() == [[1, 2, 3, 4, 0, 15]]


def test_reference_error_messages(oracle):
    """The reference's error text for rejected programs (golden/errors.json)."""
    with open(os.path.join(GOLDEN, "errors.json")) as f:
        errors = json.load(f)
    blob = np.zeros(4096, dtype=np.float32)
    x = np.zeros(1024, dtype=np.float32)
    for name, e in errors.items():
        rc, _, err = oracle.run_program(np.array(e["program"], np.uint32), 64,
                                        blob.view(np.uint8).copy(), blob, x)
        assert rc == e["rc"] == -1, name
        assert err == e["err"], name


# ── against the reference's own compiled C (oracle/_ref), when it was built ───────────────────

needs_ref = pytest.mark.skipif(not Reference.available(), reason="oracle/_ref not built (reference absent)")


@needs_ref
@pytest.mark.parametrize("seed", range(4))
def test_random_shapes_against_reference(oracle, seed):
    ref = Reference()
    r = np.random.default_rng(100 + seed)
    M = int(r.integers(1, 9))
    K = 64 * int(r.integers(1, 5))
    N = 16 * int(r.integers(1, 5)) + int(r.integers(0, 3))
    x = r.standard_normal(M * K).astype(np.float32)
    packed = r.integers(0, 256, N * K // 2 + N * K // 32, dtype=np.uint8)
    table = np.concatenate([FP4_VALUES, r.standard_normal(256).astype(np.float32)])
    prog = fp4_tile_program(0, K, N, N * K // 2, 0)
    a = oracle.run_program(prog, M * N, packed, table, x)
    b = ref.run_program(prog, M * N, packed, table, x)
    assert a[0] == b[0] == 0 and np.array_equal(bits(a[1]), bits(b[1]))
    grp = [8, 16, 32, 64][int(r.integers(0, 4))]
    ng = K // grp
    wq = r.integers(0, 256, N * K // 2, dtype=np.uint8)
    sc = r.random(N * ng).astype(np.float32)
    ze = (r.random(N * ng) * 16).astype(np.float32)
    u8, f32 = q4_blob(wq, sc, ze, K, N, ng)
    for op in (OP_Q4_GEMV, OP_Q4_COOP_GEMM):
        prog = shape_op_program(op, M, K, N, grp, ng)
        a = oracle.run_program(prog, M * N, u8, f32, x)
        b = ref.run_program(prog, M * N, u8, f32, x)
        assert a[0] == b[0] == 0, (a[2], b[2])
        assert np.array_equal(bits(a[1]), bits(b[1]))
    assert np.array_equal(bits(oracle.matmul_q4(x, wq, sc, ze, M, K, N, grp, ng)),
                          bits(ref.matmul_q4(x, wq, sc, ze, M, K, N, grp, ng)))


@needs_ref
def test_cpu_benchmark_config_against_reference(oracle):
    """Config 0 in full: Q4 M=16, K=N=4096, block-32 fp16 scales, through the Q4 shape op."""
    from bybylang_amd import synth
    g = synth.rng(0)
    M, K, N = 16, 4096, 4096
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    x = synth.activations(g, M, K, np.float32).reshape(-1)
    u8, f32 = q4_blob(wq, sc, ze, K, N, K // 32)
    prog = shape_op_program(OP_Q4_GEMV, M, K, N, 32, K // 32)
    a = oracle.run_program(prog, M * N, u8, f32, x)
    b = Reference().run_program(prog, M * N, u8, f32, x, n_threads=1, tg_size=1)
    assert a[0] == b[0] == 0
    assert np.array_equal(bits(a[1]), bits(b[1]))
