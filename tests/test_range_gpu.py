"""Inputs outside fp16's range, on every route, against the oracle at the reference's tolerance.

The reference computes in fp32 for any decode table, any scales and any activations
(cpu_vm.c:583-628, cpu_kernels_impl.inc:293-319); its own test draws its tables at random
(t_fp4_tile_gemm.nim:35-44). The HIP routes must give the same numbers wherever the data lies:
  - fp32 activations spanning 1e-8 .. 1e6 on the decode GEMV (1, 2, 4 and 8 chunks per lane, so
    K up to 14336), the fused GEMV, the fp16 MFMA GEMM and the wide tile over two fp16 activation
    planes, which fp32 decode rows take from M = 3 (per-row power-of-two shift, weight
    remainders);
  - Q4 scales whose weights leave fp16's range (the exact fp32 GEMM);
  - FP4-KM tables whose products are not halves: every E8M0 byte 0..254, normal-distributed scale
    tables, arbitrary fp32 value tables (the exact fp32 GEMM).
Bar: max|diff| <= 1e-4 * max(1, peak) (t_fp4_tile_gemm.nim:53-67); the E8M0 sweep holds each
column to 1e-4 of its own peak, so the columns with tiny scales are checked as strictly.
"""
import numpy as np
import pytest

from bybylang_amd import synth
from oracle_lib import OP_Q4_COOP_GEMM, OP_Q4_GEMV, f16_tile_program, q4_blob, shape_op_program
from parity import REF_TOL, bf16_bits_to_f32, f32_to_bf16_rne, ref_check

pytestmark = pytest.mark.gpu


def wide_x(g, M, K, lo=-8.0, hi=6.0):
    """Activations with magnitudes log-uniform over 10^lo .. 10^hi and random signs."""
    mag = 10.0 ** g.uniform(lo, hi, size=(M, K))
    return (np.where(g.random((M, K)) < 0.5, -1.0, 1.0) * mag).astype(np.float32)


def run_q4(hip, x, x_dtype, w, M, N, y_dtype=None):
    y_dtype = hip.F32 if y_dtype is None else y_dtype
    xd = hip.DeviceBuffer.from_array(np.ascontiguousarray(x).reshape(-1))
    yd = hip.DeviceBuffer(M * N * (4 if y_dtype == hip.F32 else 2))
    hip.q4_matmul(xd, x_dtype, w, yd, y_dtype, M)
    return yd.read(hip.np_dtype(y_dtype), M * N).astype(np.float32).reshape(M, N)


@pytest.mark.parametrize("x_kind", ["f32_wide", "f32", "f16"])
@pytest.mark.parametrize("K", [2048, 4096, 8192, 14336])
@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_gemv_chunks_and_range(hip, oracle, monkeypatch, M, K, x_kind):
    """The decode GEMV at 1, 2, 4 and 8 chunks per lane (K = 2048 .. 14336), M = 1 .. 8, fp16 and
    fp32 activations (fp32 also over 1e-8 .. 1e6), forced onto the GEMV route."""
    g = synth.rng(7000 + M * 31 + K)
    N = 384
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    if x_kind == "f32_wide":
        x = wide_x(g, M, K)
    else:
        x = synth.activations(g, M, K, np.float32)
    xt = hip.F16 if x_kind == "f16" else hip.F32
    xin = x.astype(np.float16) if x_kind == "f16" else x
    print(f"gemv M={M} K={K} x={x_kind}", flush=True)
    w = hip.Q4Weights(wq, sc, ze, K, N, 32, K // 32)
    monkeypatch.setenv("BYHIP_Q4_ROUTE", "1")
    got = run_q4(hip, xin, xt, w, M, N)
    want = oracle.matmul_q4(np.asarray(xin, np.float32).reshape(-1), wq, sc, ze, M, K, N, 32, K // 32)
    ref_check(got, want)


@pytest.mark.parametrize("M", [2, 16])
def test_gemv_chunk_extremes(hip, oracle, M):
    """A chunk holding 1e6 next to 1e-30, a zero and an fp32 subnormal; chunks of subnormals, of
    values near 1e30 and near 1e-30: the per-chunk (GEMV, M = 2) and per-row (GEMM, M = 16) shifts
    keep every finite value. Each row is checked against its own peak."""
    g = synth.rng(7100 + M)
    K, N = 512, 256
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    x = synth.activations(g, M, K, np.float32)
    x[0, :32] = 1e-30
    x[0, 5] = 1e6
    x[0, 7] = 0.0
    x[0, 9] = 1e-41  # an fp32 subnormal
    x[0, 32:64] *= np.float32(1e-39)
    x[1, 96:] *= np.float32(1e30)
    x[M - 1, :] *= np.float32(1e-30)
    w = hip.Q4Weights(wq, sc, ze, K, N, 32, K // 32)
    want = oracle.matmul_q4(x.reshape(-1), wq, sc, ze, M, K, N, 32, K // 32)
    got = run_q4(hip, x, hip.F32, w, M, N)
    for m in range(M):
        peak = float(np.max(np.abs(want[m])))
        assert np.all(np.isfinite(got[m]))
        assert float(np.max(np.abs(got[m].astype(np.float64) - want[m]))) <= REF_TOL * peak, f"row {m}"


@pytest.mark.parametrize("scale", [1e5, 1e-6])
@pytest.mark.parametrize("mode", [0, 1])
def test_fused_input_far_from_unit_norm(hip, oracle, mode, scale):
    """sessionMatmulQ4Fused with RMSNorm on an input whose norm is far from 1 (the kernel applies
    the norm factor after the dot products, so the staged a * gamma must keep its range)."""
    g = synth.rng(7200 + mode)
    K, Ns = 4096, ([512, 256] if mode == 0 else [384, 384])
    mats, ws = [], []
    for N in Ns:
        wq, sc, ze, _ = synth.q4_weights(g, N, K)
        mats.append((wq, sc, ze, N))
        ws.append(hip.Q4Weights(wq, sc, ze, K, N, 32, K // 32))
    a = (g.standard_normal(K) * scale).astype(np.float32)
    gamma = (1.0 + 0.1 * g.standard_normal(K)).astype(np.float32)
    res = g.standard_normal(max(Ns)).astype(np.float32)
    outs = [hip.DeviceBuffer(N * 4) for N in Ns]
    rc = hip.q4_matmul_fused(mode, hip.DeviceBuffer.from_array(a), ws, outs, hip.DeviceBuffer.from_array(res),
                             hip.DeviceBuffer.from_array(gamma), 1e-5)
    assert rc == 0
    want = oracle.q4_fused(mode, a, mats, K, 32, K // 32, residual=res, gamma=gamma, eps=1e-5)
    for o, wv, N in zip(outs, want, Ns):
        ref_check(o.read(np.float32, N), wv)


def test_fused_long_rows_wide_input(hip, oracle):
    """Mode 0 at K = 14336 (8 chunks per lane) with activations over 1e-8 .. 1e6, no norm."""
    g = synth.rng(7250)
    K, N = 14336, 256
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    a = wide_x(g, 1, K).reshape(-1)
    out = hip.DeviceBuffer(N * 4)
    w = hip.Q4Weights(wq, sc, ze, K, N, 32, K // 32)
    assert hip.q4_matmul_fused(0, hip.DeviceBuffer.from_array(a), [w], [out]) == 0
    want = oracle.q4_fused(0, a, [(wq, sc, ze, N)], K, 32, K // 32)
    ref_check(out.read(np.float32, N), want[0])


@pytest.mark.parametrize("weights", ["fast", "fp32_scales", "asym_zero"])
@pytest.mark.parametrize("M", [16, 64, 130])
def test_gemm_fp32_activations_wide_range(hip, oracle, M, weights):
    """The fp16 MFMA GEMM with fp32 activations over 1e-8 .. 1e6 (per-row shift onto fp16's range,
    hi + lo activations, the weights' fp16 remainders): the reference's fp32 tolerance."""
    g = synth.rng(7300 + M)
    K, N = 768, 320
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    if weights == "fp32_scales":
        sc = (np.abs(g.normal(0.0, 0.02, size=sc.size)) + 1e-3).astype(np.float32)  # not halves
    elif weights == "asym_zero":
        ze = g.uniform(6.0, 9.0, size=ze.size).astype(np.float32)
    w = hip.Q4Weights(wq, sc, ze, K, N, 32, K // 32)
    assert w.info()["f16_safe"] == 1
    x = wide_x(g, M, K)
    print(f"gemm fp32 wide M={M} weights={weights}", flush=True)
    got = run_q4(hip, x, hip.F32, w, M, N)
    ref_check(got, oracle.matmul_q4(x.reshape(-1), wq, sc, ze, M, K, N, 32, K // 32))


@pytest.mark.parametrize("splits", ["", "1", "2", "5"])
@pytest.mark.parametrize("M", [9, 40])
def test_gemm_fp32_activations_split_k(hip, oracle, monkeypatch, M, splits):
    """The same GEMM on a long K with few tiles, where it splits K (fp32 partial sums added by
    splitk_sum in slice order): the default split (8 slices of 8 steps here), none, and forced
    2 and 5 (unequal slices: 64 steps as 13 + 13 + 13 + 13 + 12), fp32 and fp16 outputs, against
    the oracle at the reference's fp32 tolerance (fp16 outputs after the oracle's own rounding,
    plus one fp16 step)."""
    g = synth.rng(7400 + M + 3 * len(splits))
    K, N = 4096, 384
    monkeypatch.setenv("BYHIP_Q4_SPLIT", splits)
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    ze = g.uniform(6.0, 9.0, size=ze.size).astype(np.float32)  # per-group zeros: the generic kernel
    w = hip.Q4Weights(wq, sc, ze, K, N, 32, K // 32)
    x = wide_x(g, M, K, -3.0, 3.0)
    want = oracle.matmul_q4(x.reshape(-1), wq, sc, ze, M, K, N, 32, K // 32)
    print(f"gemm fp32 split-K M={M} splits={splits or 'default'}", flush=True)
    ref_check(run_q4(hip, x, hip.F32, w, M, N), want)
    got16 = run_q4(hip, x, hip.F32, w, M, N, hip.F16)
    # both roundings to fp16 may land one fp16 step apart: at most 2^-10 of the peak
    ref_check(got16, np.asarray(want, np.float32).astype(np.float16).astype(np.float32), REF_TOL + 2.0 ** -10)


@pytest.mark.parametrize("splits", ["", "1", "3"])
@pytest.mark.parametrize("M", [2, 3, 5, 8, 9, 16, 17, 40, 130, 512])
def test_gemm_fp32_activations_wide_tile(hip, oracle, monkeypatch, M, splits):
    """fp32 activations on weights with a prefill copy (fp16 scales, one zero): the 16- or 32-row
    wide tile on the activations' two fp16 planes (hi . w_hi + lo . w_hi + hi . w_lo), with the
    default K split, none, and 3 slices (rounded to whole rounds of the four K groups), ragged N
    (320 = 2.5 column tiles) and M (decode rows 3 .. 8, which take the tile from M = 3, and 17,
    130); activations over 1e-8 .. 1e6 against the oracle at the reference's fp32 tolerance, and
    the same rows with the wide tile switched off (BYHIP_Q4_F32_WIDE=0: the GEMV up to M = 8, the
    generic GEMM above) to the same bar."""
    g = synth.rng(7500 + M + 7 * len(splits))
    K, N = 2048, 320
    monkeypatch.setenv("BYHIP_Q4_SPLIT", splits)
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    w = hip.Q4Weights(wq, sc, ze, K, N, 32, K // 32)
    x = wide_x(g, M, K)
    want = oracle.matmul_q4(x.reshape(-1), wq, sc, ze, M, K, N, 32, K // 32)
    print(f"gemm fp32 wide tile M={M} splits={splits or 'default'}", flush=True)
    ref_check(run_q4(hip, x, hip.F32, w, M, N), want)
    monkeypatch.setenv("BYHIP_Q4_F32_WIDE", "0")
    ref_check(run_q4(hip, x, hip.F32, w, M, N), want)


@pytest.mark.parametrize("M", [2, 4, 8])
def test_fp32_decode_rows_long_k(hip, oracle, M):
    """fp32 decode rows at c4's down-projection K (14336, where one GEMV launch holds one row):
    from M = 2 they take the wide tile; activations over 1e-8 .. 1e6 against the oracle at the
    reference's fp32 tolerance."""
    g = synth.rng(7550 + M)
    K, N = 14336, 256
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    w = hip.Q4Weights(wq, sc, ze, K, N, 32, K // 32)
    x = wide_x(g, M, K)
    print(f"fp32 decode rows M={M} K={K}", flush=True)
    ref_check(run_q4(hip, x, hip.F32, w, M, N), oracle.matmul_q4(x.reshape(-1), wq, sc, ze, M, K, N, 32, K // 32))


@pytest.mark.parametrize("tile", ["", "1", "0"])
@pytest.mark.parametrize("K,N", [(4096, 320), (14336, 256)])
@pytest.mark.parametrize("M", [2, 3, 5, 8])
def test_fp16_decode_rows_exact_weights(hip, oracle, monkeypatch, M, K, N, tile):
    """fp16 decode rows on the wide tile with each weight as two fp16 terms that add up to it
    (past 4 rows, or past what one GEMV launch holds: one row at K = 14336), forced onto it
    (BYHIP_Q4_DECODE_TILE=1) and off it (0: the GEMV); the weights stay exact, so the bar is the
    reference's fp32 tolerance against the oracle on the fp16 activations."""
    g = synth.rng(7560 + M + K)
    monkeypatch.setenv("BYHIP_Q4_DECODE_TILE", tile)
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    w = hip.Q4Weights(wq, sc, ze, K, N, 32, K // 32)
    xh = synth.activations(g, M, K, np.float16)
    want = oracle.matmul_q4(xh.astype(np.float32).reshape(-1), wq, sc, ze, M, K, N, 32, K // 32)
    print(f"fp16 decode rows M={M} K={K} tile={tile or 'default'}", flush=True)
    ref_check(run_q4(hip, xh, hip.F16, w, M, N), want)
    got16 = run_q4(hip, xh, hip.F16, w, M, N, hip.F16)
    ref_check(got16, np.asarray(want, np.float32).astype(np.float16).astype(np.float32), REF_TOL + 2.0 ** -10)


@pytest.mark.parametrize("y", ["f16", "bf16"])
@pytest.mark.parametrize("M", [3, 12, 64])
def test_gemm_fp32_activations_wide_tile_half_outputs(hip, oracle, M, y):
    """The fp32-activation wide tile writing fp16 and bf16 outputs: the oracle's fp32 result
    rounded to the output type, plus one step of that type (both roundings may land a step apart:
    2^-10 of the peak for fp16, 2^-7 for bf16)."""
    g = synth.rng(7600 + M)
    K, N = 4096, 384
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    w = hip.Q4Weights(wq, sc, ze, K, N, 32, K // 32)
    x = wide_x(g, M, K, -3.0, 3.0)
    want = np.asarray(oracle.matmul_q4(x.reshape(-1), wq, sc, ze, M, K, N, 32, K // 32), np.float32)
    print(f"gemm fp32 wide tile M={M} y={y}", flush=True)
    if y == "f16":
        got = run_q4(hip, x, hip.F32, w, M, N, hip.F16)
        ref_check(got, want.astype(np.float16).astype(np.float32), REF_TOL + 2.0 ** -10)
    else:
        xd = hip.DeviceBuffer.from_array(np.ascontiguousarray(x).reshape(-1))
        yd = hip.DeviceBuffer(M * N * 2)
        hip.q4_matmul(xd, hip.F32, w, yd, hip.BF16, M)
        got = bf16_bits_to_f32(yd.read(np.uint16, M * N)).reshape(M, N)
        ref_check(got, f32_to_bf16_rne(want), REF_TOL + 2.0 ** -7)


@pytest.mark.parametrize("scales", ["tiny", "huge", "mixed"])
@pytest.mark.parametrize("M", [3, 40])
def test_q4_scales_outside_fp16(hip, oracle, M, scales):
    """Scales whose weights fall below fp16's normal range or overflow it: the upload marks the
    weights unsafe for fp16 and the exact fp32 GEMM (M > 8) or the GEMV (M <= 8) runs them."""
    g = synth.rng(7400 + M)
    K, N = 512, 200
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    base = np.abs(g.normal(0.0, 1.0, size=sc.size)).astype(np.float32) + 0.1
    if scales == "tiny":
        sc = (base * 1e-9).astype(np.float32)
    elif scales == "huge":
        sc = (base * 1e5).astype(np.float32)
    else:
        sc = (base * np.where(g.random(sc.size) < 0.5, 1e-9, 1e5)).astype(np.float32)
    w = hip.Q4Weights(wq, sc, ze, K, N, 32, K // 32)
    assert w.info()["f16_safe"] == 0
    x = synth.activations(g, M, K, np.float32)
    got = run_q4(hip, x, hip.F32, w, M, N)
    ref_check(got, oracle.matmul_q4(x.reshape(-1), wq, sc, ze, M, K, N, 32, K // 32))
    # fp16 activations too (the exact route widens them)
    xh = x.astype(np.float16)
    got = run_q4(hip, xh, hip.F16, w, M, N)
    ref_check(got, oracle.matmul_q4(xh.astype(np.float32).reshape(-1), wq, sc, ze, M, K, N, 32, K // 32))


def fp4km_case(g, M, K, N, table, scale_bytes=None, codes=None):
    if codes is None:
        codes = g.integers(0, 16, size=(N, K), dtype=np.uint8)
    if scale_bytes is None:
        scale_bytes = g.integers(0, 256, size=(N, K // 32), dtype=np.uint8)
    packed = np.concatenate([synth.fp4km_pack(codes).reshape(-1), scale_bytes.reshape(-1)])
    return packed, np.asarray(table, np.float32)


def run_fp4km(hip, x, packed, table, M, K, N, x_dtype=None):
    x_dtype = hip.F32 if x_dtype is None else x_dtype
    yd = hip.DeviceBuffer(M * N * 4)
    hip.fp4km_tile_gemm(hip.DeviceBuffer.from_array(np.ascontiguousarray(x).reshape(-1)), x_dtype,
                        hip.DeviceBuffer.from_array(packed), N * (K // 2), hip.DeviceBuffer.from_array(table), 0,
                        yd, hip.F32, M, K, N)
    return yd.read(np.float32, M * N).reshape(M, N)


@pytest.mark.parametrize("half", ["low", "high"])
def test_fp4km_every_e8m0_byte(hip, oracle, half):
    """The E2M1 / E8M0 table with every scale byte 0..254 (column n uses byte n, or 128 + n): the
    products span 2^-128 .. 1.5 * 2^128 and the exact route keeps each column to 1e-4 of its own
    peak. The high bytes run with activations scaled by 2^-100 so the sums stay finite."""
    g = synth.rng(7500 + (half == "high"))
    M, K = 24, 128
    table = synth.mx_table()
    first, count = (0, 128) if half == "low" else (128, 127)
    N = count
    sb = np.repeat((first + np.arange(N, dtype=np.int64)).astype(np.uint8)[:, None], K // 32, axis=1)
    codes = g.integers(0, 16, size=(N, K), dtype=np.uint8)
    # bytes 253 and 254: 4 and 6 times 2^126 overflow fp32 in the table product itself (the
    # reference's weight is inf there); those columns use the codes of magnitude <= 1.5
    top = (first + np.arange(N)) >= 253
    codes[top] = (codes[top] & 3) | (codes[top] & 8)
    packed, table = fp4km_case(g, M, K, N, table, sb, codes)
    x = synth.activations(g, M, K, np.float32)
    if half == "high":
        x = (x * np.float32(2.0 ** -100)).astype(np.float32)
    got = run_fp4km(hip, x, packed, table, M, K, N)
    want = oracle.tile_gemm(0, M, K, N, N * (K // 2), 0, packed, table, x.reshape(-1))
    assert np.all(np.isfinite(want))
    ref_check(got, want)  # the reference test's bar over the whole output
    # Each column against its own peak where the products are normal fp32 (bytes >= 24; below, a
    # product of a small activation and a 2^-100 weight is an fp32 subnormal, an absolute 2^-149
    # matter). The low columns' relative errors are printed.
    peak = np.max(np.abs(want), axis=0)
    err = np.max(np.abs(got.astype(np.float64) - want.astype(np.float64)), axis=0)
    rel = err / np.maximum(peak, 1e-45)
    byte = first + np.arange(N)
    low = byte < 24
    if low.any():
        print("relative error by scale byte (< 24):", dict(zip(byte[low].tolist(), np.round(rel[low], 8).tolist())))
    bad = np.nonzero((rel > REF_TOL) & ~low)[0]
    assert bad.size == 0, f"scale bytes {byte[bad][:8]}: err {err[bad][:4]} peak {peak[bad][:4]}"


@pytest.mark.parametrize("table_kind", ["normal_scales", "random_values", "reference_test"])
@pytest.mark.parametrize("M", [1, 5, 37, 96])
def test_fp4km_tables(hip, oracle, M, table_kind):
    """Tables whose products are not halves (normal-distributed scales as in
    test_oracle.py:test_random_shapes_against_reference; arbitrary fp32 values) take the exact
    route; the reference test's table (1 + i mod 13) / 64 takes the fp16 MFMA route. Activations
    over 1e-8 .. 1e6 in fp32 and N(0, 1) in fp16."""
    g = synth.rng(7600 + M)
    K, N = 256, 136
    table = np.zeros(272, np.float32)
    table[:16] = synth.E2M1
    if table_kind == "normal_scales":
        table[16:] = g.standard_normal(256).astype(np.float32)
    elif table_kind == "random_values":
        table[:16] = (g.standard_normal(16) * 3).astype(np.float32)
        table[16:] = np.exp(g.normal(0, 2, 256)).astype(np.float32)
    else:
        table[16:] = (1 + np.arange(256) % 13).astype(np.float32) / 64
    packed, table = fp4km_case(g, M, K, N, table)
    x = wide_x(g, M, K)
    got = run_fp4km(hip, x, packed, table, M, K, N)
    ref_check(got, oracle.tile_gemm(0, M, K, N, N * (K // 2), 0, packed, table, x.reshape(-1)))
    xh = synth.activations(g, M, K, np.float16)
    got = run_fp4km(hip, xh, packed, table, M, K, N, hip.F16)
    ref_check(got, oracle.tile_gemm(0, M, K, N, N * (K // 2), 0, packed, table, xh.astype(np.float32).reshape(-1)))


@pytest.mark.parametrize("M", [3, 70])
def test_f16_tile_wide_activations(hip, oracle, M):
    """FP16 weights (exact halves) with fp32 activations over 1e-8 .. 1e6, through the program
    route's OP_TILE_GEMM format 1."""
    g = synth.rng(7700 + M)
    K, N = 320, 96
    w = (g.standard_normal((N, K)) * 4).astype(np.float16)
    halves = w.view(np.uint8).reshape(-1)
    x = wide_x(g, M, K)
    mem = hip.DeviceBuffer(M * N * 4)
    hip.program_dispatch(f16_tile_program(M, K, N), mem, hip.DeviceBuffer.from_array(halves), None,
                         hip.DeviceBuffer.from_array(x.reshape(-1)))
    want = oracle.tile_gemm(1, M, K, N, 0, 0, halves, None, x.reshape(-1))
    ref_check(mem.read(np.float32), want)


@pytest.mark.parametrize("op", [OP_Q4_GEMV, OP_Q4_COOP_GEMM])
@pytest.mark.parametrize("M", [9, 16, 40])
def test_q4_program_route_exact(hip, oracle, op, M):
    """The micro-VM Q4 shape ops above the GEMV's rows: fp32 arithmetic as in the reference (the
    exact GEMM), asymmetric fp32 scales and zeros, wide activations, group 64."""
    g = synth.rng(7800 + M + op)
    K, N, grp = 512, 96, 64
    ng = K // grp
    q = g.integers(0, 16, size=(N, K), dtype=np.uint8)
    wq = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8).reshape(-1)
    sc = (np.abs(g.normal(0, 0.05, N * ng)) + 1e-3).astype(np.float32)
    ze = g.uniform(4, 11, N * ng).astype(np.float32)
    u8, f32 = q4_blob(wq, sc, ze, K, N, ng)
    x = wide_x(g, M, K, -4, 4)
    mem = hip.DeviceBuffer(M * N * 4)
    hip.program_dispatch(shape_op_program(op, M, K, N, grp, ng), mem, hip.DeviceBuffer.from_array(u8),
                         hip.DeviceBuffer.from_array(f32), hip.DeviceBuffer.from_array(x.reshape(-1)))
    want = oracle.q4_shape_op(op == OP_Q4_COOP_GEMM, M, K, N, grp, ng, u8, f32, x.reshape(-1))
    ref_check(mem.read(np.float32), want)
