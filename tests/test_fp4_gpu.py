"""FP4-KM tile GEMM, native MXFP4 and FP16 tile GEMM on the MI355X against the oracle.

Bar: the reference test's tolerance (max|diff| <= 1e-4 * max(1, peak), t_fp4_tile_gemm.nim:53-67)
for the session and micro-VM routes with fp32 activations; the MXFP4 route's products and
scales are exact, so its fp32 output meets the fp32-accumulate tier (1e-3) and its bf16 output is
compared with the oracle rounded to bf16. Unpacked codes and decoded weights are bit-exact.
"""
import os

import numpy as np
import pytest

from oracle_lib import (OP_FP4_COOP_GEMM, f16_tile_program, fp4_coop_lut_word, fp4_tile_program,
                        shape_op_program)
from parity import (TIER_BF16_OUT, TIER_F32_ACC, bf16_bits_to_f32, f32_to_bf16_rne, max_abs_rel, ref_check,
                    tier_check)

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def case(i):
    g = load("fp4km_cases.npz")
    M, K, N = (int(v) for v in g[f"shape_{i}"])
    return M, K, N, g[f"x_{i}"], g[f"packed_{i}"], g["table"], g[f"out_{i}"], g


@pytest.mark.parametrize("i", range(5))
def test_fp4km_session_route_golden(hip, i):
    """sessionFp4GemmTiledEnc / sessionFp4GemmTensorCore on the reference test's cases."""
    from bybylang_amd import gpubackend as gb
    M, K, N, x, packed, table, want, _ = case(i)
    print(f"fp4km session case {i} M={M} K={K} N={N}", flush=True)
    for enc in (gb.sessionFp4GemmTiledEnc, gb.sessionFp4GemmTensorCore):
        assert gb.sessionBegin(gb.gbHip)
        hx = gb.sessionUpload(gb.gbHip, x)
        words = np.zeros((packed.size + 3) // 4, np.float32)
        words.view(np.uint8)[: packed.size] = packed
        hw = gb.sessionUpload(gb.gbHip, words)
        hl = gb.sessionUpload(gb.gbHip, table)
        o = gb.sessionAllocScratch(gb.gbHip, M * N)
        ok = enc(gb.gbHip, hx, hw, hl, o, M, K, N)
        assert gb.sessionEnd(gb.gbHip), gb.sessionGetLastError(gb.gbHip)
        assert ok
        ref_check(gb.sessionRead(gb.gbHip, o, M * N), want)
        for h in (hx, hw, hl, o):
            gb.sessionFree(gb.gbHip, h)


@pytest.mark.parametrize("i", range(5))
def test_fp4km_program_route_golden(hip, i):
    """OP_TILE_GEMM programs (dynamic rows, fixed rows, a dispatch row count) and the legacy
    OP_FP4_COOP_GEMM one-blob op over the micro-VM slots."""
    M, K, N, x, packed, table, want, g = case(i)
    u8 = hip.DeviceBuffer.from_array(packed)
    lut = hip.DeviceBuffer.from_array(table)
    xin = hip.DeviceBuffer.from_array(x)
    for Mh, rows in ((0, 0), (M, 0), (0, M)):
        mem = hip.DeviceBuffer(M * N * 4)
        hip.program_dispatch(fp4_tile_program(Mh, K, N, N * (K // 2), 0), mem, u8, lut, xin, rows=rows)
        ref_check(mem.read(np.float32), want)
    if f"legacy_{i}" in g:
        words = np.zeros((packed.size + 3) // 4, np.float32)
        words.view(np.uint8)[: packed.size] = packed
        lw = fp4_coop_lut_word(K, N)
        blob = np.zeros(lw + 272, np.float32)
        blob[: min(lw, words.size)] = words[:lw]
        blob[lw:] = table
        b = hip.DeviceBuffer.from_array(blob)
        mem = hip.DeviceBuffer(M * N * 4)
        hip.program_dispatch(shape_op_program(OP_FP4_COOP_GEMM, M, K, N, 32, K // 32), mem, b, b, xin)
        ref_check(mem.read(np.float32), g[f"legacy_{i}"])


@pytest.mark.parametrize("i", range(5))
def test_fp4km_fp16_activations(hip, oracle, i):
    M, K, N, x, packed, table, _, _ = case(i)
    xh = x.astype(np.float16)
    want = oracle.tile_gemm(0, M, K, N, N * (K // 2), 0, packed, table, xh.astype(np.float32))
    y = hip.DeviceBuffer(M * N * 4)
    hip.fp4km_tile_gemm(hip.DeviceBuffer.from_array(xh), hip.F16, hip.DeviceBuffer.from_array(packed),
                        N * (K // 2), hip.DeviceBuffer.from_array(table), 0, y, hip.F32, M, K, N)
    ref_check(y.read(np.float32), want)


@pytest.mark.parametrize("i", range(5))
def test_fp4km_unpack_bit_exact(hip, oracle, i):
    M, K, N, x, packed, table, _, _ = case(i)
    import ctypes as C
    from bybylang_amd import _abi
    codes = np.empty(N * K, np.uint8)
    w = np.empty(N * K, np.float32)
    b = hip.DeviceBuffer.from_array(packed)
    t = hip.DeviceBuffer.from_array(table)
    _abi.check(_abi.load().byhip_debug_unpack_fp4km(b.ptr, N * (K // 2), t.ptr, 0, K, N,
                                                    codes.ctypes.data, w.ctypes.data))
    oc, sb = oracle.unpack_fp4km(packed, N * (K // 2), K, N)
    assert np.array_equal(codes.reshape(N, K), oc)
    want = table[oc] * np.repeat(table[16 + sb.astype(np.int64)], 32, axis=1)
    assert np.array_equal(w.reshape(N, K).view(np.uint32), want.astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("i", range(5))
def test_f16_tile_golden(hip, i):
    """FP16 tile GEMM (format 1): session route and program route (t_fp4_tile_gemm.nim:195-285)."""
    from bybylang_amd import gpubackend as gb
    g = load("f16_cases.npz")
    M, K, N = (int(v) for v in g[f"shape_{i}"])
    x, halves, want = g[f"x_{i}"], g[f"halves_{i}"], g[f"out_{i}"]
    assert gb.sessionBegin(gb.gbHip)
    hx = gb.sessionUpload(gb.gbHip, x)
    hw = gb.sessionUpload(gb.gbHip, halves.view(np.float32))
    o = gb.sessionAllocScratch(gb.gbHip, M * N)
    assert gb.sessionF16GemmTile(gb.gbHip, hx, hw, o, M, K, N, True)
    assert gb.sessionEnd(gb.gbHip)
    ref_check(gb.sessionRead(gb.gbHip, o, M * N), want)
    mem = hip.DeviceBuffer(M * N * 4)
    hip.program_dispatch(f16_tile_program(0, K, N), mem, hip.DeviceBuffer.from_array(halves), None,
                         hip.DeviceBuffer.from_array(x))
    ref_check(mem.read(np.float32), want)


def test_tile_gemm_ready_gates(hip):
    from bybylang_amd import gpubackend as gb
    for f16 in (True, False):
        for tc in (True, False):
            assert gb.sessionTileGemmReady(gb.gbHip, f16, tc)


def mx_case(M, K, N, seed):
    from bybylang_amd import synth
    g = synth.rng(seed)
    xb, xc, xe = synth.mxfp4_operand(g, M, K)
    wb, wc, we = synth.mxfp4_operand(g, N, K)
    return xb, synth.mx_decode(xc, xe), wb, synth.mx_table()


@pytest.mark.parametrize("shape", [(128, 128, 128), (5, 256, 40), (130, 384, 200), (256, 1024, 384)])
@pytest.mark.parametrize("yt", ["f32", "bf16", "f16"])
def test_mxfp4_gemm_against_oracle(hip, oracle, shape, yt):
    """Native scaled-MFMA route. The oracle runs the FP4-KM tile GEMM on the exactly decoded fp32
    activations with the E2M1 / E8M0 table."""
    M, K, N = shape
    xb, xdec, wb, table = mx_case(M, K, N, M * 7 + K)
    want = oracle.tile_gemm(0, M, K, N, N * (K // 2), 0, wb, table, xdec.reshape(-1))
    ycode = {"f32": hip.F32, "bf16": hip.BF16, "f16": hip.F16}[yt]
    y = hip.DeviceBuffer(M * N * (4 if yt == "f32" else 2))
    print(f"mxfp4 {shape} y={yt}", flush=True)
    hip.mxfp4_gemm(hip.DeviceBuffer.from_array(xb), hip.DeviceBuffer.from_array(wb), y, ycode, M, K, N)
    if yt == "f32":
        tier_check(y.read(np.float32), want, TIER_F32_ACC)
        assert max_abs_rel(y.read(np.float32), want) < 1e-5
    elif yt == "bf16":
        got = bf16_bits_to_f32(y.read(np.uint16))
        tier_check(got, f32_to_bf16_rne(want), TIER_F32_ACC)
    else:
        tier_check(y.read(np.float16).astype(np.float32), want.astype(np.float16).astype(np.float32),
                   TIER_F32_ACC)
    # the same product through the tile GEMM entry with MXFP4 activations
    y2 = hip.DeviceBuffer(M * N * 4)
    hip.fp4km_tile_gemm(hip.DeviceBuffer.from_array(xb), hip.MXFP4_KM, hip.DeviceBuffer.from_array(wb),
                        N * (K // 2), hip.DeviceBuffer.from_array(table), 0, y2, hip.F32, M, K, N)
    tier_check(y2.read(np.float32), want, TIER_F32_ACC)


@pytest.mark.parametrize("shape", [(300, 640, 520), (70, 768, 260), (257, 896, 300), (40, 1152, 600),
                                   (520, 1536, 130)])
def test_mxfp4_gemm_pipeline_tails(hip, oracle, shape):
    """K steps (128 deep) of 5, 6, 7, 9 and 12: the step loop runs in groups of four with one to three
    steps after it, and loads come in pairs of steps, so odd counts end on half a pair. M and N are
    not multiples of the 256 x 256 tile. fp32 output against the oracle at 1e-5 (exact products)."""
    M, K, N = shape
    xb, xdec, wb, table = mx_case(M, K, N, 11 * M + N)
    want = oracle.tile_gemm(0, M, K, N, N * (K // 2), 0, wb, table, xdec.reshape(-1))
    y = hip.DeviceBuffer(M * N * 4)
    print(f"mxfp4 tails {shape}", flush=True)
    hip.mxfp4_gemm(hip.DeviceBuffer.from_array(xb), hip.DeviceBuffer.from_array(wb), y, hip.F32, M, K, N)
    got = y.read(np.float32)
    assert np.isfinite(got).all()
    assert max_abs_rel(got, want) < 1e-5


def test_mxfp4_bf16_output_is_rne_of_f32(hip):
    """The bf16 output is the fp32 result rounded to nearest even, bit for bit: both come from the
    same accumulators, so this pins the hardware conversion on the GEMM's own values."""
    M, K, N = 256, 1024, 512
    xb, _, wb, _ = mx_case(M, K, N, 5)
    x, w = hip.DeviceBuffer.from_array(xb), hip.DeviceBuffer.from_array(wb)
    y32, y16 = hip.DeviceBuffer(M * N * 4), hip.DeviceBuffer(M * N * 2)
    hip.mxfp4_gemm(x, w, y32, hip.F32, M, K, N)
    hip.mxfp4_gemm(x, w, y16, hip.BF16, M, K, N)
    f = y32.read(np.float32)
    want = (f32_to_bf16_rne(f).view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(y16.read(np.uint16), want)


def test_mxfp4_route_refuses_other_tables(hip):
    M, K, N = 16, 128, 32
    xb, _, wb, table = mx_case(M, K, N, 1)
    table = table.copy()
    table[16 + 127] = 1.5
    y = hip.DeviceBuffer(M * N * 4)
    with pytest.raises(hip.HipUnsupported):
        hip.fp4km_tile_gemm(hip.DeviceBuffer.from_array(xb), hip.MXFP4_KM,
                            hip.DeviceBuffer.from_array(wb), N * (K // 2),
                            hip.DeviceBuffer.from_array(table), 0, y, hip.F32, M, K, N)


def test_mxfp4_benchmark_config_rows(hip, oracle):
    """Config 3 (M=2048, K=N=8192, bf16 out) on the GPU; 4 rows against the oracle, and a
    K-split checksum: y over all rows equals the sum of two half-K products."""
    M, K, N = 2048, 8192, 8192
    xb, xdec, wb, table = mx_case(M, K, N, 3)
    y = hip.DeviceBuffer(M * N * 4)
    hip.mxfp4_gemm(hip.DeviceBuffer.from_array(xb), hip.DeviceBuffer.from_array(wb), y, hip.F32, M, K, N)
    got = y.read(np.float32).reshape(M, N)
    rows = [0, 1, 1027, M - 1]
    for r in rows:
        want = oracle.tile_gemm(0, 1, K, N, N * (K // 2), 0, wb, table, xdec[r].copy())
        tier_check(got[r], want, TIER_F32_ACC)
    # column sums over all rows against fp64 from the decoded operands (size-independent check)
    from bybylang_amd import synth
    g = synth.rng(3)
    _, xc, xe = synth.mxfp4_operand(g, M, K)
    _, wc, we = synth.mxfp4_operand(g, N, K)
    wdec = synth.mx_decode(wc, we).astype(np.float64)
    colsum = (xdec.astype(np.float64).sum(axis=0) @ wdec.T)
    tier_check(got.astype(np.float64).sum(axis=0), colsum, 1e-4)


def test_mxfp4_benchmark_config_bf16(hip, oracle):
    """Config 3 exactly as the benchmark runs it: M=2048, K=N=8192, bf16 output. 4 rows against the
    oracle rounded to bf16 (one bf16 step on top of the fp32-accumulate tier), the same rows equal to
    the fp32 output rounded to nearest even bit for bit, and the column sums of all rows against an
    fp64 product of the decoded operands."""
    M, K, N = 2048, 8192, 8192
    xb, xdec, wb, table = mx_case(M, K, N, 3)
    x, w = hip.DeviceBuffer.from_array(xb), hip.DeviceBuffer.from_array(wb)
    y16 = hip.DeviceBuffer(M * N * 2)
    print("mxfp4 config 3 bf16", flush=True)
    hip.mxfp4_gemm(x, w, y16, hip.BF16, M, K, N)
    bits = y16.read(np.uint16).reshape(M, N)
    got = bf16_bits_to_f32(bits.reshape(-1)).reshape(M, N)
    rows = [0, 1, 1027, M - 1]
    for r in rows:
        want = oracle.tile_gemm(0, 1, K, N, N * (K // 2), 0, wb, table, xdec[r].copy())
        tier_check(got[r], f32_to_bf16_rne(want).reshape(-1), TIER_BF16_OUT)
    y32 = hip.DeviceBuffer(M * N * 4)
    hip.mxfp4_gemm(x, w, y32, hip.F32, M, K, N)
    f = y32.read(np.float32).reshape(M, N)
    for r in rows:
        assert np.array_equal(bits[r], (f32_to_bf16_rne(f[r]).view(np.uint32) >> 16).astype(np.uint16))
    from bybylang_amd import synth
    g = synth.rng(3)
    _, xc, xe = synth.mxfp4_operand(g, M, K)
    _, wc, we = synth.mxfp4_operand(g, N, K)
    wdec = synth.mx_decode(wc, we).astype(np.float64)
    colsum = xdec.astype(np.float64).sum(axis=0) @ wdec.T
    tier_check(got.astype(np.float64).sum(axis=0), colsum, TIER_BF16_OUT)
