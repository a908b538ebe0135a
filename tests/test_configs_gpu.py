"""The benchmark configurations at full size on the HIP path, against the oracle.

c0  (M = 16, K = N = 4096, fp32 in and out; the reference's CPU-interpreter configuration): through
    the micro-VM route (OP_Q4_GEMV and OP_Q4_COOP_GEMM over the one-blob slots, cpu_vm.c:420-482)
    and through sessionMatmulQ4 (gpubackend.nim:3000-3061), every output at the reference test's
    tolerance, 1e-4 * max(1, peak).
c4  (one decoder layer: qkv 4096 -> 6144, o 4096 -> 4096, gate+up 4096 -> 2 x 14336, down
    14336 -> 4096; M = 1, 32, 256; fp16 activations and outputs): per projection, rows spread over
    the output against the oracle's own loops, and every row against a float64 product of the
    dequantized weights (fp16 output and the weights rounded once to fp16 at M > 8: the
    fp32-accumulate tier on the oracle's value rounded to fp16); then the four projections recorded
    as one session and replayed, which must reproduce the per-projection outputs bit for bit.
"""
import numpy as np
import pytest

from bybylang_amd import synth
from oracle_lib import OP_Q4_COOP_GEMM, OP_Q4_GEMV, q4_blob, shape_op_program
from parity import TIER_F32_ACC, ref_check, tier_check

pytestmark = pytest.mark.gpu

C4_OPS = [("qkv", 4096, 6144), ("o", 4096, 4096), ("gate_up", 4096, 2 * 14336), ("down", 14336, 4096)]


@pytest.fixture(scope="module")
def c0():
    g = synth.rng(0)
    M, K, N = 16, 4096, 4096
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    x = synth.activations(g, M, K, np.float32)
    return M, K, N, wq, sc, ze, x


@pytest.mark.parametrize("op", [OP_Q4_GEMV, OP_Q4_COOP_GEMM])
def test_c0_program_route_full(hip, oracle, c0, op):
    M, K, N, wq, sc, ze, x = c0
    u8, f32 = q4_blob(wq, sc, ze, K, N, K // 32)
    print(f"c0 program route op=0x{op:02x}", flush=True)
    mem = hip.DeviceBuffer(M * N * 4)
    hip.program_dispatch(shape_op_program(op, M, K, N, 32, K // 32), mem, hip.DeviceBuffer.from_array(u8),
                         hip.DeviceBuffer.from_array(f32), hip.DeviceBuffer.from_array(x.reshape(-1)))
    want = oracle.q4_shape_op(op == OP_Q4_COOP_GEMM, M, K, N, 32, K // 32, u8, f32, x.reshape(-1))
    ref_check(mem.read(np.float32), want)


def test_c0_session_matmul_full(hip, oracle, c0):
    from bybylang_amd import gpubackend as gb
    M, K, N, wq, sc, ze, x = c0
    w = gb.residentUploadQ4(gb.gbHip, wq, sc, ze, K, N, 32, K // 32)
    assert gb.sessionBegin(gb.gbHip)
    ha = gb.sessionUpload(gb.gbHip, x.reshape(-1))
    hc = gb.SessionHandle()
    assert gb.sessionMatmulQ4(gb.gbHip, ha, w, hc, M)
    assert gb.sessionEnd(gb.gbHip), gb.sessionGetLastError(gb.gbHip)
    got = gb.sessionRead(gb.gbHip, hc, M * N)
    ref_check(got, oracle.matmul_q4(x.reshape(-1), wq, sc, ze, M, K, N, 32, K // 32))
    for h in (ha, hc):
        gb.sessionFree(gb.gbHip, h)
    gb.residentFreeQ4(w)


def dequant(codes, scales, group=32):
    """Weights (q - 8) * s of the synthetic Q4 format, as float32 [N, K]."""
    N, K = codes.shape
    return (codes.astype(np.float32).reshape(N, K // group, group) *
            scales.reshape(N, K // group, 1)).reshape(N, K)


@pytest.fixture(scope="module")
def c4_weights(hip):
    g = synth.rng(4)
    out = {}
    for name, K, N in C4_OPS:
        wq, sc, ze, codes = synth.q4_weights(g, N, K)
        out[name] = (K, N, wq, sc, ze, codes, hip.Q4Weights(wq, sc, ze, K, N, 32, K // 32))
    return out


@pytest.mark.parametrize("M", [1, 32, 256])
@pytest.mark.parametrize("name", [o[0] for o in C4_OPS])
def test_c4_projection(hip, oracle, c4_weights, name, M):
    K, N, wq, sc, ze, codes, w = c4_weights[name]
    g = synth.rng(40 + M)
    x = synth.activations(g, M, K, np.float16)
    print(f"c4 {name} M={M} K={K} N={N}", flush=True)
    xd = hip.DeviceBuffer.from_array(x.reshape(-1))
    yd = hip.DeviceBuffer(M * N * 2)
    hip.q4_matmul(xd, hip.F16, w, yd, hip.F16, M)
    got = yd.read(np.float16, M * N).astype(np.float32).reshape(M, N)
    xf = x.astype(np.float32)
    # rows spread over the output against the oracle's loops
    rows = sorted({0, M // 3, (2 * M) // 3, M - 1})
    for r in rows:
        want = oracle.matmul_q4(xf.reshape(-1), wq, sc, ze, M, K, N, 32, K // 32, rows=(r, r + 1))[r]
        tier_check(got[r], want.astype(np.float16).astype(np.float32), TIER_F32_ACC)
    # every row against a float64 product
    W = dequant(codes, sc)
    want = np.empty((M, N), np.float64)
    for n0 in range(0, N, 4096):
        want[:, n0:n0 + 4096] = xf.astype(np.float64) @ W[n0:n0 + 4096].astype(np.float64).T
    tier_check(got, want.astype(np.float16).astype(np.float32), TIER_F32_ACC)


@pytest.mark.parametrize("M", [1, 32, 256])
def test_c4_layer_batch_recorded(hip, c4_weights, M):
    """The four projections recorded as one session (HIP graph) and replayed twice: each replay
    reproduces the outputs of the same calls made one by one."""
    from bybylang_amd import gpubackend as gb
    g = synth.rng(50 + M)
    xs, ys, want = [], [], []
    for name, K, N in C4_OPS:
        w = c4_weights[name][-1]
        xs.append(hip.DeviceBuffer.from_array(synth.activations(g, M, K, np.float16).reshape(-1)))
        ys.append(hip.DeviceBuffer(M * N * 2))
        hip.q4_matmul(xs[-1], hip.F16, w, ys[-1], hip.F16, M)
        want.append(ys[-1].read(np.uint16, M * N))
    for y in ys:
        y.zero()
    assert gb.sessionBeginRecording(gb.gbHip)
    for (name, K, N), x, y in zip(C4_OPS, xs, ys):
        hip.q4_matmul(x, hip.F16, c4_weights[name][-1], y, hip.F16, M)
    assert gb.sessionEnd(gb.gbHip), gb.sessionGetLastError(gb.gbHip)
    rid = gb.sessionLastRecording(gb.gbHip)
    assert rid >= 0
    for _ in range(2):
        for y, wv in zip(ys, want):
            assert np.array_equal(y.read(np.uint16, wv.size), wv)
            y.zero()
        assert gb.sessionReplay(gb.gbHip, rid, 1), gb.sessionGetLastError(gb.gbHip)
    for y, wv in zip(ys, want):
        assert np.array_equal(y.read(np.uint16, wv.size), wv)
    gb.sessionFreeRecording(gb.gbHip, rid)
