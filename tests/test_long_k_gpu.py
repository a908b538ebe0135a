"""Decode GEMV and fused decode GEMV at long rows (K past one launch's register tile), on the MI355X
against the oracle.

The reference's decode shader streams any K (backends/vulkan/kernels/matmul_q4_sg.glsl:59,68), its
micro-VM Q4 GEMV takes any K that is a multiple of 8 (micro_kernel/session_vm.nim:426-429) and its
fused encoder any K that is a multiple of 8 (backends/vulkan/q4_autotune.nim:338-346). Here rows
longer than the GEMV's register tile (16,384 values with fp16 activations, 15,392 with fp32) run as
K slices whose fp32 partial sums are added in slice order: a 70B-class down projection (K =
28,672) and a longer row (53,248), at M = 1 and 4, fp16 and fp32 activations, resident weights
(blocked scales) and the micro-VM's slot weights (plain fp32 scales and zeros); the fused GEMV in
both modes with the norm and the residual past its single-pass limits (mode 0 above 474 chunks,
mode 1 above 256).

Bar: the reference test's tolerance for fp32 paths, max|diff| <= 1e-4 * max(1, peak) (fp32 outputs;
fp16 outputs after the oracle's values are rounded the same way, at the fp32-accumulate tier).
"""
import os

import numpy as np
import pytest

from oracle_lib import OP_Q4_GEMV, q4_blob, shape_op_program
from parity import TIER_F32_ACC, ref_check, tier_check

pytestmark = pytest.mark.gpu


class forced_route:
    """BYHIP_Q4_ROUTE=1 keeps a call on the GEMV (M > 1 fp16 rows would take the wide tile)."""

    def __enter__(self):
        os.environ["BYHIP_Q4_ROUTE"] = "1"

    def __exit__(self, *a):
        os.environ.pop("BYHIP_Q4_ROUTE", None)


def q4_case(seed, M, K, N, group=32, asym=False):
    from bybylang_amd import synth
    g = synth.rng(seed)
    wq, sc, ze, _ = synth.q4_weights(g, N, K, group)
    if asym:
        ze = (g.random(ze.size) * 15).astype(np.float32)
    x = synth.activations(g, M, K, np.float32)
    return wq, sc, ze, x


@pytest.mark.parametrize("K", [28672, 53248])
@pytest.mark.parametrize("M", [1, 4])
@pytest.mark.parametrize("x_dtype", ["f32", "f16"])
@pytest.mark.parametrize("gemv", [False, True], ids=["default", "gemv"])
def test_long_k_decode(hip, oracle, K, M, x_dtype, gemv):
    N = 72
    wq, sc, ze, x = q4_case(7000 + K // 1024 + M + 3 * (x_dtype == "f16"), M, K, N)
    xt = hip.F32 if x_dtype == "f32" else hip.F16
    xin = x if x_dtype == "f32" else x.astype(np.float16)
    w = hip.Q4Weights(wq, sc, ze, K, N, 32, K // 32)
    xd = hip.DeviceBuffer.from_array(np.ascontiguousarray(xin).reshape(-1))
    yd = hip.DeviceBuffer(M * N * 4)
    print(f"long-K decode K={K} M={M} x={x_dtype} gemv={gemv}", flush=True)
    if gemv:
        with forced_route():
            hip.q4_matmul(xd, xt, w, yd, hip.F32, M)
    else:
        hip.q4_matmul(xd, xt, w, yd, hip.F32, M)
    got = yd.read(np.float32, M * N)
    want = oracle.matmul_q4(np.asarray(xin, np.float32).reshape(-1), wq, sc, ze, M, K, N, 32, K // 32)
    ref_check(got, want)
    # a second call leaves the same outputs (the partial sums are rewritten, not accumulated)
    if gemv:
        with forced_route():
            hip.q4_matmul(xd, xt, w, yd, hip.F32, M)
    else:
        hip.q4_matmul(xd, xt, w, yd, hip.F32, M)
    assert np.array_equal(yd.read(np.float32, M * N), got)
    w.close()


@pytest.mark.parametrize("group,asym", [(128, False), (0, True), (64, True)])
def test_long_k_groups_and_fp16_out(hip, oracle, group, asym):
    """Other groups (a whole row, 64, 128), per-group zeros, and fp16 output after the slice sum."""
    M, K, N = 2, 28672, 40
    gsz = group if group else K
    wq, sc, ze, x = q4_case(7100 + group, M, K, N, gsz, asym)
    w = hip.Q4Weights(wq, sc, ze, K, N, group, K // gsz)
    xd = hip.DeviceBuffer.from_array(x.reshape(-1))
    want = oracle.matmul_q4(x.reshape(-1), wq, sc, ze, M, K, N, gsz, K // gsz)
    print(f"long-K group={group} asym={asym}", flush=True)
    with forced_route():
        yd = hip.DeviceBuffer(M * N * 4)
        hip.q4_matmul(xd, hip.F32, w, yd, hip.F32, M)
        ref_check(yd.read(np.float32, M * N), want)
        yh = hip.DeviceBuffer(M * N * 2)
        hip.q4_matmul(xd, hip.F32, w, yh, hip.F16, M)
        tier_check(yh.read(np.float16, M * N).astype(np.float32), want.astype(np.float16).astype(np.float32),
                   TIER_F32_ACC)
    w.close()


@pytest.mark.parametrize("M", [1, 3])
def test_long_k_program_route(hip, oracle, M):
    """The micro-VM's OP_Q4_GEMV over the one-blob slots (plain fp32 scales and zeros, cpu_vm.c:446-450)
    at K = 28,672: the sliced GEMV on slot weights, against the oracle's shape op."""
    K, N, grp = 28672, 48, 32
    wq, sc, ze, x = q4_case(7200 + M, M, K, N, grp, asym=True)
    u8, f32 = q4_blob(wq, sc, ze, K, N, K // grp)
    mem = hip.DeviceBuffer(M * N * 4)
    print(f"long-K program M={M}", flush=True)
    hip.program_dispatch(shape_op_program(OP_Q4_GEMV, M, K, N, grp, K // grp), mem,
                         hip.DeviceBuffer.from_array(u8), hip.DeviceBuffer.from_array(f32),
                         hip.DeviceBuffer.from_array(x.reshape(-1)))
    want = oracle.q4_shape_op(False, M, K, N, grp, K // grp, u8, f32, x.reshape(-1))
    ref_check(mem.read(np.float32), want)


def fused_case(seed, K, Ns):
    from bybylang_amd import synth
    g = synth.rng(seed)
    mats = []
    for N in Ns:
        wq, sc, ze, _ = synth.q4_weights(g, N, K)
        mats.append((wq, sc, ze, N))
    a = g.standard_normal(K).astype(np.float32)
    gamma = (1.0 + 0.25 * g.standard_normal(K)).astype(np.float32)
    res = g.standard_normal(max(Ns)).astype(np.float32)
    return mats, a, gamma, res


@pytest.mark.parametrize("mode,Ns", [(0, [40]), (0, [37, 24, 61]), (1, [50, 50])])
@pytest.mark.parametrize("K", [8224, 15200, 28672])
@pytest.mark.parametrize("norm_res", [False, True])
def test_long_k_fused(hip, oracle, mode, Ns, K, norm_res):
    """The fused GEMV past its single-pass rows (mode 1 from 257 chunks, mode 0 from 475): K slices,
    then the finishing kernel (norm factor from the slices' sums of squares, silu(gate) * up, the
    residual)."""
    mats, a, gamma, res = fused_case(7300 + K // 32 + 7 * mode + len(Ns), K, Ns)
    ws = [hip.Q4Weights(wq, sc, ze, K, N, 32, K // 32) for wq, sc, ze, N in mats]
    xd = hip.DeviceBuffer.from_array(a)
    sentinel = np.float32(-12345.0)
    outs = [hip.DeviceBuffer.from_array(np.full(N, sentinel, np.float32)) for *_, N in mats]
    rd = hip.DeviceBuffer.from_array(res) if norm_res else None
    gd = hip.DeviceBuffer.from_array(gamma) if norm_res else None
    print(f"long-K fused mode={mode} Ns={Ns} K={K} norm_res={norm_res}", flush=True)
    assert hip.q4_matmul_fused(mode, xd, ws, outs, rd, gd, 1e-5) == 0
    want = oracle.q4_fused(mode, a, mats, K, 32, K // 32, residual=res if norm_res else None,
                           gamma=gamma if norm_res else None, eps=1e-5)
    n_out = 1 if mode == 1 else len(mats)
    for i in range(n_out):
        ref_check(outs[i].read(np.float32, mats[i][3]), want[i])
    if mode == 1:  # only the first output is written in mode 1 (gpubackend.nim:3204-3206)
        assert np.all(outs[1].read(np.float32, mats[1][3]) == sentinel)
    for w in ws:
        w.close()
