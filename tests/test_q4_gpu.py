"""Q4 block-dequant GEMV / GEMM on the MI355X against the oracle (reference CPU semantics).

Bar: fp32 activations and fp32 accumulation on the decode GEMV match the reference test's own
tolerance (max|diff| <= 1e-4 * max(1, peak)); the fp16-MFMA GEMM, whose weights are rounded once to
fp16, meets the fp32-accumulate tier (max-abs-rel <= 1e-3); fp16 outputs are compared after the
oracle's values are rounded the same way. Unpacked codes and scales are bit-exact.
"""
import os
import zlib

import numpy as np
import pytest

from oracle_lib import OP_Q4_COOP_GEMM, OP_Q4_GEMV, q4_blob, shape_op_program
from parity import TIER_BF16_OUT, TIER_F32_ACC, bf16_bits_to_f32, f32_to_bf16_rne, ref_check, tier_check

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


class route:
    """Forces the library's Q4 route (BYHIP_Q4_ROUTE: 1 GEMV, 2 GEMM, 3 generic) for a block."""

    def __init__(self, r):
        self.r = r

    def __enter__(self):
        os.environ["BYHIP_Q4_ROUTE"] = str(self.r)

    def __exit__(self, *a):
        os.environ.pop("BYHIP_Q4_ROUTE", None)


def run_q4(hip, x, wq, sc, ze, M, K, N, grp, x_dtype=None, y_dtype=None, gpr=None):
    x_dtype = hip.F32 if x_dtype is None else x_dtype
    y_dtype = hip.F32 if y_dtype is None else y_dtype
    w = hip.Q4Weights(wq, sc, ze, K, N, grp, gpr if gpr else max(1, K // grp if grp else 1))
    xd = hip.DeviceBuffer.from_array(np.asarray(x, dtype=hip.np_dtype(x_dtype)).reshape(-1))
    yd = hip.DeviceBuffer(M * N * (4 if y_dtype == hip.F32 else 2))
    hip.q4_matmul(xd, x_dtype, w, yd, y_dtype, M)
    out = yd.read(hip.np_dtype(y_dtype), M * N)
    if y_dtype == hip.BF16:
        out = bf16_bits_to_f32(out)
    return out.astype(np.float32).reshape(M, N), w


def golden_q4(i):
    g = load("q4_cases.npz")
    M, K, N, grp, sym = (int(v) for v in g[f"shape_{i}"])
    return M, K, N, grp, g[f"x_{i}"], g[f"wq_{i}"], g[f"scales_{i}"], g[f"zeros_{i}"], g[f"gemv_{i}"]


@pytest.mark.parametrize("i", range(10))
@pytest.mark.parametrize("r", [0, 1, 2, 3])
def test_q4_golden_routes(hip, i, r):
    M, K, N, grp, x, wq, sc, ze, want = golden_q4(i)
    print(f"q4 golden case {i} route {r} M={M} K={K} N={N} group={grp}", flush=True)
    if r == 2 and K % 32:
        pytest.skip("GEMM route needs K % 32 == 0")
    with route(r):
        got, _ = run_q4(hip, x, wq, sc, ze, M, K, N, grp)
    if r == 3 or (r in (0, 1) and M <= 8):
        ref_check(got, want)  # fp32 routes: the reference test's tolerance
    else:
        tier_check(got, want, TIER_F32_ACC)


@pytest.mark.parametrize("i", range(10))
def test_q4_unpack_bit_exact(hip, oracle, i):
    M, K, N, grp, x, wq, sc, ze, _ = golden_q4(i)
    w = hip.Q4Weights(wq, sc, ze, K, N, grp, K // grp)
    codes, s2, z2 = w.unpack()
    assert np.array_equal(codes, oracle.unpack_q4(wq, K, N))
    assert np.array_equal(s2.view(np.uint32), sc.view(np.uint32))
    assert np.array_equal(z2.view(np.uint32), ze.view(np.uint32))
    info = w.info()
    sym = bool(load("q4_cases.npz")[f"shape_{i}"][4])
    assert info["scale_is_f16"] == int(sym) and info["zero_uniform"] == int(sym)


@pytest.mark.parametrize("op", [OP_Q4_GEMV, OP_Q4_COOP_GEMM])
@pytest.mark.parametrize("i", range(10))
def test_q4_program_route_golden(hip, i, op):
    """The micro-VM route: the shape op over the one-blob slots (cpu_vm.c:446-450)."""
    g = load("q4_cases.npz")
    M, K, N, grp, x, wq, sc, ze, _ = golden_q4(i)
    key = ("gemv_" if op == OP_Q4_GEMV else "coop_") + str(i)
    if key not in g:
        pytest.skip("shape not valid for this op")
    u8, f32 = q4_blob(wq, sc, ze, K, N, K // grp)
    mem = hip.DeviceBuffer(M * N * 4)
    hip.program_dispatch(shape_op_program(op, M, K, N, grp, K // grp), mem,
                         hip.DeviceBuffer.from_array(u8), hip.DeviceBuffer.from_array(f32),
                         hip.DeviceBuffer.from_array(x))
    got = mem.read(np.float32)
    if M <= 8:
        ref_check(got, g[key])
    else:
        tier_check(got, g[key], TIER_F32_ACC)


@pytest.mark.parametrize("x_dtype", ["f32", "f16"])
@pytest.mark.parametrize("y_dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 9, 64, 130])
def test_q4_dtypes_and_rows(hip, oracle, M, x_dtype, y_dtype):
    from bybylang_amd import synth
    g = synth.rng(1000 + M)
    K, N = 512, 200
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    x = synth.activations(g, M, K, np.float32)
    xt = {"f32": hip.F32, "f16": hip.F16}[x_dtype]
    yt = {"f32": hip.F32, "f16": hip.F16, "bf16": hip.BF16}[y_dtype]
    xin = x if x_dtype == "f32" else x.astype(np.float16)
    print(f"q4 M={M} x={x_dtype} y={y_dtype}", flush=True)
    got, _ = run_q4(hip, xin, wq, sc, ze, M, K, N, 32, xt, yt)
    want = oracle.matmul_q4(np.asarray(xin, np.float32).reshape(-1), wq, sc, ze, M, K, N, 32, K // 32)
    if y_dtype == "f16":
        want_r = want.astype(np.float16).astype(np.float32)
        tier_check(got, want_r, TIER_F32_ACC)
    elif y_dtype == "bf16":
        tier_check(got, f32_to_bf16_rne(want).reshape(M, N), TIER_BF16_OUT)
    elif M <= 8:
        ref_check(got, want)
    else:
        tier_check(got, want, TIER_F32_ACC)


@pytest.mark.parametrize("tile", [1, 2, 3, 4])
@pytest.mark.parametrize("shape", [(64, 512, 256), (130, 256, 200), (24, 640, 136), (33, 128, 64)])
def test_q4_gemm_tiles(hip, oracle, monkeypatch, tile, shape):
    """Every tile shape of the pipelined (LDS-staged) Q4 GEMM (64x128, 64x64, 32x128, 32x64, forced
    through BYHIP_Q4_TILE), on ragged M and N and short K, fp16 in and out, against the oracle."""
    from bybylang_amd import synth
    M, K, N = shape
    monkeypatch.setenv("BYHIP_Q4_TILE", str(tile))
    monkeypatch.setenv("BYHIP_Q4_ROUTE", "2")
    monkeypatch.setenv("BYHIP_Q4_SKINNY_MAX_M", "0")  # the LDS-staged kernel for every M
    monkeypatch.setenv("BYHIP_Q4_PREFILL", "1")
    g = synth.rng(7000 + 17 * M + N)
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    x = synth.activations(g, M, K, np.float16)
    print(f"q4 pipe tile={tile} M={M} K={K} N={N}", flush=True)
    got, _ = run_q4(hip, x, wq, sc, ze, M, K, N, 32, hip.F16, hip.F16)
    want = oracle.matmul_q4(x.astype(np.float32).reshape(-1), wq, sc, ze, M, K, N, 32, K // 32)
    tier_check(got, want.astype(np.float16).astype(np.float32), TIER_F32_ACC)


@pytest.mark.parametrize("splits", [2, 3, 5])
@pytest.mark.parametrize("shape", [(64, 512, 256), (33, 640, 136), (130, 1024, 200)])
@pytest.mark.parametrize("y_dtype", ["F32", "F16", "BF16"])
def test_q4_gemm_split_k(hip, oracle, monkeypatch, splits, shape, y_dtype):
    """Split-K (forced through BYHIP_Q4_SPLIT): partial sums over K slices added in slice order
    by a second kernel, every output dtype, ragged shapes, against the oracle; a repeat call is
    bit-identical (the sum order does not depend on block timing)."""
    from bybylang_amd import synth
    M, K, N = shape
    monkeypatch.setenv("BYHIP_Q4_SPLIT", str(splits))
    monkeypatch.setenv("BYHIP_Q4_ROUTE", "2")
    monkeypatch.setenv("BYHIP_Q4_SKINNY_MAX_M", "0")  # the LDS-staged kernel for every M
    monkeypatch.setenv("BYHIP_Q4_PREFILL", "1")
    g = synth.rng(7100 + 13 * M + N + splits)
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    x = synth.activations(g, M, K, np.float16)
    yt = getattr(hip, y_dtype)
    print(f"q4 split-k splits={splits} M={M} K={K} N={N} y={y_dtype}", flush=True)
    got, _ = run_q4(hip, x, wq, sc, ze, M, K, N, 32, hip.F16, yt)
    again, _ = run_q4(hip, x, wq, sc, ze, M, K, N, 32, hip.F16, yt)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    want = oracle.matmul_q4(x.astype(np.float32).reshape(-1), wq, sc, ze, M, K, N, 32, K // 32)
    if y_dtype == "F16":
        want = want.astype(np.float16).astype(np.float32)
    elif y_dtype == "BF16":
        want = f32_to_bf16_rne(want)
    tier_check(got, want.reshape(M, N), TIER_F32_ACC if y_dtype != "BF16" else TIER_BF16_OUT)


@pytest.mark.parametrize("M", [9, 16, 17, 32, 40, 64])
@pytest.mark.parametrize("splits", [0, 3])
@pytest.mark.parametrize("group", [32, 128, 0])
def test_q4_gemm_skinny(hip, oracle, monkeypatch, M, splits, group):
    """The skinny small-M kernel (weights straight to MFMA registers, K split over the block's
    waves): 16- and 32-row blocks, ragged M and N, groups 32 / 128 / whole row, with and without
    split-K, fp16 in and out, against the oracle; M above 32 takes the prefill route."""
    from bybylang_amd import synth
    K, N = 768, 200
    monkeypatch.setenv("BYHIP_Q4_ROUTE", "2")
    monkeypatch.setenv("BYHIP_Q4_STREAM", "0")
    if splits:
        monkeypatch.setenv("BYHIP_Q4_SPLIT", str(splits))
    g = synth.rng(7300 + 7 * M + group + splits)
    wq, sc, ze, _ = synth.q4_weights(g, N, K, group if group else K)
    gpr = K // group if group else 1
    x = synth.activations(g, M, K, np.float16)
    print(f"q4 skinny M={M} splits={splits} group={group}", flush=True)
    got, _ = run_q4(hip, x, wq, sc, ze, M, K, N, group, hip.F16, hip.F16, gpr=gpr)
    want = oracle.matmul_q4(x.astype(np.float32).reshape(-1), wq, sc, ze, M, K, N, group, gpr)
    tier_check(got, want.astype(np.float16).astype(np.float32), TIER_F32_ACC)


@pytest.mark.parametrize("kind", ["big", "wide"])
@pytest.mark.parametrize("shape", [(130, 768, 520), (40, 512, 136), (256, 1024, 264), (64, 384, 128)])
@pytest.mark.parametrize("splits", [0, 3])
@pytest.mark.parametrize("group", [32, 128, 0])
def test_q4_gemm_prefill_tiles(hip, oracle, monkeypatch, kind, shape, splits, group):
    """The prefill kernels (forced through BYHIP_Q4_PREFILL): the 128 x 256 tile (activations
    shared through LDS, weights straight to MFMA registers) and the 64 x 128 wide tile (K split
    over four groups of two waves, 16-byte output stores); ragged M and N, groups 32 / 128 / whole
    row, with and without split-K, fp16 in and out, against the oracle; a repeat call is
    bit-identical."""
    from bybylang_amd import synth
    M, K, N = shape
    monkeypatch.setenv("BYHIP_Q4_ROUTE", "2")
    monkeypatch.setenv("BYHIP_Q4_SKINNY_MAX_M", "0")
    monkeypatch.setenv("BYHIP_Q4_PREFILL", "2" if kind == "big" else "3")
    if splits:
        monkeypatch.setenv("BYHIP_Q4_SPLIT", str(splits))
    g = synth.rng(7500 + 11 * M + N + group + splits)
    wq, sc, ze, _ = synth.q4_weights(g, N, K, group if group else K)
    gpr = K // group if group else 1
    x = synth.activations(g, M, K, np.float16)
    print(f"q4 prefill {kind} M={M} K={K} N={N} splits={splits} group={group}", flush=True)
    got, _ = run_q4(hip, x, wq, sc, ze, M, K, N, group, hip.F16, hip.F16, gpr=gpr)
    again, _ = run_q4(hip, x, wq, sc, ze, M, K, N, group, hip.F16, hip.F16, gpr=gpr)
    assert np.array_equal(got, again)
    want = oracle.matmul_q4(x.astype(np.float32).reshape(-1), wq, sc, ze, M, K, N, group, gpr)
    tier_check(got, want.astype(np.float16).astype(np.float32), TIER_F32_ACC)


@pytest.mark.parametrize("M", [1, 5, 9, 16, 17, 31, 32])
@pytest.mark.parametrize("splits", [0, 3, 5])
@pytest.mark.parametrize("group", [32, 0])
def test_q4_gemm_wide_small_m(hip, oracle, monkeypatch, M, splits, group):
    """The wide tile with 16 and 32 rows (forced for small M): ragged M, K and N, K split so that
    the groups' sub-step counts differ and the last sub-steps lie past the end (K = 1344: 21
    sub-steps of 64), fp16 in and out, against the oracle; a repeat call is bit-identical."""
    from bybylang_amd import synth
    K, N = 1344, 264
    monkeypatch.setenv("BYHIP_Q4_ROUTE", "2")
    monkeypatch.setenv("BYHIP_Q4_SKINNY_MAX_M", "0")
    monkeypatch.setenv("BYHIP_Q4_PREFILL", "3")
    if splits:
        monkeypatch.setenv("BYHIP_Q4_SPLIT", str(splits))
    g = synth.rng(7700 + 13 * M + group + splits)
    wq, sc, ze, _ = synth.q4_weights(g, N, K, group if group else K)
    gpr = K // group if group else 1
    x = synth.activations(g, M, K, np.float16)
    print(f"q4 wide small M={M} splits={splits} group={group}", flush=True)
    got, _ = run_q4(hip, x, wq, sc, ze, M, K, N, group, hip.F16, hip.F16, gpr=gpr)
    again, _ = run_q4(hip, x, wq, sc, ze, M, K, N, group, hip.F16, hip.F16, gpr=gpr)
    assert np.array_equal(got, again)
    want = oracle.matmul_q4(x.astype(np.float32).reshape(-1), wq, sc, ze, M, K, N, group, gpr)
    tier_check(got, want.astype(np.float16).astype(np.float32), TIER_F32_ACC)


@pytest.mark.parametrize("M", [1, 5, 9, 16, 17, 24, 32])
@pytest.mark.parametrize("N", [264, 4096 + 40])
@pytest.mark.parametrize("splits", [0, 3])
@pytest.mark.parametrize("group", [32, 0])
def test_q4_gemm_stream(hip, oracle, monkeypatch, M, N, splits, group):
    """The small-M streaming GEMM (forced: BYHIP_Q4_STREAM=1): ragged M and N (N = 4136 takes two
    column fragments per block, the last block partly past N), K = 1344 (21 sub-steps of 64, so the
    eight waves run 2 or 3 each), with and without a K split, fp16 in and out, against the oracle;
    a repeat call is bit-identical."""
    from bybylang_amd import synth
    K = 1344
    monkeypatch.setenv("BYHIP_Q4_ROUTE", "2")
    monkeypatch.setenv("BYHIP_Q4_STREAM", "1")
    if splits:
        monkeypatch.setenv("BYHIP_Q4_SPLIT", str(splits))
    g = synth.rng(7900 + 13 * M + group + splits + N)
    wq, sc, ze, _ = synth.q4_weights(g, N, K, group if group else K)
    gpr = K // group if group else 1
    x = synth.activations(g, M, K, np.float16)
    print(f"q4 stream M={M} N={N} splits={splits} group={group}", flush=True)
    got, _ = run_q4(hip, x, wq, sc, ze, M, K, N, group, hip.F16, hip.F16, gpr=gpr)
    again, _ = run_q4(hip, x, wq, sc, ze, M, K, N, group, hip.F16, hip.F16, gpr=gpr)
    assert np.array_equal(got, again)
    want = oracle.matmul_q4(x.astype(np.float32).reshape(-1), wq, sc, ze, M, K, N, group, gpr)
    tier_check(got, want.astype(np.float16).astype(np.float32), TIER_F32_ACC)


@pytest.mark.parametrize("M", [17, 32])
@pytest.mark.parametrize("N", [264, 4096 + 40])
@pytest.mark.parametrize("splits", [0, 3])
def test_q4_gemm_stream_one_row_block(hip, oracle, monkeypatch, M, N, splits):
    """Above 16 rows the streaming GEMM runs each strip as two 16-row blocks; BYHIP_Q4_STREAM_HALVES=0
    keeps one 32-row block per strip. That geometry against the oracle, as above."""
    from bybylang_amd import synth
    K = 1344
    monkeypatch.setenv("BYHIP_Q4_ROUTE", "2")
    monkeypatch.setenv("BYHIP_Q4_STREAM", "1")
    monkeypatch.setenv("BYHIP_Q4_STREAM_HALVES", "0")
    if splits:
        monkeypatch.setenv("BYHIP_Q4_SPLIT", str(splits))
    g = synth.rng(7930 + M + splits + N)
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    x = synth.activations(g, M, K, np.float16)
    print(f"q4 stream one row block M={M} N={N} splits={splits}", flush=True)
    got, _ = run_q4(hip, x, wq, sc, ze, M, K, N, 32, hip.F16, hip.F16)
    want = oracle.matmul_q4(x.astype(np.float32).reshape(-1), wq, sc, ze, M, K, N, 32, K // 32)
    tier_check(got, want.astype(np.float16).astype(np.float32), TIER_F32_ACC)


@pytest.mark.parametrize("y_dtype", ["F32", "BF16"])
@pytest.mark.parametrize("M,K,N", [(32, 4096, 28672), (24, 14336, 4096), (32, 4096, 6144)])
def test_q4_gemm_stream_layer_shapes(hip, oracle, monkeypatch, y_dtype, M, K, N):
    """The streaming GEMM (forced) at the layer batch's shapes (7, 1 and 2 column fragments per
    block; the down projection's K = 14336 as 224 sub-steps, 28 per wave), fp32 and bf16 outputs:
    4 rows against the oracle, every row against an fp64 product of the fp16-rounded weights."""
    from bybylang_amd import synth
    monkeypatch.setenv("BYHIP_Q4_STREAM", "1")
    g = synth.rng(7950 + M + K // 1024 + N // 1024)
    wq, sc, ze, codes = synth.q4_weights(g, N, K)
    x = synth.activations(g, M, K, np.float16)
    print(f"q4 stream layer M={M} K={K} N={N} y={y_dtype}", flush=True)
    got, _ = run_q4(hip, x, wq, sc, ze, M, K, N, 32, hip.F16, getattr(hip, y_dtype))
    xf = x.astype(np.float32).reshape(-1)
    want = oracle.matmul_q4(xf, wq, sc, ze, M, K, N, 32, K // 32, rows=(M - 4, M))[M - 4:M]
    w = (codes.astype(np.float32) * np.repeat(sc.reshape(N, -1), 32, axis=1)).astype(np.float64)
    full = x.astype(np.float64) @ w.T
    if y_dtype == "BF16":
        tier_check(got[M - 4:M], f32_to_bf16_rne(want).reshape(4, N), TIER_BF16_OUT)
        tier_check(got, full, TIER_BF16_OUT)
    else:
        tier_check(got[M - 4:M], want, TIER_F32_ACC)
        tier_check(got, full, TIER_F32_ACC)


@pytest.mark.parametrize("kind", ["big", "wide"])
@pytest.mark.parametrize("y_dtype", ["F32", "BF16"])
def test_q4_gemm_prefill_out_dtypes(hip, oracle, monkeypatch, kind, y_dtype):
    """fp32 and bf16 outputs of the prefill kernels (the fp32 path also through split-K)."""
    from bybylang_amd import synth
    M, K, N = 200, 1024, 300
    monkeypatch.setenv("BYHIP_Q4_ROUTE", "2")
    monkeypatch.setenv("BYHIP_Q4_PREFILL", "2" if kind == "big" else "3")
    if y_dtype == "F32":
        monkeypatch.setenv("BYHIP_Q4_SPLIT", "2")
    g = synth.rng(7600 + len(kind) + len(y_dtype))
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    x = synth.activations(g, M, K, np.float16)
    print(f"q4 prefill {kind} y={y_dtype}", flush=True)
    got, _ = run_q4(hip, x, wq, sc, ze, M, K, N, 32, hip.F16, getattr(hip, y_dtype))
    want = oracle.matmul_q4(x.astype(np.float32).reshape(-1), wq, sc, ze, M, K, N, 32, K // 32)
    if y_dtype == "BF16":
        tier_check(got, f32_to_bf16_rne(want).reshape(M, N), TIER_BF16_OUT)
    else:
        tier_check(got, want, TIER_F32_ACC)


@pytest.mark.parametrize("M", [32, 256])
def test_q4_layer_down_auto_split(hip, oracle, M):
    """The layer batch's down projection (K=14336, N=4096) at M=32 and 256, where the tiles alone
    leave most CUs idle and the launcher splits K; rows against the oracle, every row against an
    fp64 product of the fp16-rounded weights."""
    from bybylang_amd import synth
    g = synth.rng(40 + M)
    K, N = 14336, 4096
    wq, sc, ze, codes = synth.q4_weights(g, N, K)
    x = synth.activations(g, M, K, np.float16)
    print(f"q4 down auto split M={M}", flush=True)
    got, _ = run_q4(hip, x, wq, sc, ze, M, K, N, 32, hip.F16, hip.F16)
    xf = x.astype(np.float32).reshape(-1)
    want = oracle.matmul_q4(xf, wq, sc, ze, M, K, N, 32, K // 32, rows=(M - 4, M))[M - 4:M]
    tier_check(got[M - 4:M], want.astype(np.float16).astype(np.float32), TIER_F32_ACC)
    w = (codes.astype(np.float32) * np.repeat(sc.reshape(N, -1), 32, axis=1)).astype(np.float64)
    tier_check(got, x.astype(np.float64) @ w.T, TIER_F32_ACC)


@pytest.mark.parametrize("case", ["group0", "group64", "group128", "asym_zero", "int_zero5",
                                  "f32_scales", "odd_k", "gpr_pad", "k32"])
@pytest.mark.parametrize("M", [1, 3, 24])
def test_q4_edge_shapes(hip, oracle, case, M):
    # a seed that does not depend on the process (str hashes are salted per process)
    r = np.random.default_rng(zlib.crc32(case.encode()) % 1000 + M)
    K, N, grp = 256, 72, 32
    if case == "group0":
        grp = 0
    elif case == "group64":
        grp = 64
    elif case == "group128":
        grp = 128
    elif case == "odd_k":
        K = 250
        grp = 50
    elif case == "k32":
        K = 32
    gpr = 1 if grp == 0 else (K + grp - 1) // grp
    if case == "gpr_pad":
        gpr += 3
    q = r.integers(0, 16, size=(N, K)).astype(np.uint8)
    if K % 2:
        q = np.concatenate([q, np.zeros((N, 1), np.uint8)], axis=1)
    wq = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8).reshape(-1)
    sc = (np.abs(r.normal(0, 0.02, N * gpr)) + 1e-4).astype(np.float16).astype(np.float32)
    ze = np.full(N * gpr, 8.0, np.float32)
    if case == "asym_zero":
        ze = (r.random(N * gpr) * 15).astype(np.float32)
    if case == "int_zero5":
        ze[:] = 5.0
    if case == "f32_scales":
        sc = (r.random(N * gpr) * 0.05 + 1e-3).astype(np.float32)
    x = r.standard_normal(M * K).astype(np.float32)
    print(f"q4 edge {case} M={M} K={K} group={grp} gpr={gpr}", flush=True)
    got, _ = run_q4(hip, x, wq, sc, ze, M, K, N, grp, gpr=gpr)
    want = oracle.matmul_q4(x, wq, sc, ze, M, K, N, grp, gpr)
    if M <= 8:
        ref_check(got, want)
    else:
        tier_check(got, want, TIER_F32_ACC)


def test_q4_decode_config_full(hip, oracle):
    """Config 1 at full size: M=1, K=4096, N=14336, fp16 x, fp16 y, against the oracle."""
    from bybylang_amd import synth
    g = synth.rng(0)
    M, K, N = 1, 4096, 14336
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    x = synth.activations(g, M, K, np.float16)
    got, _ = run_q4(hip, x, wq, sc, ze, M, K, N, 32, hip.F16, hip.F16)
    want = oracle.matmul_q4(x.astype(np.float32).reshape(-1), wq, sc, ze, M, K, N, 32, K // 32)
    r = tier_check(got, want.astype(np.float16).astype(np.float32), 1e-3)
    print(f"c1 max-abs-rel vs fp16-rounded oracle {r:.2e}")


def test_q4_prefill_config_rows(hip, oracle):
    """Config 2 (M=512, K=N=4096, fp16 in/out) on the GPU; rows 0-7 and the last 8 against the
    oracle, and every row against an fp64 product of the fp16-rounded weights."""
    from bybylang_amd import synth
    g = synth.rng(2)
    M, K, N = 512, 4096, 4096
    wq, sc, ze, codes = synth.q4_weights(g, N, K)
    x = synth.activations(g, M, K, np.float16)
    got, _ = run_q4(hip, x, wq, sc, ze, M, K, N, 32, hip.F16, hip.F16)
    xf = x.astype(np.float32).reshape(-1)
    for r0 in (0, M - 8):
        want = oracle.matmul_q4(xf, wq, sc, ze, M, K, N, 32, K // 32, rows=(r0, r0 + 8))[r0:r0 + 8]
        tier_check(got[r0:r0 + 8], want.astype(np.float16).astype(np.float32), TIER_F32_ACC)
    w = (codes.astype(np.float32) * np.repeat(sc.reshape(N, -1), 32, axis=1)).astype(np.float64)
    full = x.astype(np.float64) @ w.T
    tier_check(got, full, TIER_F32_ACC)


def test_q4_gemv_rotating_copies_consistent(hip):
    """Independent weight copies (the benchmark's rotation) give identical outputs."""
    from bybylang_amd import synth
    g = synth.rng(5)
    K, N = 4096, 1024
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    x = synth.activations(g, 1, K, np.float16)
    a, _ = run_q4(hip, x, wq, sc, ze, 1, K, N, 32, hip.F16, hip.F32)
    b, _ = run_q4(hip, x, wq, sc, ze, 1, K, N, 32, hip.F16, hip.F32)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_gpu_matmul_q4_immediate(hip, oracle):
    """gpuMatmulQ4 (host in/out, weights uploaded per call) through the session mirror."""
    from bybylang_amd import gpubackend as gb
    M, K, N, grp, x, wq, sc, ze, want = golden_q4(5)
    got = gb.gpuMatmulQ4(gb.gbHip, x, wq, sc, ze, M, K, N, grp, K // grp)
    ref_check(got, oracle.matmul_q4(x, wq, sc, ze, M, K, N, grp, K // grp))


def test_resident_upload_mapped(hip, tmp_path):
    """residentUploadQ4Mapped (gpubackend.nim:2961-2998): packed weights inside a mapped checkpoint
    at an odd offset are copied straight from the mapping; the result matches an upload from an
    array bit for bit, stays valid after unmapping, and reports no zero-copy (discrete HBM)."""
    from bybylang_amd import gpubackend as gb
    from bybylang_amd import synth
    g = synth.rng(77)
    K, N, M = 512, 96, 3
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    f = tmp_path / "model.bin"
    head = b"BYBYCKPT" + bytes(29)  # weights start at byte 37
    f.write_bytes(head + wq.tobytes() + b"tail")
    m = gb.openReadOnlyMapping(str(f))
    wm, zero_copy = gb.residentUploadQ4Mapped(gb.gbHip, m.data + len(head), wq.nbytes, sc, ze, K, N, 32, K // 32)
    gb.unmapReadOnlyFile(m)
    assert zero_copy is False
    wa = gb.residentUploadQ4(gb.gbHip, wq, sc, ze, K, N, 32, K // 32)
    x = synth.activations(g, M, K, np.float32)
    assert gb.sessionBegin(gb.gbHip)
    hx = gb.sessionUpload(gb.gbHip, x.reshape(-1))
    cm, ca = gb.SessionHandle(), gb.SessionHandle()
    assert gb.sessionMatmulQ4(gb.gbHip, hx, wm, cm, M)
    assert gb.sessionMatmulQ4(gb.gbHip, hx, wa, ca, M)
    assert gb.sessionEnd(gb.gbHip), gb.sessionGetLastError(gb.gbHip)
    a = gb.sessionRead(gb.gbHip, cm, M * N)
    b = gb.sessionRead(gb.gbHip, ca, M * N)
    assert np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))
    for h in (hx, cm, ca):
        gb.sessionFree(gb.gbHip, h)
    gb.residentFreeQ4(wm)
    gb.residentFreeQ4(wa)
