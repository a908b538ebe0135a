"""The fused decode GEMV oracle (orc_q4_fused) pinned on the CPU.

sessionMatmulQ4Fused (gpubackend.nim:3185-3231) replaces an unfused sequence that the reference's
callers run when it returns false: RMSNorm (nimf_cpu_rmsnorm, cpu_kernels_impl.inc:175-189), the Q4
matmul (nimf_cpu_matmul_q4, cpu_kernels_impl.inc:293-319), silu(gate) * up and the residual add.
The oracle follows the fused shader's arithmetic (q4_autotune.nim:194-330), which applies the norm
factor after the dot product; it is checked here against that unfused sequence computed by the
reference's own C (oracle/_ref), against a closed form, and against planted mistakes.

Tolerance: max-abs-rel <= 1e-5 (fp32 accumulation of K <= 1024 terms in a different order: the
norm factor before or after the sum, a fused or unfused multiply-add).
"""
import numpy as np
import pytest

from oracle_lib import Reference
from parity import max_abs_rel

needs_ref = pytest.mark.skipif(not Reference.available(), reason="oracle/_ref not built (reference absent)")
TOL = 1e-5


def silu(v):
    v = np.asarray(v, np.float64)
    return v / (1.0 + np.exp(-v))


def make_case(seed, K, Ns, group, asym=False):
    from bybylang_amd import synth
    g = synth.rng(seed)
    mats = []
    for N in Ns:
        wq, sc, ze, _ = synth.q4_weights(g, N, K, group)
        if asym:
            ze = (g.random(ze.size) * 15).astype(np.float32)
        mats.append((wq, sc, ze, N))
    a = g.standard_normal(K).astype(np.float32)
    gamma = (1.0 + 0.25 * g.standard_normal(K)).astype(np.float32)
    res = g.standard_normal(max(Ns)).astype(np.float32)
    return mats, a, gamma, res


def unfused(ref, mode, mats, a, K, group, gamma, eps, res):
    """The reference's unfused sequence on its own compiled C, then silu * up and the residual."""
    x = ref.rmsnorm(a, gamma, 1, K, eps) if gamma is not None else a
    outs = [ref.matmul_q4(x, wq, sc, ze, 1, K, N, group, K // group).reshape(-1).astype(np.float64)
            for wq, sc, ze, N in mats]
    if mode == 1:
        outs = [silu(outs[0]) * outs[1]]
    if res is not None:
        outs = [o + res[:o.size] for o in outs]
    return outs


@needs_ref
@pytest.mark.parametrize("mode,Ns", [(0, [40]), (0, [40, 24]), (0, [40, 24, 56]), (1, [48, 48])])
@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("with_res", [False, True])
def test_fused_oracle_matches_reference_unfused(oracle, mode, Ns, norm, with_res):
    K, group, eps = 512, 32, 1e-5
    mats, a, gamma, res = make_case(100 + 7 * len(Ns) + mode, K, Ns, group)
    gam = gamma if norm else None
    r = res if with_res else None
    got = oracle.q4_fused(mode, a, mats, K, group, K // group, residual=r, gamma=gam, eps=eps)
    want = unfused(Reference(), mode, mats, a, K, group, gam, eps, r)
    assert got is not None and len(got) == len(want)
    for o, w in zip(got, want):
        assert max_abs_rel(o, w) <= TOL


@needs_ref
@pytest.mark.parametrize("group", [64, 128])
def test_fused_oracle_groups_and_asymmetric_zeros(oracle, group):
    K, eps = 1024, 1e-6
    mats, a, gamma, res = make_case(200 + group, K, [33, 33], group, asym=True)
    for mode in (0, 1):
        got = oracle.q4_fused(mode, a, mats, K, group, K // group, residual=res, gamma=gamma, eps=eps)
        want = unfused(Reference(), mode, mats, a, K, group, gamma, eps, res)
        for o, w in zip(got, want):
            assert max_abs_rel(o, w) <= TOL


def test_fused_oracle_closed_form(oracle):
    """All codes 9 with zero 8 and scale 0.5: every weight is 0.5; a = 2, gamma = 1, eps = 0.
    No norm: 128 * 0.5 * 2 = 128. Norm: ssq / K = 4, inv = 0.5, so 64; silu(64) * 64 is 4096 to
    fp32 precision (exp(-64) is far below an ulp)."""
    K, N = 128, 8
    wq = np.full(N * K // 2, 0x99, np.uint8)
    sc = np.full(N * K // 32, 0.5, np.float32)
    ze = np.full(N * K // 32, 8.0, np.float32)
    a = np.full(K, 2.0, np.float32)
    gamma = np.ones(K, np.float32)
    mats = [(wq, sc, ze, N), (wq, sc, ze, N)]
    plain = oracle.q4_fused(0, a, mats[:1], K, 32, K // 32)
    assert np.array_equal(plain[0], np.full(N, 128.0, np.float32))
    normed = oracle.q4_fused(0, a, mats[:1], K, 32, K // 32, gamma=gamma, eps=0.0)
    assert np.array_equal(normed[0], np.full(N, 64.0, np.float32))
    gu = oracle.q4_fused(1, a, mats, K, 32, K // 32, gamma=gamma, eps=0.0)
    assert np.array_equal(gu[0], np.full(N, 4096.0, np.float32))
    res = np.arange(N, dtype=np.float32)
    gur = oracle.q4_fused(1, a, mats, K, 32, K // 32, residual=res, gamma=gamma, eps=0.0)
    assert np.array_equal(gur[0], 4096.0 + res)


def test_fused_oracle_rejects_what_the_reference_rejects(oracle):
    """gpubackend.nim:3200 (and 3219): ws.len outside 1..3, or mode 1 without exactly two."""
    mats, a, _, _ = make_case(300, 64, [8, 8, 8, 8], 32)
    assert oracle.q4_fused(0, a, mats[:4], 64, 32, 2) is None
    assert oracle.q4_fused(0, a, [], 64, 32, 2) is None
    assert oracle.q4_fused(1, a, mats[:1], 64, 32, 2) is None
    assert oracle.q4_fused(1, a, mats[:3], 64, 32, 2) is None
    assert oracle.q4_fused(2, a, mats[:2], 64, 32, 2) is None


@needs_ref
def test_fused_planted_mistakes_are_caught(oracle):
    """Plausible slips in the oracle's formula (on the CPU) fail the comparison used above: silu on
    the wrong operand, the norm factor dropped or applied twice, the residual left out."""
    K, group, eps = 512, 32, 1e-5
    mats, a, gamma, res = make_case(400, K, [64, 64], group)
    ref = Reference()
    want = unfused(ref, 1, mats, a, K, group, gamma, eps, res)[0]
    x = ref.rmsnorm(a, gamma, 1, K, eps)
    g = ref.matmul_q4(x, *mats[0][:3], 1, K, 64, group, K // group).reshape(-1).astype(np.float64)
    u = ref.matmul_q4(x, *mats[1][:3], 1, K, 64, group, K // group).reshape(-1).astype(np.float64)
    xg = (a * gamma).astype(np.float32)
    g_raw = ref.matmul_q4(xg, *mats[0][:3], 1, K, 64, group, K // group).reshape(-1).astype(np.float64)
    u_raw = ref.matmul_q4(xg, *mats[1][:3], 1, K, 64, group, K // group).reshape(-1).astype(np.float64)
    inv = 1.0 / np.sqrt(np.mean(a.astype(np.float64) ** 2) + eps)
    for wrong in (silu(u) * g + res, silu(g_raw) * u_raw + res, silu(g * inv) * (u * inv) + res,
                  silu(g) * u):
        assert max_abs_rel(wrong, want) > 100 * TOL
    got = oracle.q4_fused(1, a, mats, K, group, K // group, residual=res, gamma=gamma, eps=eps)[0]
    assert max_abs_rel(got, want) <= TOL
