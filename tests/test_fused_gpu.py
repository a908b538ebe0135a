"""The fused decode GEMV (sessionMatmulQ4Fused, gpubackend.nim:3185-3231) on the MI355X against the
oracle (orc_q4_fused, itself pinned to the reference's unfused sequence in test_fused_oracle.py).

Bar: the reference test's tolerance for fp32 paths, max|diff| <= 1e-4 * max(1, peak) (the kernel
splits the fp32 input into two fp16 terms, about 22 bits, with exact products and fp32 sums).
Unsupported combinations return BYHIP_UNSUPPORTED and leave the outputs untouched.
"""
import numpy as np
import pytest

from parity import ref_check

pytestmark = pytest.mark.gpu


def make(seed, K, Ns, group=32, f32_scales=False, asym=False):
    from bybylang_amd import synth
    g = synth.rng(seed)
    mats = []
    for N in Ns:
        wq, sc, ze, _ = synth.q4_weights(g, N, K, group)
        if f32_scales:
            sc = (g.random(sc.size) * 0.05 + 1e-3).astype(np.float32)
        if asym:
            ze = (g.random(ze.size) * 15).astype(np.float32)
        mats.append((wq, sc, ze, N))
    a = g.standard_normal(K).astype(np.float32)
    gamma = (1.0 + 0.25 * g.standard_normal(K)).astype(np.float32)
    res = g.standard_normal(max(Ns)).astype(np.float32)
    return mats, a, gamma, res


def run_fused(hip, mode, mats, a, K, group, res=None, gamma=None, eps=0.0, n_out=None):
    ws = [hip.Q4Weights(wq, sc, ze, K, N, group, K // group) for wq, sc, ze, N in mats]
    xd = hip.DeviceBuffer.from_array(a)
    n_out = n_out if n_out is not None else len(mats)  # one per weight, as the reference wants
    sentinel = np.float32(-12345.0)
    outs = [hip.DeviceBuffer.from_array(np.full(mats[i][3], sentinel, np.float32)) for i in range(n_out)]
    rd = hip.DeviceBuffer.from_array(res) if res is not None else None
    gd = hip.DeviceBuffer.from_array(gamma) if gamma is not None else None
    rc = hip.q4_matmul_fused(mode, xd, ws, outs, rd, gd, eps)
    got = [o.read(np.float32, mats[i][3]) for i, o in enumerate(outs)]
    for w in ws:
        w.close()
    return rc, got


@pytest.mark.parametrize("mode,Ns", [(0, [40]), (0, [40, 24]), (0, [37, 24, 61]), (1, [50, 50])])
@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("with_res", [False, True])
@pytest.mark.parametrize("K", [256, 4096])
def test_fused_modes(hip, oracle, mode, Ns, norm, with_res, K):
    mats, a, gamma, res = make(900 + K + 5 * len(Ns) + mode, K, Ns)
    gam = gamma if norm else None
    r = res if with_res else None
    print(f"fused mode={mode} Ns={Ns} K={K} norm={norm} res={with_res}", flush=True)
    rc, got = run_fused(hip, mode, mats, a, K, 32, r, gam, 1e-5)
    assert rc == 0
    want = oracle.q4_fused(mode, a, mats, K, 32, K // 32, residual=r, gamma=gam, eps=1e-5)
    for o, w in zip(got, want):
        ref_check(o, w)


@pytest.mark.parametrize("f32_scales,asym", [(False, True), (True, False), (True, True)])
@pytest.mark.parametrize("group,K", [(64, 512), (128, 8192), (0, 1024)])
def test_fused_scale_formats_and_groups(hip, oracle, f32_scales, asym, group, K):
    """Every kernel variant: fp16 / fp32 scales, uniform / per-group zeros; groups 64, 128 and a
    whole row; K up to 8192 (four chunks per lane)."""
    gsz = group if group else K
    mats, a, gamma, res = make(1000 + group + K + 3 * f32_scales + asym, K, [45, 45], gsz, f32_scales, asym)
    for mode in (0, 1):
        print(f"fused formats mode={mode} group={group} K={K} f32={f32_scales} asym={asym}", flush=True)
        ws = [hip.Q4Weights(wq, sc, ze, K, N, group, K // gsz) for wq, sc, ze, N in mats]
        xd = hip.DeviceBuffer.from_array(a)
        outs = [hip.DeviceBuffer(45 * 4) for _ in range(2)]
        rc = hip.q4_matmul_fused(mode, xd, ws, outs, hip.DeviceBuffer.from_array(res),
                                 hip.DeviceBuffer.from_array(gamma), 1e-6)
        assert rc == 0
        want = oracle.q4_fused(mode, a, mats, K, gsz, K // gsz, residual=res, gamma=gamma, eps=1e-6)
        for o, w in zip(outs, want):
            ref_check(o.read(np.float32, 45), w)
        for w in ws:
            w.close()


def test_fused_decode_layer_shapes(hip, oracle):
    """The decode step of the layer batch's shapes: QKV as three matrices (4096, 1024, 1024) with the
    attention norm, and gate * up (2 x 14336) with the MLP norm and a residual."""
    K = 4096
    mats, a, gamma, res = make(1100, K, [4096, 1024, 1024])
    print("fused qkv 4096/1024/1024 norm", flush=True)
    rc, got = run_fused(hip, 0, mats, a, K, 32, None, gamma, 1e-5)
    assert rc == 0
    for o, w in zip(got, oracle.q4_fused(0, a, mats, K, 32, K // 32, gamma=gamma, eps=1e-5)):
        ref_check(o, w)
    mats, a, gamma, res = make(1101, K, [14336, 14336])
    print("fused gate*up 14336 norm residual", flush=True)
    rc, got = run_fused(hip, 1, mats, a, K, 32, res, gamma, 1e-5)
    assert rc == 0
    ref_check(got[0], oracle.q4_fused(1, a, mats, K, 32, K // 32, residual=res, gamma=gamma, eps=1e-5)[0])
    K = 14336
    mats, a, gamma, res = make(1102, K, [4096])
    print("fused down 14336 -> 4096 residual", flush=True)
    rc, got = run_fused(hip, 0, mats, a, K, 32, res, None, 0.0)
    assert rc == 0
    ref_check(got[0], oracle.q4_fused(0, a, mats, K, 32, K // 32, residual=res)[0])


@pytest.mark.parametrize("K,Ns,norm", [(10240, [37, 21], True), (14336, [50], True), (12288, [8, 8, 8], False)])
def test_fused_long_rows(hip, oracle, K, Ns, norm):
    """Rows of more than four chunks per lane (two rows per wave) and inputs staged as two chunks
    per thread (K > 8192), mode 0; gate * up keeps four chunks per lane and runs such rows in K
    slices (the slices' partial dot products and sums of squares finished by a second kernel)."""
    mats, a, gamma, res = make(1400 + K, K, Ns)
    gam = gamma if norm else None
    print(f"fused long rows K={K} Ns={Ns} norm={norm}", flush=True)
    rc, got = run_fused(hip, 0, mats, a, K, 32, res, gam, 1e-5)
    assert rc == 0
    for o, w in zip(got, oracle.q4_fused(0, a, mats, K, 32, K // 32, residual=res, gamma=gam, eps=1e-5)):
        ref_check(o, w)
    if len(Ns) >= 2 and Ns[0] == Ns[1] or len(Ns) == 1:
        pair = [mats[0], mats[0]]
        rc, got = run_fused(hip, 1, pair, a, K, 32, res, gam, 1e-5)
        assert rc == 0
        ref_check(got[0], oracle.q4_fused(1, a, pair, K, 32, K // 32, residual=res, gamma=gam, eps=1e-5)[0])
        assert np.all(got[1] == np.float32(-12345.0))


@pytest.mark.parametrize("case", ["mode1_one_weight", "mode1_three_weights", "four_weights",
                                  "few_outputs", "mode1_one_output", "k_mismatch", "n_mismatch_mode1",
                                  "k_not_32", "mode2"])
def test_fused_unsupported_leaves_outputs(hip, case):
    """The combinations the reference's encoders reject (gpubackend.nim:3200-3206), and weights the
    kernel does not take, return BYHIP_UNSUPPORTED before any work: the outputs keep their contents."""
    from bybylang_amd import _abi
    K, Ns, mode, n_out = 256, [16, 16], 1, None
    if case == "mode1_one_weight":
        Ns = [16]
    elif case == "mode1_three_weights":
        Ns = [16, 16, 16]
    elif case == "four_weights":
        Ns, mode = [16, 16, 16, 16], 0
    elif case == "few_outputs":
        Ns, mode, n_out = [16, 16], 0, 1
    elif case == "mode1_one_output":
        n_out = 1
    elif case == "n_mismatch_mode1":
        Ns = [16, 24]
    elif case == "mode2":
        mode = 2
    group = 32
    if case == "k_not_32":  # the kernel reads whole 32-value chunks
        K, group = 272, 16
    mats, a, _, _ = make(1200, K, Ns, group)
    if case == "k_mismatch":
        other, _, _, _ = make(1201, 2 * K, [16])
        ws = [hip.Q4Weights(*mats[0][:3], K, 16, 32, K // 32), hip.Q4Weights(*other[0][:3], 2 * K, 16, 32, 2 * K // 32)]
        outs = [hip.DeviceBuffer.from_array(np.full(16, 7.0, np.float32)) for _ in range(2)]
        rc = hip.q4_matmul_fused(1, hip.DeviceBuffer.from_array(np.zeros(2 * K, np.float32)), ws, outs)
        assert rc == _abi.BYHIP_UNSUPPORTED
        assert np.all(outs[0].read(np.float32, 16) == 7.0)
        return
    rc, got = run_fused(hip, mode, mats, a, K, group, n_out=n_out)
    assert rc == _abi.BYHIP_UNSUPPORTED
    for o in got:
        assert np.all(o == np.float32(-12345.0))


def test_session_matmul_q4_fused(hip, oracle):
    """The session mirror (gpubackend.sessionMatmulQ4Fused) on session buffers, and its False for a
    rejected combination (mode 1 with one output for two weights, gpubackend.nim:3200)."""
    from bybylang_amd import gpubackend as gb
    K = 1024
    mats, a, gamma, res = make(1300, K, [64, 64])
    ws = [gb.residentUploadQ4(gb.gbHip, wq, sc, ze, K, N, 32, K // 32) for wq, sc, ze, N in mats]
    assert gb.sessionBegin(gb.gbHip)
    ha = gb.sessionUpload(gb.gbHip, a)
    hr = gb.sessionUpload(gb.gbHip, res)
    hg = gb.sessionUpload(gb.gbHip, gamma)
    o = gb.sessionAllocScratch(gb.gbHip, 64)
    o2 = gb.sessionAllocScratch(gb.gbHip, 64)  # the reference wants one output per weight
    ok = gb.sessionMatmulQ4Fused(gb.gbHip, 1, ha, ws, [o, o2], hr, True, hg, 1e-5, True)
    rejected = gb.sessionMatmulQ4Fused(gb.gbHip, 1, ha, ws, [o], hr, True, hg, 1e-5, True)
    assert gb.sessionEnd(gb.gbHip), gb.sessionGetLastError(gb.gbHip)
    assert ok and not rejected
    want = oracle.q4_fused(1, a, mats, K, 32, K // 32, residual=res, gamma=gamma, eps=1e-5)[0]
    ref_check(gb.sessionRead(gb.gbHip, o, 64), want)
    for h in (ha, hr, hg, o, o2):
        gb.sessionFree(gb.gbHip, h)
    for w in ws:
        gb.residentFreeQ4(w)
