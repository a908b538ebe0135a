"""Per-shape Q4 kernel plans (byhip_q4_prepare: residentPrepareQ4, gpubackend.nim:2871-2880;
vulkanPrepareQ4Tuned, q4_autotune.nim:387-543) on the MI355X.

Every candidate passes a parity gate against the exact per-element kernel before it can be chosen;
here the calls that follow a plan are checked against the oracle with the same bars as the
untuned routes (the reference test's tolerance for the fp32 decode GEMV, the fp32-accumulate tier
for the fp16 MFMA GEMMs). The plan file is written to a temporary directory.
"""
import os

import numpy as np
import pytest

from parity import TIER_F32_ACC, ref_check, tier_check

pytestmark = pytest.mark.gpu


@pytest.fixture
def plans(hip, tmp_path, monkeypatch):
    """A private plan-file directory and no plans in memory, before and after the test."""
    monkeypatch.setenv("BYHIP_CACHE_DIR", str(tmp_path))
    monkeypatch.delenv("BYHIP_Q4_TUNED", raising=False)
    monkeypatch.delenv("BYHIP_GPU_AUTOTUNE", raising=False)
    hip.q4_plans_reset()
    yield tmp_path
    hip.q4_plans_reset()


def weights(hip, seed, K, N):
    from bybylang_amd import synth
    g = synth.rng(seed)
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    return g, (wq, sc, ze), hip.Q4Weights(wq, sc, ze, K, N, 32, K // 32)


def matmul(hip, w, x, x_dtype, M, N):
    xd = hip.DeviceBuffer.from_array(np.asarray(x).reshape(-1))
    yd = hip.DeviceBuffer(M * N * 4)
    hip.q4_matmul(xd, x_dtype, w, yd, hip.F32, M)
    return yd.read(np.float32, M * N).reshape(M, N)


def test_prepare_decode_and_prefill(hip, oracle, plans):
    from bybylang_amd import synth
    K, N = 1024, 520
    g, (wq, sc, ze), w = weights(hip, 500, K, N)
    # decode, fp32 activations (the reference's session dtype)
    print("prepare decode f32", flush=True)
    assert hip.q4_prepare(w, 1, hip.F32) == 0
    name, cached = hip.q4_plan_info(w, 1, hip.F32)
    assert name in ("generic", "gemv") and not cached
    x = synth.activations(g, 1, K, np.float32)
    ref_check(matmul(hip, w, x, hip.F32, 1, N), oracle.matmul_q4(x.reshape(-1), wq, sc, ze, 1, K, N, 32, K // 32))
    # prefill classes, fp16 activations
    for M_tune, Ms in ((64, (64, 40, 128)), (16, (16, 9, 32)), (300, (130, 300))):
        print(f"prepare prefill M={M_tune} f16", flush=True)
        assert hip.q4_prepare(w, M_tune, hip.F16) == 0
        name, cached = hip.q4_plan_info(w, M_tune, hip.F16)
        assert not cached
        assert name in ("generic", "gemm") or name.split("-")[0] in ("pipe", "skinny", "big", "wide", "stream")
        if M_tune > 32:
            assert not name.startswith(("skinny-", "stream-"))
        else:
            assert not name.startswith(("big-", "wide-"))
        for M in Ms:
            assert hip.q4_plan_info(w, M, hip.F16)[0] == name  # one plan per class
            x = synth.activations(g, M, K, np.float16)
            got = matmul(hip, w, x, hip.F16, M, N)
            want = oracle.matmul_q4(x.astype(np.float32).reshape(-1), wq, sc, ze, M, K, N, 32, K // 32)
            tier_check(got, want, TIER_F32_ACC)
    assert hip.q4_plan_info(w, 1, hip.F16) is None  # no plan for a class never prepared
    w.close()


def test_plan_file_reused_and_signature_checked(hip, plans):
    K, N = 512, 256
    _, _, w = weights(hip, 501, K, N)
    print("prepare for the plan file", flush=True)
    assert hip.q4_prepare(w, 64, hip.F16) == 0
    first, cached = hip.q4_plan_info(w, 64, hip.F16)
    assert not cached
    files = [f for f in os.listdir(plans) if f.startswith("q4-plans-") and f.endswith(".txt")]
    assert len(files) == 1
    text = open(os.path.join(plans, files[0])).read().splitlines()
    assert text[0].startswith("signature v1|") and any(line.endswith(" " + first) for line in text[1:])
    # a new process (here: the plans forgotten) reads the plan back instead of tuning
    hip.q4_plans_reset()
    assert hip.q4_plan_info(w, 64, hip.F16) is None
    assert hip.q4_prepare(w, 64, hip.F16) == 0
    assert hip.q4_plan_info(w, 64, hip.F16) == (first, True)
    # a plan file written for another device or build is ignored
    with open(os.path.join(plans, files[0]), "w") as f:
        f.write("signature v1|another-device\n" + "\n".join(text[1:]) + "\n")
    hip.q4_plans_reset()
    assert hip.q4_prepare(w, 64, hip.F16) == 0
    assert hip.q4_plan_info(w, 64, hip.F16)[1] is False
    w.close()


def test_prepare_off_and_inside_session(hip, plans, monkeypatch):
    """Tuning disabled, or a session open: BYHIP_UNSUPPORTED and no plan, as the reference returns
    false (q4_autotune.nim:389-390)."""
    from bybylang_amd import _abi
    from bybylang_amd import gpubackend as gb
    _, _, w = weights(hip, 502, 256, 64)
    for var in ("BYHIP_Q4_TUNED", "BYHIP_GPU_AUTOTUNE"):
        monkeypatch.setenv(var, "0")
        assert hip.q4_prepare(w, 1, hip.F32) == _abi.BYHIP_UNSUPPORTED
        monkeypatch.delenv(var)
    assert gb.sessionBegin(gb.gbHip)
    assert hip.q4_prepare(w, 1, hip.F32) == _abi.BYHIP_UNSUPPORTED
    assert gb.sessionEnd(gb.gbHip)
    assert hip.q4_plan_info(w, 1, hip.F32) is None
    w.close()


def test_resident_prepare_q4_mirror(hip, oracle, plans):
    """residentPrepareQ4 on resident weights, then sessionMatmulQ4 (fp32) follows the plan."""
    from bybylang_amd import gpubackend as gb
    from bybylang_amd import synth
    K, N, M = 768, 300, 48
    g = synth.rng(503)
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    w = gb.residentUploadQ4(gb.gbHip, wq, sc, ze, K, N, 32, K // 32)
    print("residentPrepareQ4", flush=True)
    assert gb.residentPrepareQ4(w, 1) and gb.residentPrepareQ4(w, M)
    x = synth.activations(g, M, K, np.float32)
    assert gb.sessionBegin(gb.gbHip)
    hx = gb.sessionUpload(gb.gbHip, x.reshape(-1))
    c = gb.SessionHandle()
    assert gb.sessionMatmulQ4(gb.gbHip, hx, w, c, M)
    assert gb.sessionEnd(gb.gbHip), gb.sessionGetLastError(gb.gbHip)
    got = gb.sessionRead(gb.gbHip, c, M * N).reshape(M, N)
    tier_check(got, oracle.matmul_q4(x.reshape(-1), wq, sc, ze, M, K, N, 32, K // 32), TIER_F32_ACC)
    for h in (hx, c):
        gb.sessionFree(gb.gbHip, h)
    gb.residentFreeQ4(w)
