"""Session semantics on the MI355X, through the Python mirror of the reference's API and the C ABI.

Record / replay (sessionCanRecord .. sessionFreeRecording, gpubackend.nim:2502-2590;
vulkan_driver.nim:1659-2030): a recording of sessionMatmulQ4 over rotating resident weights and an
FP4-KM tile GEMM is replayed several times, with new activations uploaded between replays, and
each replay is checked against the oracle. Freed and unknown ids are refused; entry points that
wait for the device are refused while recording (the recording itself stays usable).
sessionCommitContinue (2444-2467), sessionRecoverQueue (2593), a free issued inside an open session
(deferred to its end, vulkan_driver.nim:1192, 1817-1819) and sessionGpuSeconds (2617-2632).
"""
import numpy as np
import pytest

from bybylang_amd import _abi, synth
from parity import ref_check

pytestmark = pytest.mark.gpu


@pytest.fixture
def gb(hip):
    from bybylang_amd import gpubackend as g
    yield g
    # leave no session open and recordings as HIP graphs for the next test
    g.sessionRecoverQueue(g.gbHip)
    _abi.check(_abi.load().byhip_session_set_direct_replay(0))


def fp4_case(g, M, K, N):
    codes = g.integers(0, 16, size=(N, K), dtype=np.uint8)
    sb = g.integers(0, 256, size=(N, K // 32), dtype=np.uint8)
    packed = np.concatenate([synth.fp4km_pack(codes).reshape(-1), sb.reshape(-1)])
    table = np.zeros(272, np.float32)
    table[:16] = synth.E2M1
    table[16:] = (1 + np.arange(256) % 13).astype(np.float32) / 64  # the reference test's table
    words = np.zeros((packed.size + 3) // 4, np.float32)
    words.view(np.uint8)[: packed.size] = packed
    return packed, words, table


@pytest.mark.parametrize("direct", [False, True], ids=["graph", "direct"])
def test_record_replay_rotating_weights_and_tile_gemm(gb, oracle, direct):
    """As HIP graphs, and with the recording's launches kept and replayed directly
    (byhip_session_set_direct_replay): the same results either way."""
    _abi.check(_abi.load().byhip_session_set_direct_replay(int(direct)))
    g = synth.rng(9100)
    M, K, N, copies = 3, 1024, 512, 3
    mats = [synth.q4_weights(g, N, K)[:3] for _ in range(copies)]
    ws = [gb.residentUploadQ4(gb.gbHip, wq, sc, ze, K, N, 32, K // 32) for wq, sc, ze in mats]
    Mf, Kf, Nf = 20, 256, 96
    packed, words, table = fp4_case(g, Mf, Kf, Nf)
    assert gb.sessionBegin(gb.gbHip)
    hx = gb.sessionUpload(gb.gbHip, np.zeros(M * K, np.float32))
    hys = [gb.sessionAllocScratch(gb.gbHip, M * N) for _ in range(copies)]
    hfx = gb.sessionUpload(gb.gbHip, np.zeros(Mf * Kf, np.float32))
    hfw = gb.sessionUpload(gb.gbHip, words)
    hfl = gb.sessionUpload(gb.gbHip, table)
    hfo = gb.sessionAllocScratch(gb.gbHip, Mf * Nf)
    assert gb.sessionEnd(gb.gbHip)

    assert gb.sessionCanRecord(gb.gbHip)
    assert gb.sessionBeginRecording(gb.gbHip)
    for i in range(copies):
        assert gb.sessionMatmulQ4(gb.gbHip, hx, ws[i], hys[i], M)
    assert gb.sessionFp4GemmTensorCore(gb.gbHip, hfx, hfw, hfl, hfo, Mf, Kf, Nf)
    assert gb.sessionEnd(gb.gbHip), gb.sessionGetLastError(gb.gbHip)
    rid = gb.sessionLastRecording(gb.gbHip)
    assert rid >= 0

    lib = _abi.load()
    for rep in range(3):
        x = synth.activations(g, M, K, np.float32).reshape(-1) * np.float32(10.0 ** (rep - 1))
        xf = synth.activations(g, Mf, Kf, np.float32).reshape(-1)
        _abi.check(lib.byhip_upload(hx.hipHandle, 0, x.ctypes.data, x.nbytes))
        _abi.check(lib.byhip_upload(hfx.hipHandle, 0, xf.ctypes.data, xf.nbytes))
        print(f"replay {rep}", flush=True)
        assert gb.sessionReplay(gb.gbHip, rid, 1), gb.sessionGetLastError(gb.gbHip)
        for i, (wq, sc, ze) in enumerate(mats):
            ref_check(gb.sessionRead(gb.gbHip, hys[i], M * N),
                      oracle.matmul_q4(x, wq, sc, ze, M, K, N, 32, K // 32))
        ref_check(gb.sessionRead(gb.gbHip, hfo, Mf * Nf),
                  oracle.tile_gemm(0, Mf, Kf, Nf, Nf * (Kf // 2), 0, packed, table, xf))

    # several replays back to back leave the same outputs
    before = gb.sessionRead(gb.gbHip, hys[0], M * N)
    assert gb.sessionReplay(gb.gbHip, rid, 4)
    assert np.array_equal(gb.sessionRead(gb.gbHip, hys[0], M * N), before)

    gb.sessionFreeRecording(gb.gbHip, rid)
    assert not gb.sessionReplay(gb.gbHip, rid, 1)
    assert "no recording" in gb.sessionGetLastError(gb.gbHip)
    assert not gb.sessionReplay(gb.gbHip, 10_000, 1)
    for h in [hx, hfx, hfw, hfl, hfo] + hys:
        gb.sessionFree(gb.gbHip, h)
    for w in ws:
        gb.residentFreeQ4(w)


@pytest.mark.parametrize("direct", [False, True], ids=["graph", "direct"])
def test_waiting_calls_refused_while_recording(gb, hip, direct):
    """Reads, uploads, frees and syncs wait for the device: refused inside a recording, which
    then still ends, replays and computes."""
    _abi.check(_abi.load().byhip_session_set_direct_replay(int(direct)))
    g = synth.rng(9200)
    K, N = 256, 64
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    w = hip.Q4Weights(wq, sc, ze, K, N, 32, K // 32)
    x = hip.DeviceBuffer.from_array(synth.activations(g, 1, K, np.float32).reshape(-1))
    y = hip.DeviceBuffer(N * 4)
    lib = _abi.load()
    assert gb.sessionBeginRecording(gb.gbHip)
    hip.q4_matmul(x, hip.F32, w, y, hip.F32, 1)
    out = np.zeros(N, np.float32)
    assert lib.byhip_read(y.ptr, 0, out.ctypes.data, out.nbytes) == _abi.BYHIP_ERROR
    assert "not allowed while a session is recorded" in _abi.last_error()
    assert lib.byhip_upload(y.ptr, 0, out.ctypes.data, out.nbytes) == _abi.BYHIP_ERROR
    assert lib.byhip_synchronize() == _abi.BYHIP_ERROR
    assert lib.byhip_memset(y.ptr, 0, out.nbytes) == _abi.BYHIP_ERROR
    assert gb.sessionEnd(gb.gbHip), gb.sessionGetLastError(gb.gbHip)
    rid = gb.sessionLastRecording(gb.gbHip)
    want = y.read(np.float32)
    y.zero()
    assert gb.sessionReplay(gb.gbHip, rid, 1)
    assert np.array_equal(y.read(np.float32), want)
    gb.sessionFreeRecording(gb.gbHip, rid)


def test_commit_continue_recover_deferred_free(gb, oracle):
    g = synth.rng(9300)
    M, K, N = 2, 512, 128
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    w = gb.residentUploadQ4(gb.gbHip, wq, sc, ze, K, N, 32, K // 32)
    x = synth.activations(g, M, K, np.float32).reshape(-1)
    # commit_continue: submits without waiting; the session stays open and ends normally
    assert gb.sessionBegin(gb.gbHip)
    ha = gb.sessionUpload(gb.gbHip, x)
    hc1, hc2 = gb.SessionHandle(), gb.SessionHandle()
    assert gb.sessionMatmulQ4(gb.gbHip, ha, w, hc1, M)
    assert gb.sessionCommitContinue(gb.gbHip)
    assert not gb.sessionBegin(gb.gbHip)  # still open
    assert gb.sessionMatmulQ4(gb.gbHip, ha, w, hc2, M)
    # a free issued inside the open session is deferred: the queued work still reads `ha`
    gb.sessionFree(gb.gbHip, ha)
    assert gb.sessionEnd(gb.gbHip), gb.sessionGetLastError(gb.gbHip)
    want = oracle.matmul_q4(x, wq, sc, ze, M, K, N, 32, K // 32)
    ref_check(gb.sessionRead(gb.gbHip, hc1, M * N), want)
    ref_check(gb.sessionRead(gb.gbHip, hc2, M * N), want)
    assert not gb.sessionCommitContinue(gb.gbHip)  # no session open
    # recover: drops an open session so a new one can begin
    assert gb.sessionBegin(gb.gbHip)
    assert gb.sessionRecoverQueue(gb.gbHip)
    assert gb.sessionBegin(gb.gbHip)
    assert gb.sessionEnd(gb.gbHip)
    for h in (hc1, hc2):
        gb.sessionFree(gb.gbHip, h)
    gb.residentFreeQ4(w)


def test_gpu_seconds(gb):
    """sessionGpuSeconds counts the timed sessions since sessionSetGpuTiming, and replays."""
    g = synth.rng(9400)
    K, N = 4096, 4096
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    w = gb.residentUploadQ4(gb.gbHip, wq, sc, ze, K, N, 32, K // 32)
    assert gb.sessionSetGpuTiming(gb.gbHip, True)
    assert gb.sessionGpuSeconds(gb.gbHip) == 0.0
    assert gb.sessionBegin(gb.gbHip)
    ha = gb.sessionUpload(gb.gbHip, synth.activations(g, 1, K, np.float32).reshape(-1))
    hc = gb.SessionHandle()
    for _ in range(20):
        assert gb.sessionMatmulQ4(gb.gbHip, ha, w, hc, 1)
    assert gb.sessionEnd(gb.gbHip)
    t1 = gb.sessionGpuSeconds(gb.gbHip)
    assert 0.0 < t1 < 1.0
    assert gb.sessionBeginRecording(gb.gbHip)
    assert gb.sessionMatmulQ4(gb.gbHip, ha, w, hc, 1)
    assert gb.sessionEnd(gb.gbHip)
    rid = gb.sessionLastRecording(gb.gbHip)
    assert gb.sessionReplay(gb.gbHip, rid, 10)
    assert gb.sessionGpuSeconds(gb.gbHip) > t1
    assert gb.sessionSetGpuTiming(gb.gbHip, False)
    assert gb.sessionGpuSeconds(gb.gbHip) == 0.0
    gb.sessionFreeRecording(gb.gbHip, rid)
    for h in (ha, hc):
        gb.sessionFree(gb.gbHip, h)
    gb.residentFreeQ4(w)


@pytest.mark.parametrize("direct", [False, True], ids=["graph", "direct"])
def test_timing_marks_direct_and_recorded(gb, hip, direct):
    """The measurement marks (no counterpart in the reference): work launched directly between
    byhip_session_mark(0) and (1) is counted by byhip_session_take_marks, the same work recorded
    between the two marks by byhip_session_replay_marked (recordings as graphs or as kept
    launches); an interval with no end mark and a marked replay of a recording without marks are
    refused."""
    lib = _abi.load()
    _abi.check(lib.byhip_session_set_direct_replay(int(direct)))
    g = synth.rng(9500)
    K, N, n = 4096, 4096, 50
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    w = hip.Q4Weights(wq, sc, ze, K, N, 32, K // 32)
    x = hip.DeviceBuffer.from_array(synth.activations(g, 1, K, np.float16).reshape(-1))
    y = hip.DeviceBuffer(N * 2)
    run = lambda: hip.q4_matmul(x, hip.F16, w, y, hip.F16, 1)  # noqa: E731
    run()
    assert gb.sessionSetGpuTiming(gb.gbHip, True)
    _abi.check(lib.byhip_session_mark(0), "mark")
    for _ in range(n):
        run()
    _abi.check(lib.byhip_session_mark(1), "mark")
    _abi.check(lib.byhip_session_take_marks(), "marks")
    t_direct = gb.sessionGpuSeconds(gb.gbHip)
    # 50 launches of a 33 MB GEMV (the weights stay in the 256 MB Infinity Cache between them): at
    # least 1 us each even from there, and well under a second in all
    assert 50 * 1e-6 < t_direct < 1.0

    assert gb.sessionBeginRecording(gb.gbHip)
    _abi.check(lib.byhip_session_mark(0), "mark")
    for _ in range(n):
        run()
    _abi.check(lib.byhip_session_mark(1), "mark")
    assert gb.sessionEnd(gb.gbHip)
    rid = gb.sessionLastRecording(gb.gbHip)
    _abi.check(lib.byhip_session_replay_marked(rid), "replay")
    t_rec = gb.sessionGpuSeconds(gb.gbHip) - t_direct
    assert 50 * 1e-6 < t_rec < 1.0

    _abi.check(lib.byhip_session_mark(0), "mark")
    with pytest.raises(_abi.HipBackendError, match="no pair of timing marks"):
        _abi.check(lib.byhip_session_take_marks(), "marks")
    assert gb.sessionBeginRecording(gb.gbHip)
    run()
    assert gb.sessionEnd(gb.gbHip)
    bare = gb.sessionLastRecording(gb.gbHip)
    with pytest.raises(_abi.HipBackendError, match="no pair of timing marks"):
        _abi.check(lib.byhip_session_replay_marked(bare), "replay")
    assert gb.sessionSetGpuTiming(gb.gbHip, False)
    for r in (rid, bare):
        gb.sessionFreeRecording(gb.gbHip, r)
    for b in (x, y, w):
        b.close()
