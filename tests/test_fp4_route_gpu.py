"""The FP4-KM tile GEMM's route follows the decode table the buffer holds when the kernels run.

The route (the fp16 MFMA GEMM when every product lut[code] * lut[16 + scale byte] is exact in fp16,
otherwise the exact fp32 GEMM; the reference computes in fp32, cpu_vm.c:583-628) is chosen from the
table's host copy outside recordings. Inside a recording, and for a table with no host copy (larger
than 64 KB, or last written by a kernel), a one-block kernel classifies the table on the device and
both routes are queued, each gated on its flag. So a recording replayed after the table changes
computes with the new table's route, and no call waits for the device to read a table.

Bar: the reference test's tolerance, max|diff| <= 1e-4 * max(1, peak), against the oracle's tile
GEMM with the table of that replay. The data make the two routes' results differ by a known margin:
codes of powers of two (0.5, 1, 2, 4), positive activations, and a "thirds" table whose products
are all 2^e / 3, which fp16 rounds down by the same 2.4e-4 of their value, so the fp16 route on it
misses the bar by more than twice (the planted-mistake check below).
"""
import numpy as np
import pytest

from bybylang_amd import _abi, synth
from parity import max_abs_rel, ref_check

pytestmark = pytest.mark.gpu

M, K, N = 24, 256, 96


POW2_CODES = np.array([1, 2, 4, 6], np.uint8)  # E2M1 0.5, 1, 2, 4


def case(seed):
    g = synth.rng(seed)
    codes = POW2_CODES[g.integers(0, 4, size=(N, K))]
    sb = g.integers(0, 256, size=(N, K // 32), dtype=np.uint8)
    packed = np.concatenate([synth.fp4km_pack(codes).reshape(-1), sb.reshape(-1)])
    halves = np.zeros(272, np.float32)
    halves[:16] = synth.E2M1
    halves[16:] = (1 + np.arange(256) % 13).astype(np.float32) / 64  # products exact in fp16
    odd = halves.copy()
    odd[16:] = np.ldexp(np.float32(1.0 / 3.0), np.arange(256) % 5 - 2)  # products 2^e / 3
    x = np.abs(synth.activations(g, M, K, np.float32)).reshape(-1)
    return packed, halves, odd, x, codes, sb


@pytest.fixture
def gb(hip):
    from bybylang_amd import gpubackend as g
    yield g
    g.sessionRecoverQueue(g.gbHip)
    _abi.check(_abi.load().byhip_session_set_direct_replay(0))


@pytest.mark.parametrize("direct", [False, True], ids=["graph", "direct"])
def test_recorded_tile_gemm_follows_the_table(gb, oracle, direct):
    """Record with a table of halves, replay, upload thirds, replay, upload halves, replay."""
    packed, halves, odd, x, _, _ = case(8100 + direct)
    lib = _abi.load()
    _abi.check(lib.byhip_session_set_direct_replay(int(direct)))
    words = np.zeros((packed.size + 3) // 4, np.float32)
    words.view(np.uint8)[: packed.size] = packed
    assert gb.sessionBegin(gb.gbHip)
    hx = gb.sessionUpload(gb.gbHip, x)
    hw = gb.sessionUpload(gb.gbHip, words)
    hl = gb.sessionUpload(gb.gbHip, halves)
    ho = gb.sessionAllocScratch(gb.gbHip, M * N)
    assert gb.sessionEnd(gb.gbHip)
    assert gb.sessionBeginRecording(gb.gbHip)
    assert gb.sessionFp4GemmTensorCore(gb.gbHip, hx, hw, hl, ho, M, K, N)
    assert gb.sessionEnd(gb.gbHip), gb.sessionGetLastError(gb.gbHip)
    rid = gb.sessionLastRecording(gb.gbHip)
    for name, table in (("halves", halves), ("thirds", odd), ("halves again", halves)):
        _abi.check(lib.byhip_upload(hl.hipHandle, 0, table.ctypes.data, table.nbytes))
        print(f"replay with {name}", flush=True)
        assert gb.sessionReplay(gb.gbHip, rid, 1), gb.sessionGetLastError(gb.gbHip)
        want = oracle.tile_gemm(0, M, K, N, N * (K // 2), 0, packed, table, x)
        ref_check(gb.sessionRead(gb.gbHip, ho, M * N), want)
    gb.sessionFreeRecording(gb.gbHip, rid)
    for h in (hx, hw, hl, ho):
        gb.sessionFree(gb.gbHip, h)


@pytest.mark.parametrize("table_kind", ["halves", "thirds"])
def test_table_without_host_copy(hip, oracle, table_kind):
    """A table at an offset inside a 128 KB buffer (no host copy is kept past 64 KB), outside
    recordings: classified on the device, with no wait for a device read."""
    packed, halves, odd, x, _, _ = case(8200)
    table = halves if table_kind == "halves" else odd
    big = np.zeros(32768, np.float32)
    base = 20000
    big[base: base + 272] = table
    want = oracle.tile_gemm(0, M, K, N, N * (K // 2), 0, packed, table, x)
    y = hip.DeviceBuffer(M * N * 4)
    print(f"no host copy, {table_kind}", flush=True)
    hip.fp4km_tile_gemm(hip.DeviceBuffer.from_array(x), hip.F32, hip.DeviceBuffer.from_array(packed), N * (K // 2),
                        hip.DeviceBuffer.from_array(big), base, y, hip.F32, M, K, N)
    ref_check(y.read(np.float32), want)


def test_kernel_write_drops_the_host_copy(hip, oracle):
    """A small table buffer uploaded with halves (the library keeps a host copy), then overwritten by
    a kernel: a tile GEMM with 272 outputs written into it (x[0] = 1/3, so the new entries are
    thirds). The next tile GEMM on that buffer must take the route of what it now holds, read back
    here for the oracle: the host copy of the halves is no longer used."""
    packed, halves, odd, x, _, _ = case(8250)
    lut = hip.DeviceBuffer.from_array(halves.copy())
    # writer: y[n] = x[0] * halves[code(n, 0)] * halves[16 + sb(n)] with x[0] = 1/3, a power-of-two
    # code and a scale entry of 1, 2, 4 or 8 (/ 64): every written entry is 2^e / 3
    Kw, Nw = 32, 272
    g = synth.rng(8251)
    codes = POW2_CODES[g.integers(0, 4, size=(Nw, Kw))]
    sb = np.array([0, 1, 3, 7], np.uint8)[g.integers(0, 4, size=(Nw, 1))]  # 1 + sb % 13 in {1, 2, 4, 8}
    wblob = np.concatenate([synth.fp4km_pack(codes).reshape(-1), sb.reshape(-1)])
    xw = np.zeros(Kw, np.float32)
    xw[0] = np.float32(1.0 / 3.0)
    hip.fp4km_tile_gemm(hip.DeviceBuffer.from_array(xw), hip.F32, hip.DeviceBuffer.from_array(wblob), Nw * (Kw // 2),
                        hip.DeviceBuffer.from_array(halves), 0, lut, hip.F32, 1, Kw, Nw)
    now = lut.read(np.float32)
    prod = np.outer(now[16:], now[:16]).astype(np.float32)
    assert np.all(np.isfinite(prod)) and np.all(prod > 0) and np.all(prod.astype(np.float16).astype(np.float32) != prod)
    y = hip.DeviceBuffer(M * N * 4)
    print("table written by a kernel", flush=True)
    hip.fp4km_tile_gemm(hip.DeviceBuffer.from_array(x), hip.F32, hip.DeviceBuffer.from_array(packed), N * (K // 2),
                        lut, 0, y, hip.F32, M, K, N)
    ref_check(y.read(np.float32), oracle.tile_gemm(0, M, K, N, N * (K // 2), 0, packed, now, x))


def test_planted_route_mistake_is_caught(oracle):
    """The bar separates the routes: each weight of the thirds table rounded to fp16 (what the fp16
    route would compute with) misses 1e-4 of the peak against the oracle by more than twice, which
    the exact route meets."""
    packed, halves, odd, x, codes, sb = case(8300)
    want = oracle.tile_gemm(0, M, K, N, N * (K // 2), 0, packed, odd, x)
    wv = (odd[codes] * np.repeat(odd[16 + sb.astype(np.int64)], 32, axis=1)).astype(np.float32)
    wrong = x.reshape(M, K).astype(np.float64) @ wv.astype(np.float16).astype(np.float64).T
    assert max_abs_rel(wrong, want) > 2e-4
