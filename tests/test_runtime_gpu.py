"""The library's measurement entry points on the MI355X: the plain device copy (the transfer the
traffic counters are scaled by) and the streaming read (what the kernels' reads are compared
with). Both must move every byte exactly once."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_debug_copy_moves_every_byte(hip):
    from bybylang_amd import _abi
    g = np.random.default_rng(11)
    a = g.integers(0, 2**32, size=(1 << 20) // 4 + 12, dtype=np.uint32)  # a tail past 1 MiB
    src = hip.DeviceBuffer.from_array(a)
    dst = hip.DeviceBuffer(a.nbytes)
    print("debug copy", a.nbytes, flush=True)
    _abi.check(_abi.load().byhip_debug_copy(dst.ptr, src.ptr, a.nbytes))
    assert np.array_equal(dst.read(np.uint32, a.size), a)


@pytest.mark.parametrize("runs,tail", [(3, 100), (0, 7), (5000, 0)])
def test_debug_read_folds_every_word(hip, runs, tail):
    """Each wave's sink word is the XOR fold of what it read: per 16-byte word the 32-bit sum of
    its four words, runs of 8 KB (512 words) dealt to the waves round-robin, then the tail words
    (their first 32 bits) one per thread. Recomputed here from the same buffer."""
    from bybylang_amd import _abi
    cus = hip.device_info()["compute_units"]
    nwaves, threads = 16 * cus, 64 * 16 * cus
    n = runs * 512 + tail  # 16-byte words
    g = np.random.default_rng(12 + runs)
    words = g.integers(0, 2**32, size=(n, 4), dtype=np.uint32)
    src = hip.DeviceBuffer.from_array(words)
    sink = hip.DeviceBuffer.from_array(np.full(nwaves, 0xDEADBEEF, np.uint32))
    print(f"debug read runs={runs} tail={tail}", flush=True)
    _abi.check(_abi.load().byhip_debug_read(src.ptr, n * 16, sink.ptr, nwaves * 4))
    got = sink.read(np.uint32, nwaves)
    want = np.zeros(nwaves, np.uint32)
    sums = words.astype(np.uint64).sum(axis=1).astype(np.uint32)  # modulo 2^32
    if runs:
        per_run = np.bitwise_xor.reduce(sums[: runs * 512].reshape(runs, 512), axis=1)
        for r in range(runs):
            want[r % nwaves] ^= per_run[r]
    for i in range(tail):  # tail word i goes to thread i (wave i // 64)
        want[(i % threads) // 64] ^= words[runs * 512 + i, 0]
    assert np.array_equal(got, want)
