"""The C ABI library and the host-side policy, without a GPU.

- libbybyhip.so loads and exports exactly the entry points include/byhip.h declares;
- the entry points fail loudly (error code + byhip_last_error) when no device is initialised, and
  an injected fault surfaces through them;
- the session mirror's selection and fallback policy (parseBackend, setForbidCpuFallback,
  handleGpuFailure, gpubackend.nim:75-114) behaves as the reference's.
"""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "byhip.h")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^(?:int|void|double|unsigned long long|const char\*|void\*)\s+\**(byhip_\w+)\(", text, re.M)))


def test_header_and_library_agree():
    from bybylang_amd import _abi
    lib = _abi.load()
    names = declared()
    assert len(names) >= 30
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(_abi.SIGNATURES) == names
    out = subprocess.run(["nm", "-D", "--defined-only", _abi.LIB_PATH], capture_output=True, text=True).stdout
    exported = sorted(set(re.findall(r" T (byhip_\w+)", out)))
    assert exported == names


def test_library_is_gfx950_code_object():
    from bybylang_amd import _abi
    data = open(_abi.LIB_PATH, "rb").read()
    assert b"gfx950" in data


def _gpu_present():
    from bybylang_amd import _abi
    return _abi.load().byhip_init(0) == 0


def test_calls_without_device_fail_loudly():
    from bybylang_amd import _abi
    lib = _abi.load()
    if _gpu_present():
        pytest.skip("a GPU is present; this checks the no-device path")
    assert lib.byhip_init(0) == _abi.BYHIP_ERROR
    assert "no HIP device" in _abi.last_error() or "gfx950" in _abi.last_error()
    p = C.c_void_p()
    assert lib.byhip_alloc(16, C.byref(p)) == _abi.BYHIP_ERROR
    assert "not initialised" in _abi.last_error()
    assert lib.byhip_session_begin() == _abi.BYHIP_ERROR
    assert lib.byhip_q4_matmul(None, 0, None, None, 0, 1) == _abi.BYHIP_ERROR


def test_fault_injection_reaches_caller():
    from bybylang_amd import _abi
    lib = _abi.load()
    lib.byhip_fault_inject(2)
    assert lib.byhip_session_begin() == _abi.BYHIP_ERROR
    assert _abi.last_error() == "byhip: injected fault"
    assert lib.byhip_synchronize() == _abi.BYHIP_ERROR
    assert _abi.last_error() == "byhip: injected fault"
    lib.byhip_fault_inject(0)
    lib.byhip_clear_error()
    assert _abi.last_error() == ""


def test_parse_backend():
    from bybylang_amd import gpubackend as gb
    assert gb.parseBackend(" HIP ") is gb.gbHip
    assert gb.parseBackend("cuda") is gb.gbVulkan  # gpubackend.nim:109
    assert str(gb.gbHip) == "hip"
    with pytest.raises(ValueError, match="unknown BybyLang backend"):
        gb.parseBackend("rocm")


def test_forbid_cpu_fallback_policy():
    """gpuMatmulQ4 after a device failure: raises under forbid; otherwise hands the call to the
    caller's CPU path (the reference's cpuDequantMatmulQ4Fallback) or re-raises without one."""
    from bybylang_amd import _abi
    from bybylang_amd import gpubackend as gb
    M, K, N, grp = 1, 64, 16, 32
    a = np.zeros(M * K, np.float32)
    wq = np.zeros(N * K // 2, np.uint8)
    sc = np.ones(N * K // grp, np.float32)
    ze = np.zeros(N * K // grp, np.float32)
    sentinel = np.full(M * N, 7.0, np.float32)
    calls = []

    def caller_cpu_path(*args):
        calls.append(args[4:])
        return sentinel

    lib = _abi.load()
    try:
        gb.setForbidCpuFallback(True)
        lib.byhip_fault_inject(1)
        with pytest.raises(_abi.HipBackendError, match="CPU fallback is forbidden"):
            gb.gpuMatmulQ4(gb.gbHip, a, wq, sc, ze, M, K, N, grp, K // grp, cpuFallback=caller_cpu_path)
        assert not calls
        gb.setForbidCpuFallback(False)
        lib.byhip_fault_inject(1)
        out = gb.gpuMatmulQ4(gb.gbHip, a, wq, sc, ze, M, K, N, grp, K // grp, cpuFallback=caller_cpu_path)
        assert out is sentinel and calls == [(M, K, N, grp, K // grp)]
        lib.byhip_fault_inject(1)
        # with a device the injected fault fails the call; without one, device selection does
        with pytest.raises(_abi.HipBackendError, match="injected fault|no HIP device"):
            gb.gpuMatmulQ4(gb.gbHip, a, wq, sc, ze, M, K, N, grp, K // grp)
    finally:
        lib.byhip_fault_inject(0)
        gb.setForbidCpuFallback(False)


def test_missing_library_fails_loudly(tmp_path):
    from bybylang_amd import _abi
    saved = _abi._lib
    try:
        _abi._lib = None
        with pytest.raises(_abi.HipBackendError, match="is missing"):
            _abi.load(str(tmp_path / "libbybyhip.so"))
    finally:
        _abi._lib = saved


def test_session_mirror_rejects_other_backends():
    from bybylang_amd import gpubackend as gb
    with pytest.raises(ValueError):
        gb.sessionBegin(gb.gbVulkan)


def test_read_only_mapping(tmp_path):
    """openReadOnlyMapping / unmapReadOnlyFile (mapped_file.nim:9-20): the mapping exposes the
    file's bytes at `data`; unmapping clears it; an empty file maps to nothing."""
    import ctypes
    from bybylang_amd import gpubackend as gb
    blob = bytes(range(256)) * 17
    f = tmp_path / "ckpt.bin"
    f.write_bytes(blob)
    m = gb.openReadOnlyMapping(str(f))
    assert m.size == len(blob) and m.data
    assert ctypes.string_at(m.data, m.size) == blob
    gb.unmapReadOnlyFile(m)
    assert m.data == 0 and m.size == 0
    e = tmp_path / "empty.bin"
    e.write_bytes(b"")
    me = gb.openReadOnlyMapping(str(e))
    assert me.size == 0 and me.data == 0
    gb.unmapReadOnlyFile(me)
