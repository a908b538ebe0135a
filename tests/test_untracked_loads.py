"""The streaming Q4 GEMM issues its weight and scale loads as inline assembly, outside the compiler's
wait-count tracking (byhip_stream.hip). Its correctness then rests on the kernel's own waits: no
instruction may read or overwrite a register whose load is still in flight. This compiles the
kernel for gfx950 and walks every instantiation's assembly (asm_hazards.simulate) through three
K-loop iterations and through the path that skips the loop, and checks that nothing touches a
pending register; the walk's load count and loads in flight must be the kernel's own ((D - 1)
sub-steps ahead, L loads per sub-step), so a wrong path cannot pass unnoticed. A copy of the
assembly with one K-loop wait taken out must fail (the check catches a missing wait).
CPU only: it needs hipcc, not a GPU."""
import os
import re
import shutil
import subprocess

import pytest

from asm_hazards import kernel_body, kernel_names, simulate

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC") or ("/opt/rocm/bin/hipcc" if os.path.exists("/opt/rocm/bin/hipcc") else shutil.which("hipcc"))
PREFIX = "_ZN5byhip12_GLOBAL__N_114q4_gemm_stream"


@pytest.fixture(scope="module")
def stream_asm(tmp_path_factory):
    if not HIPCC:
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("asm") / "stream.s"
    src = os.path.join(ROOT, "bybylang_amd", "csrc", "byhip_stream.hip")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(ROOT, "bybylang_amd", "csrc"),
           "--cuda-device-only", "-S", src, "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return out.read_text()


def shape(name):
    fm, fn, _, d = (int(v) for v in re.findall(r"Li(\d+)E", name[len(PREFIX):])[:4])
    return fm, fn, d


def test_every_instantiation_waits_before_use(stream_asm):
    names = kernel_names(stream_asm, PREFIX)
    assert len(names) >= 48
    for name in names:
        fm, fn, d = shape(name)
        per_step = 2 * fm + 2 * fn  # direct activation loads, weight loads, scale loads
        raw = kernel_body(stream_asm, name)
        run = simulate(raw, iterations=3, enter_loop=True)
        assert run["hazards"] == [], (name, run["hazards"][:3])
        assert run["iterations"] == 3, name
        assert run["loads"] == (d - 1) * per_step + 3 * d * per_step, (name, run["loads"])
        assert run["max_in_flight"] == (d - 1) * per_step, (name, run["max_in_flight"])
        skip = simulate(raw, iterations=0, enter_loop=False)
        assert skip["hazards"] == [], (name, skip["hazards"][:3])
        assert skip["loads"] == (d - 1) * per_step, (name, skip["loads"])


def test_missing_wait_is_caught(stream_asm):
    name = next(n for n in kernel_names(stream_asm, PREFIX) if shape(n) == (2, 2, 4))
    raw = kernel_body(stream_asm, name)
    waits = [k for k, l in enumerate(raw) if re.search(r"s_waitcnt vmcnt\(\d+\)", l)]
    header = next(k for k, l in enumerate(raw) if "Inner Loop Header" in l)
    k = next(k for k in waits if k > header)  # the first wait inside the K loop
    planted = raw[:k] + ["\ts_nop 0"] + raw[k + 1:]
    assert simulate(planted, iterations=3)["hazards"]
