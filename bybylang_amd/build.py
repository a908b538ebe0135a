"""Builds libbybyhip.so (the HIP kernels and the C ABI) in-tree for gfx950.

    python -m bybylang_amd.build          # or bybylang_amd.build.build()

Every .hip source under csrc/ is compiled by hipcc in parallel into _build/, then linked into
bybylang_amd/libbybyhip.so. Packed fp32 instructions are disabled for every kernel
(-target-feature -packed-fp32-ops).
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(PKG, "libbybyhip.so")
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def source_hash() -> str:
    """FNV-1a (64-bit) of the kernel sources and the C ABI header, in name order: the tuned-plan
    cache is keyed by it, so plans tuned for other kernels are not reused."""
    h = 0xCBF29CE484222325
    files = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.h")) +
                   glob.glob(os.path.join(INCLUDE, "*.h")))
    for path in files:
        with open(path, "rb") as f:
            for b in os.path.basename(path).encode() + f.read():
                h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return f"{h:016x}"


def common_flags() -> list[str]:
    return [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
            "-Wno-unused-function", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            f"-I{INCLUDE}", f"-I{CSRC}", f'-DBYHIP_SOURCE_HASH="{source_hash()}"']


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [hipcc()] + common_flags() + ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; that line is harmless.
    noise = ("packed-fp32-ops", "unknown target feature")
    msgs = [ln for ln in (r.stdout + r.stderr).splitlines() if not any(t in ln for t in noise)]
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n" + "\n".join(msgs))
    if msgs and any("warning" in m or "error" in m for m in msgs):
        sys.stderr.write("\n".join(msgs) + "\n")
    return obj


def build(jobs: int | None = None) -> str:
    """Compiles every kernel source and links libbybyhip.so; returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    # --no-undefined: a kernel whose host stub the compiler did not emit fails here, not at load.
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
