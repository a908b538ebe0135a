"""bybylang_amd - MI355X (gfx950) backend for BybyLang's quantized tile-GEMM path.

libbybyhip.so holds the HIP kernels and the C ABI (include/byhip.h). `device` gives numpy callers
typed access to it; `gpubackend` mirrors the reference's session API for the hip backend.
"""
from ._abi import HipBackendError, HipUnsupported, load  # noqa: F401

__all__ = ["HipBackendError", "HipUnsupported", "load"]
