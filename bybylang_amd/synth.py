"""Synthetic inputs in the benchmark configurations' formats (deterministic, numpy PCG64).

Q4 block-32 (configs 0-2, 4): int4 codes uniform in [-8, 7] stored as q = code + 8 (two per byte,
even k in the low nibble, the reference's layout, cpu_kernels_impl.inc:311-312), zero point 8.0,
one fp16 scale |N(0, 0.02)| + 1e-4 per 32 values along K, given to the reference API as fp32.
MXFP4 (config 3): E2M1 codes uniform over all 16 values, one E8M0 exponent per 32 values drawn
uniform from 2^-4 .. 2^2 (bytes 123..129), in the FP4-KM packing (byte j of a group holds element j
low and element j + 16 high, session_vm.nim:384-388); scale bytes follow the nibbles.
"""
from __future__ import annotations

import numpy as np

E2M1 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6], dtype=np.float32)


def rng(seed: int = 0) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def q4_weights(g: np.random.Generator, N: int, K: int, group: int = 32):
    """Returns (wq [N*K/2] u8, scales [N*K/group] f32 (fp16 values), zeros f32, codes [N, K] i8)."""
    codes = g.integers(-8, 8, size=(N, K), dtype=np.int8)
    q = (codes + 8).astype(np.uint8)
    wq = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8).reshape(-1)
    ng = K // group
    scales = (np.abs(g.normal(0.0, 0.02, size=(N, ng))) + 1e-4).astype(np.float16).astype(np.float32)
    zeros = np.full(N * ng, 8.0, dtype=np.float32)
    return wq, scales.reshape(-1), zeros, codes


def activations(g: np.random.Generator, M: int, K: int, dtype=np.float16) -> np.ndarray:
    return g.standard_normal((M, K), dtype=np.float32).astype(dtype)


def fp4km_pack(codes: np.ndarray) -> np.ndarray:
    """codes [R, K] (0..15) -> FP4-KM nibble bytes [R, K/2]: byte j of group g = element j | j+16."""
    R, K = codes.shape
    c = codes.reshape(R, K // 32, 2, 16).astype(np.uint8)
    return (c[:, :, 0, :] | (c[:, :, 1, :] << 4)).reshape(R, K // 2)


def mxfp4_operand(g: np.random.Generator, R: int, K: int):
    """An MXFP4 operand in the FP4-KM packing: (blob [R*K/2 + R*K/32] u8, codes [R, K], ebytes
    [R, K/32])."""
    codes = g.integers(0, 16, size=(R, K), dtype=np.uint8)
    ebytes = g.integers(123, 130, size=(R, K // 32), dtype=np.uint8)
    blob = np.concatenate([fp4km_pack(codes).reshape(-1), ebytes.reshape(-1)])
    return blob, codes, ebytes


def mx_decode(codes: np.ndarray, ebytes: np.ndarray) -> np.ndarray:
    """Exact fp32 values of an MXFP4 operand: E2M1[code] * 2^(e - 127)."""
    R, K = codes.shape
    scale = np.ldexp(np.float32(1.0), ebytes.astype(np.int32) - 127).astype(np.float32)
    return (E2M1[codes] * np.repeat(scale, 32, axis=1)).astype(np.float32).reshape(R, K)


def mx_table() -> np.ndarray:
    """The 272-float FP4-KM decode table of an MXFP4 operand: E2M1, then 2^(e-127) for e = 0..255."""
    t = np.zeros(272, dtype=np.float32)
    t[:16] = E2M1
    with np.errstate(over="ignore"):
        t[16:] = np.ldexp(np.float32(1.0), np.arange(256) - 127).astype(np.float32)
    return t
