"""Tolerances of the parity tests (the reference's and the benchmark's), stated once."""
import numpy as np

# t_fp4_tile_gemm.nim:53-67: max|diff| <= tol * max(1, max|ref|), tol 1e-4 (2e-3 for fp16 coop).
REF_TOL = 1e-4
REF_TOL_F16_COOP = 2e-3
# Benchmark parity tiers (max-abs-rel = max|diff| / max|ref|): fp32 accumulate 1e-3, fp16 paths 1e-2.
TIER_F32_ACC = 1e-3
TIER_F16 = 1e-2
# bf16 outputs against the oracle rounded to bf16: a sum that differs in its last fp32 bits can
# round to the neighbouring bf16, one unit in the last place (at most 2^-7 of the peak), on top of
# the fp32-accumulate tier.
TIER_BF16_OUT = 2.0 ** -7 + TIER_F32_ACC


def ref_check(got, want, tol=REF_TOL):
    got = np.asarray(got, dtype=np.float64).reshape(-1)
    want = np.asarray(want, dtype=np.float64).reshape(-1)
    assert got.shape == want.shape
    assert np.all(np.isfinite(got)), "non-finite output"
    worst = float(np.max(np.abs(got - want))) if want.size else 0.0
    peak = float(np.max(np.abs(want))) if want.size else 0.0
    assert worst <= tol * max(1.0, peak), f"max|diff|={worst:.3e} peak={peak:.3f} tol={tol}"
    return worst


def max_abs_rel(got, want) -> float:
    got = np.asarray(got, dtype=np.float64).reshape(-1)
    want = np.asarray(want, dtype=np.float64).reshape(-1)
    peak = float(np.max(np.abs(want)))
    return float(np.max(np.abs(got - want))) / (peak if peak > 0 else 1.0)


def tier_check(got, want, tier):
    assert np.all(np.isfinite(np.asarray(got, dtype=np.float64))), "non-finite output"
    r = max_abs_rel(got, want)
    assert r <= tier, f"max-abs-rel {r:.3e} > {tier}"
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_rne(f: np.ndarray) -> np.ndarray:
    """Round fp32 to bf16 (nearest even), returned as fp32 values."""
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32)
