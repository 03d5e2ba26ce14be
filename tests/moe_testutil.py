"""Shared helpers of the parity tests: bf16 comparison statistics and device plumbing."""
import numpy as np

from astronomical_amd.layout import bf16_to_f32

# Parity bar of the block's floating-point outputs (bf16 out, fp32 accumulation):
REL_L2_TOL = 1e-2        # relative L2 error
MEDIAN_ULP_TOL = 2.0     # median distance in bf16 ulps


def bf16_ordinal(h: np.ndarray) -> np.ndarray:
    """Monotone integer image of bf16 bit patterns (adjacent values differ by 1)."""
    h = np.asarray(h, dtype=np.uint16).astype(np.int32)
    return np.where(h & 0x8000, -(h & 0x7FFF), h)


def ulp_distance(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    return np.abs(bf16_ordinal(a) - bf16_ordinal(b))


def rel_l2(a: np.ndarray, b: np.ndarray) -> float:
    af = bf16_to_f32(a).astype(np.float64)
    bf = bf16_to_f32(b).astype(np.float64)
    return float(np.linalg.norm(af - bf) / max(np.linalg.norm(bf), 1e-30))


def assert_bf16_close(got: np.ndarray, want: np.ndarray, what: str = "",
                      rel_tol: float = REL_L2_TOL, median_ulp: float = MEDIAN_ULP_TOL) -> dict:
    got = np.asarray(got, np.uint16)
    want = np.asarray(want, np.uint16)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    if got.size == 0:
        return {}
    r = rel_l2(got, want)
    u = ulp_distance(got, want)
    stats = dict(rel_l2=r, median_ulp=float(np.median(u)), max_ulp=int(u.max()),
                 exact=float(np.mean(u == 0)))
    assert r <= rel_tol and stats["median_ulp"] <= median_ulp, (what, stats)
    return stats
