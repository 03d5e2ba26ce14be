"""Pins the oracle's scalar arithmetic against closed forms (CPU only)."""
import numpy as np
import pytest

from astronomical_amd.layout import bf16_to_f32, f32_to_bf16


def _rne_bf16_reference(f: np.ndarray) -> np.ndarray:
    """Nearest bf16 by float64 distance, ties to the even pattern (independent of bit tricks)."""
    bits = f.view(np.uint32)
    lo = (bits >> 16).astype(np.uint32)
    lo_f = (lo << 16).view(np.float32).astype(np.float64)
    hi = lo + 1
    hi_f = (hi.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    x = f.astype(np.float64)
    dlo, dhi = np.abs(x - lo_f), np.abs(hi_f - x)
    pick_hi = (dhi < dlo) | ((dhi == dlo) & ((lo & 1) == 1))
    return np.where(pick_hi, hi, lo).astype(np.uint16)


def test_bf16_rounding_matches_nearest_even(orc):
    rng = np.random.default_rng(1)
    pats = rng.integers(0, 0x7F7F0000, size=4000, dtype=np.uint32)
    ties = (rng.integers(0, 0x7F7F, size=500, dtype=np.uint32) << 16) | 0x8000
    pats = np.concatenate([pats, ties, ties | 0x80000000, pats | 0x80000000]).astype(np.uint32)
    f = pats.view(np.float32)
    want = _rne_bf16_reference(f)
    got_np = f32_to_bf16(f)
    got_orc = np.array([orc.f32_to_bf16_scalar(v) for v in f[:3000]], dtype=np.uint16)
    assert np.array_equal(got_np, want)
    assert np.array_equal(got_orc, want[:3000])
    assert orc.f32_to_bf16_scalar(float("inf")) == 0x7F80
    assert bf16_to_f32(np.array([0x3F80], np.uint16))[0] == 1.0


def test_expf_within_two_ulp_of_float64(orc):
    xs = np.concatenate([np.linspace(-80.0, 88.72, 20000, dtype=np.float32),
                         np.linspace(-1.0, 1.0, 4001, dtype=np.float32)])
    got = np.array([orc.expf(float(v)) for v in xs], dtype=np.float32)
    ref = np.exp(xs.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    err = np.abs(got.astype(np.float64) - ref) / ulp
    assert err.max() <= 2.0, float(err.max())
    assert orc.expf(0.0) == 1.0
    assert orc.expf(-80.5) == 0.0
    assert orc.expf(89.0) == float("inf")
