"""Inputs and float64 references of the target-verification QMV tests.

The geometries and the input recipes are the reference's own
(crates/model-serving/tests/direct_mlx/qwen3_5/target_verification_quantized_linear.rs:22-51,
:103-141 and projection_inputs at :176-222): activations ((i % 29) - 14) / 16 and weights
((i % 31) - 15) / 32, cast to the activation dtype and quantized per group.  The quantizer
here only produces valid affine inputs (min/max per group); it is not the arithmetic under test.
"""
from dataclasses import dataclass

import numpy as np

from astronomical_amd.layout import AffineWeights, bf16_to_f32, f32_to_bf16, pack_codes


@dataclass(frozen=True)
class Geometry:
    tokens: int
    input_dimension: int
    output_dimension: int
    f16: bool
    bits: int
    group_size: int


# target_verification_quantized_linear.rs:27-51 (the reference's optimized dispatch)
SUPPORTED = (Geometry(2, 512, 8, False, 4, 32), Geometry(3, 1024, 16, True, 5, 64),
             Geometry(4, 512, 24, False, 4, 128))
# :108-141 (the reference's token-local fallback): 6-bit codes, K = 256, N = 10, float32
FALLBACK = (Geometry(3, 512, 8, False, 6, 32), Geometry(3, 256, 8, True, 4, 64),
            Geometry(3, 512, 10, False, 5, 128))
FALLBACK_F32 = Geometry(3, 512, 8, False, 4, 32)  # float32 activations at :134-141


def to_dtype(a, f16: bool) -> np.ndarray:
    """float values -> bf16 or binary16 bit patterns (round to nearest even)."""
    a = np.asarray(a, np.float32)
    return a.astype(np.float16).view(np.uint16) if f16 else f32_to_bf16(a)


def from_dtype(h, f16: bool) -> np.ndarray:
    h = np.asarray(h, np.uint16)
    return h.view(np.float16).astype(np.float32) if f16 else bf16_to_f32(h)


def quantize(w: np.ndarray, bits: int, group: int, f16: bool) -> AffineWeights:
    """Per-group min/max affine quantization of w [N, K] -> one-expert AffineWeights."""
    N, K = w.shape
    g = w.reshape(N, K // group, group).astype(np.float64)
    lo, hi = g.min(-1), g.max(-1)
    levels = (1 << bits) - 1
    scale = np.where(hi > lo, (hi - lo) / levels, 1.0)
    s = to_dtype(scale, f16)
    b = to_dtype(lo, f16)
    sf = from_dtype(s, f16).astype(np.float64)[..., None]
    bf = from_dtype(b, f16).astype(np.float64)[..., None]
    q = np.clip(np.rint((g - bf) / sf), 0, levels).astype(np.uint32).reshape(N, K)
    return AffineWeights(pack_codes(q, bits)[None], s[None], b[None], bits, group)


def reference_inputs(geo: Geometry, batch: int = 1):
    """projection_inputs (target_verification_quantized_linear.rs:176-222)."""
    n_act = batch * geo.tokens * geo.input_dimension
    act = ((np.arange(n_act) % 29).astype(np.float32) - 14.0) / 16.0
    x = to_dtype(act, geo.f16).reshape(batch, geo.tokens, geo.input_dimension)
    n_w = geo.output_dimension * geo.input_dimension
    wv = ((np.arange(n_w) % 31).astype(np.float32) - 15.0) / 32.0
    wv = from_dtype(to_dtype(wv, geo.f16), geo.f16).reshape(geo.output_dimension, geo.input_dimension)
    return x, quantize(wv, geo.bits, geo.group_size, geo.f16)


def random_inputs(rng, batch: int, tokens: int, K: int, N: int, bits: int, group: int, f16: bool):
    """Seeded codes, scales ~ U[0.002, 0.02], biases ~ -2^(bits-1) * scale, x ~ N(0, 1)."""
    codes = rng.integers(0, 1 << bits, size=(N, K), dtype=np.uint32)
    scale = rng.uniform(0.002, 0.02, size=(N, K // group))
    bias = -(1 << (bits - 1)) * scale + rng.normal(0, 1e-3, size=scale.shape)
    w = AffineWeights(pack_codes(codes, bits)[None], to_dtype(scale, f16)[None], to_dtype(bias, f16)[None],
                      bits, group)
    x = to_dtype(rng.standard_normal((batch, tokens, K)), f16)
    return x, w


def unpack_row_codes(w: AffineWeights) -> np.ndarray:
    from astronomical_amd.layout import unpack_codes
    return unpack_codes(np.asarray(w.w)[0], w.bits, w.in_features)


def float64_projection(x, w: AffineWeights, f16: bool) -> np.ndarray:
    """sum_k x * (s q + b) in float64 from the stored codes, scales and biases."""
    q = unpack_row_codes(w).astype(np.float64)
    N, K = q.shape
    s = np.repeat(from_dtype(np.asarray(w.scales)[0], f16).astype(np.float64), w.group_size, axis=1)
    b = np.repeat(from_dtype(np.asarray(w.biases)[0], f16).astype(np.float64), w.group_size, axis=1)
    deq = s * q + b
    xf = from_dtype(x, f16).astype(np.float64).reshape(-1, K)
    return (xf @ deq.T).reshape(*np.shape(x)[:-1], N)


def ordinal(h: np.ndarray) -> np.ndarray:
    """Monotone integer image of bf16 or binary16 bit patterns (both sign-magnitude)."""
    h = np.asarray(h, dtype=np.uint16).astype(np.int32)
    return np.where(h & 0x8000, -(h & 0x7FFF), h)


def ulps(a, b) -> np.ndarray:
    return np.abs(ordinal(a) - ordinal(b))


def rel_l2(a, b, f16: bool) -> float:
    af = from_dtype(a, f16).astype(np.float64)
    bf = from_dtype(b, f16).astype(np.float64)
    return float(np.linalg.norm(af - bf) / max(np.linalg.norm(bf), 1e-30))
