"""The oracle's target-verification quantized linear and binary16 conversions (CPU), pinned by
numpy's float16 rounding, the reference QMV's byte masks for the 4/5-bit code order and a
float64 brute force on the reference's test geometries; the host-side checks of the C ABI and
of the Python mirror (no GPU call)."""
import ctypes as C

import numpy as np
import pytest
import torch

from astronomical_amd import _lib, ops
from astronomical_amd.layout import AffineWeights, bf16_to_f32, pack_codes
from verify_util import (FALLBACK, FALLBACK_F32, SUPPORTED, float64_projection, reference_inputs, to_dtype,
                         ulps)


# ------------------------------------------------------------------ binary16 conversions

def test_f32_to_f16_matches_numpy(orc):
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 4000),
        np.float32([0.0, -0.0, 65504.0, 65519.996, 65520.0, 1e9, -1e9, np.inf, -np.inf,
                    2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 3 * 2.0 ** -26, 2.0 ** -14,
                    2.0 ** -14 * (1 - 2.0 ** -11), 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 1e-30]),
        # exact ties between adjacent binary16 values, normal and subnormal
        (np.arange(1, 2048, dtype=np.float32) + 0.5) * np.float32(2.0 ** -24),
        (np.arange(1024, 2048, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    got = np.array([orc.f32_to_f16_scalar(v) for v in vals], np.uint16)
    assert np.array_equal(got, want)


def test_f16_to_f32_is_exact_for_every_pattern(orc):
    h = np.arange(0, 65536, 7, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32_scalar(int(v)) for v in h], np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(want))


# ------------------------------------------------------------------ code order

def _ref_mask_codes_4bit(words: np.ndarray) -> np.ndarray:
    """The reference QMV's 4-bit reading (target_verification_quantized_linear.rs:63-70): per
    16-bit half ws, x0 * (ws & 0x000f) + (x1 / 16) * (ws & 0x00f0) + (x2 / 256) * (ws & 0x0f00)
    + (x3 / 4096) * (ws & 0xf000), i.e. codes (ws & 0xf), (ws & 0xf0) / 16, ..."""
    ws = words.view(np.uint16)
    out = []
    for h in ws:
        h = int(h)
        out += [h & 0x000F, (h & 0x00F0) / 16, (h & 0x0F00) / 256, (h & 0xF000) / 4096]
    return np.array(out)


def _ref_mask_codes_5bit(words: np.ndarray) -> np.ndarray:
    """The reference QMV's 5-bit reading (:71-86): 8 codes per 5 bytes, each term a byte mask
    times the activation pre-scaled by the position's power of two (:37-45)."""
    b = words.view(np.uint8).astype(np.float64)
    out = []
    for i in range(0, b.size, 5):
        w0, w1, w2, w3, w4 = (int(v) for v in b[i:i + 5])
        out += [w0 & 0x1F,
                (w0 & 0xE0) / 32 + (w1 & 0x3) * 256 / 32,
                (w1 & 0x7C) / 4,
                (w1 & 0x80) / 128 + (w2 & 0xF) * 256 / 128,
                (w2 & 0xF0) / 16 + (w3 & 0x1) * 256 / 16,
                (w3 & 0x3E) / 2,
                (w3 & 0xC0) / 64 + (w4 & 0x7) * 256 / 64,
                (w4 & 0xF8) / 8]
    return np.array(out)


@pytest.mark.parametrize("bits,ref", [(4, _ref_mask_codes_4bit), (5, _ref_mask_codes_5bit)])
def test_code_order_matches_the_reference_masks(orc, bits, ref):
    rng = np.random.default_rng(bits)
    K = 256
    words = rng.integers(0, 2 ** 32, size=(1, 1, K * bits // 32), dtype=np.uint64).astype(np.uint32)
    ones = np.full((1, 1, K // 32), 0x3F80, np.uint16)  # scale 1.0
    zeros = np.zeros((1, 1, K // 32), np.uint16)
    codes = bf16_to_f32(orc.dequantize(AffineWeights(words, ones, zeros, bits, 32)))[0]
    assert np.array_equal(codes, ref(words.reshape(-1)))


# ------------------------------------------------------------------ values

@pytest.mark.parametrize("geo", SUPPORTED + FALLBACK[:3], ids=lambda g: f"T{g.tokens}K{g.input_dimension}"
                         f"N{g.output_dimension}{'f16' if g.f16 else 'bf16'}b{g.bits}g{g.group_size}")
def test_verification_linear_matches_float64(orc, geo):
    x, w = reference_inputs(geo, batch=2)
    y = orc.verification_quantized_linear(x, w, f16=geo.f16)
    want = to_dtype(float64_projection(x, w, geo.f16), geo.f16)
    u = ulps(y, want)
    assert y.shape == (2, geo.tokens, geo.output_dimension)
    assert u.max() <= 1 and np.mean(u == 0) >= 0.9, (u.max(), np.mean(u == 0))


def test_verification_linear_random_codes_match_float64(orc):
    from verify_util import random_inputs
    rng = np.random.default_rng(7)
    for bits, f16 in ((4, False), (5, True), (8, False), (8, True)):
        x, w = random_inputs(rng, 2, 3, 512, 40, bits, 64, f16)
        y = orc.verification_quantized_linear(x, w, f16=f16)
        u = ulps(y, to_dtype(float64_projection(x, w, f16), f16))
        assert u.max() <= 2 and np.mean(u == 0) >= 0.8, (bits, f16, u.max())


def test_verification_linear_is_row_local(orc):
    x, w = reference_inputs(SUPPORTED[1], batch=1)
    whole = orc.verification_quantized_linear(x, w, f16=True)
    for t in range(x.shape[1]):
        assert np.array_equal(whole[0, t], orc.verification_quantized_linear(x[:, t:t + 1], w, f16=True)[0, 0])


def test_oracle_rejects_invalid_geometry(orc):
    x, w = reference_inputs(SUPPORTED[0])
    for bad in (AffineWeights(w.w, w.scales, w.biases, 7, 32), AffineWeights(w.w, w.scales, w.biases, 4, 16),
                AffineWeights(np.concatenate([w.w, w.w]), np.concatenate([w.scales, w.scales]),
                              np.concatenate([w.biases, w.biases]), 4, 32)):
        with pytest.raises(RuntimeError):
            orc.verification_quantized_linear(x, bad)


# ------------------------------------------------------------------ host-side checks (no GPU call)

def _affine(N, K, bits, group, experts=1):
    return _lib.Affine(16, 16, 16, experts, N, K, bits, group)  # non-null, never dereferenced


@pytest.mark.parametrize("args,status,message", [
    ((0, 2, 512, (8, 512, 4, 32)), _lib.INVALID_ARGUMENT, "positive rank-three activations"),
    ((1, 2, 512, (0, 512, 4, 32)), _lib.INVALID_ARGUMENT, "positive rank-three activations"),
    ((1, 2, 512, (8, 512, 4, 16)), _lib.INVALID_ARGUMENT, "affine metadata is not supported by MLX"),
    ((1, 2, 512, (8, 512, 7, 32)), _lib.INVALID_ARGUMENT, "affine metadata is not supported by MLX"),
    ((1, 2, 256, (8, 512, 4, 32)), _lib.INVALID_ARGUMENT, "do not match activation and weight geometry"),
    ((1, 2, 96, (8, 96, 4, 64)), _lib.INVALID_ARGUMENT, "do not match activation and weight geometry"),
    ((1, 2, 512, (8, 512, 6, 32)), _lib.UNSUPPORTED, "4-, 5- or 8-bit codes"),
    ((1, 2, 192, (8, 192, 4, 64)), _lib.UNSUPPORTED, "multiple of 128"),
])
def test_abi_rejects_like_the_reference(args, status, message):
    lib = _lib.lib()
    b, t, k, (n, kw, bits, g) = args
    w = _affine(n, kw, bits, g)
    rc = lib.astro_moe_verification_quantized_linear(C.c_void_p(16), b, t, k, C.byref(w), 8, C.c_void_p(16), None)
    assert rc == status
    msg = lib.astro_moe_last_error().decode()
    assert msg.startswith("project Qwen3.5 target-verification tokens") and message in msg, msg


def test_abi_rejects_float32_activations():
    lib = _lib.lib()
    w = _affine(8, 512, 4, 32)
    rc = lib.astro_moe_verification_quantized_linear(C.c_void_p(16), 1, 3, 512, C.byref(w),
                                                     _lib.DTYPES.index("F32"), C.c_void_p(16), None)
    assert rc == _lib.UNSUPPORTED and "bfloat16 or float16" in lib.astro_moe_last_error().decode()


def test_dispatch_classification_follows_the_reference():
    """target_verification_uses_optimized_dispatch (:332-356) on the reference's two geometry lists."""
    for g in SUPPORTED:
        dt = torch.float16 if g.f16 else torch.bfloat16
        assert ops.target_verification_uses_optimized_dispatch(dt, dt, dt, g.group_size, g.bits,
                                                               g.input_dimension, g.output_dimension)
    for g in FALLBACK:
        dt = torch.float16 if g.f16 else torch.bfloat16
        assert not ops.target_verification_uses_optimized_dispatch(dt, dt, dt, g.group_size, g.bits,
                                                                   g.input_dimension, g.output_dimension)
    g = FALLBACK_F32
    assert not ops.target_verification_uses_optimized_dispatch(torch.float32, torch.float32, torch.float32,
                                                               g.group_size, g.bits, g.input_dimension,
                                                               g.output_dimension)


def test_python_mirror_checks_geometry_before_any_device_call():
    x = torch.zeros(1, 2, 512, dtype=torch.bfloat16)
    w = torch.zeros(8, 64, dtype=torch.int32)
    s = torch.zeros(8, 16, dtype=torch.bfloat16)
    with pytest.raises(ops.AstroMoeError, match="positive rank-three"):
        ops.qwen3_5_target_verification_quantized_linear(x[0], w, s, s, 32, 4)
    with pytest.raises(ops.AstroMoeError, match="not supported by MLX"):
        ops.qwen3_5_target_verification_quantized_linear(x, w, s, s, 32, 7)
    with pytest.raises(ops.AstroMoeError, match="do not match"):
        ops.qwen3_5_target_verification_quantized_linear(x, w, s[:, :8], s, 32, 4)
    with pytest.raises(ops.AstroMoeError, match="bfloat16 or float16"):
        ops.qwen3_5_target_verification_quantized_linear(x.float(), w, s.float(), s.float(), 32, 4)
