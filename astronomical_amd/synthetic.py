"""Seeded synthetic inputs for the benchmark configurations (host side, numpy).

A counter-based generator, so any element can be produced independently (the HIP
generator ``astro_synth_*`` in the library produces the same streams on the device):

* stream key ``K = splitmix64(seed ^ fnv1a64(name))`` for a tensor name such as
  ``"L3/gate/w"``;
* element ``i`` draws ``h = splitmix64(K + i)``;
* packed code words are ``h & 0xffffffff`` (uniform codes for every bit width);
* uniforms are ``(h >> 11) * 2**-53``;
* normals use Box–Muller on the pair ``(splitmix64(K + 2i), splitmix64(K + 2i + 1))``
  with ``u1 = ((h1 >> 11) + 0.5) * 2**-53`` and ``u2 = (h2 >> 11) * 2**-53``, evaluated in
  float64 and rounded to bf16 once.

Distributions follow the configuration descriptions: codes uniform; scales uniform in
``scale_range`` (bf16); 4-bit biases ``bf16(-8*scale + N(0, bias_noise))``, 8-bit biases
``bf16(-128*scale)``; router ``bf16(N(0, 0.02))`` stored ``[E, H]``; activations
``N(0, 1)`` RMS-normalised per token (``x / sqrt(mean(x^2) + 1e-6)``) then bf16.
"""
from __future__ import annotations

import numpy as np

from .configs import LayerConfig
from .layout import AffineWeights, MoeLayerWeights, f32_to_bf16

M64 = (1 << 64) - 1


def fnv1a64(name: str) -> int:
    h = 0xCBF29CE484222325
    for b in name.encode():
        h ^= b
        h = (h * 0x100000001B3) & M64
    return h


def splitmix64(x: np.ndarray) -> np.ndarray:
    z = x + np.uint64(0x9E3779B97F4A7C15)
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def stream_key(seed: int, name: str) -> int:
    return int(splitmix64(np.array([(seed ^ fnv1a64(name)) & M64], dtype=np.uint64))[0])


def _hashes(key: int, start: int, count: int, step: int = 1) -> np.ndarray:
    i = np.arange(count, dtype=np.uint64) * np.uint64(step) + np.uint64(start)
    with np.errstate(over="ignore"):
        return splitmix64(i + np.uint64(key))


def code_words(seed: int, name: str, shape) -> np.ndarray:
    n = int(np.prod(shape))
    return (_hashes(stream_key(seed, name), 0, n) & np.uint64(0xFFFFFFFF)).astype(np.uint32).reshape(shape)


def uniform(seed: int, name: str, shape) -> np.ndarray:
    n = int(np.prod(shape))
    h = _hashes(stream_key(seed, name), 0, n)
    return ((h >> np.uint64(11)).astype(np.float64) * 2.0 ** -53).reshape(shape)


def normal(seed: int, name: str, shape) -> np.ndarray:
    n = int(np.prod(shape))
    key = stream_key(seed, name)
    h1 = _hashes(key, 0, n, 2)
    h2 = _hashes(key, 1, n, 2)
    u1 = ((h1 >> np.uint64(11)).astype(np.float64) + 0.5) * 2.0 ** -53
    u2 = (h2 >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    return (np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)).reshape(shape)


def activations(seed: int, name: str, tokens: int, hidden: int) -> np.ndarray:
    x = normal(seed, name, (tokens, hidden))
    x = x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + 1e-6)
    return f32_to_bf16(x.astype(np.float32))


def affine(cfg: LayerConfig, seed: int, name: str, experts: int, out: int, inp: int,
           bits: int | None = None, group: int | None = None) -> AffineWeights:
    bits = cfg.bits if bits is None else bits
    group = cfg.group_size if group is None else group
    words = code_words(seed, name + "/w", (experts, out, inp * bits // 32))
    lo, hi = cfg.scale_range
    scales = f32_to_bf16((lo + uniform(seed, name + "/s", (experts, out, inp // group)) * (hi - lo)).astype(np.float32))
    sf = (scales.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    center = float(1 << (bits - 1))
    b = -center * sf
    if cfg.bias_noise:
        b = b + cfg.bias_noise * normal(seed, name + "/b", sf.shape)
    biases = f32_to_bf16(b.astype(np.float32))
    return AffineWeights(words, scales, biases, bits, group)


def zipf_router_bias(cfg: LayerConfig, seed: int) -> np.ndarray:
    """b_e = scale * ln(r_e^-s / sum_j j^-s), r_e a seeded permutation of 1..E (bf16)."""
    E = cfg.experts
    order = np.argsort(uniform(seed, "zipf/perm", (E,)), kind="stable")
    rank = np.empty(E, dtype=np.int64)
    rank[order] = np.arange(1, E + 1)
    z = np.sum(np.arange(1, E + 1, dtype=np.float64) ** -cfg.zipf_s)
    b = cfg.zipf_scale * np.log(rank.astype(np.float64) ** -cfg.zipf_s / z)
    return f32_to_bf16(b.astype(np.float32))


def router_config(cfg: LayerConfig, bits: int) -> LayerConfig:
    """Distributions of an affine router (mlp.gate quantized, as the reference's certified
    Qwen3.5/3.6-MoE checkpoints have it): group 64, codes uniform, biases centred as for the
    experts; scales U[0.002, 0.02] at 4 bits and U[1e-4, 1e-3] at 8 bits, so the dequantised
    weights have a standard deviation of a few hundredths, like the bf16 router's N(0, 0.02)."""
    lo_hi = (0.002, 0.02) if bits == 4 else (1e-4, 1e-3)
    return cfg.with_(bits=bits, group_size=64, scale_range=lo_hi, bias_noise=1e-3 if bits == 4 else 0.0)


def make_layer(cfg: LayerConfig, layer: int = 0, fused_gate_up: bool = True,
               keep_separate: bool = False, router_bits: int | None = None) -> MoeLayerWeights:
    """Weights of one synthetic layer as numpy arrays (host).  router_bits (4 or 8): an affine
    router [1, E, H*bits/32] instead of the bf16 one."""
    s = cfg.seed
    p = f"L{layer}/"
    H, E, I, Is = cfg.hidden, cfg.experts, cfg.intermediate, cfg.shared_intermediate
    router = None
    if router_bits is None:
        router = f32_to_bf16((0.02 * normal(s, p + "router", (E, H))).astype(np.float32))
    gate = affine(cfg, s, p + "gate", E, I, H)
    up = affine(cfg, s, p + "up", E, I, H)
    down = affine(cfg, s, p + "down", E, H, I)
    gate_up = None
    if fused_gate_up:
        gate_up = AffineWeights(np.concatenate([gate.w, up.w], axis=1),
                                np.concatenate([gate.scales, up.scales], axis=1),
                                np.concatenate([gate.biases, up.biases], axis=1),
                                cfg.bits, cfg.group_size)
    L = MoeLayerWeights(H, E, cfg.top_k, I, Is, cfg.normalize_top_k, router, gate_up, down,
                        gate=gate if (keep_separate or not fused_gate_up) else None,
                        up=up if (keep_separate or not fused_gate_up) else None)
    if router_bits is not None:
        L.router_q = affine(router_config(cfg, router_bits), s, p + f"router_q{router_bits}", 1, E, H)
    if cfg.zipf_s:
        L.router_bias = zipf_router_bias(cfg, s)
    if Is:
        L.shared_gate = affine(cfg, s, p + "shared_gate", 1, Is, H)
        L.shared_up = affine(cfg, s, p + "shared_up", 1, Is, H)
        L.shared_down = affine(cfg, s, p + "shared_down", 1, H, Is)
        L.shared_expert_gate = affine(cfg, s, p + "shared_expert_gate", 1, 1, H)
    return L


def make_tokens(cfg: LayerConfig, tokens: int, step: int = 0) -> np.ndarray:
    return activations(cfg.seed, f"x/T{tokens}/step{step}", tokens, cfg.hidden)
