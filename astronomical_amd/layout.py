"""MLX affine expert layout and bf16 helpers (host side, numpy).

The block keeps the reference's packed expert arrays unchanged so resident and paged
pages stay drop-in (qwen3_5/artifacts/tensor_spec.rs:247-285,
qwen3_5_moe/artifacts/tensor_spec.rs:7-94):

* ``w``      uint32 ``[experts, out, in * bits / 32]`` — element ``j`` of a row occupies
  bits ``[j*bits, j*bits + bits)`` of the row's little-endian bit stream (LSB first;
  the QMV masks in target_verification_quantized_linear.rs:28-35,63-70 read nibble 0
  from ``& 0x000f``).
* ``scales`` / ``biases`` bf16 ``[experts, out, in / group]``; the dequantised value is
  ``scale * q + bias``.
* Fused gate/up (resident_gate_up_fusion.rs:221-260) concatenates gate rows then up
  rows on the output axis: ``[experts, 2*I, in*bits/32]``.

bf16 tensors are carried as ``uint16`` bit patterns on the host.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np

SUPPORTED_BITS = (2, 3, 4, 5, 6, 8)
SUPPORTED_GROUPS = (32, 64, 128)


def f32_to_bf16(x) -> np.ndarray:
    """Round float values to bf16 (round to nearest even), returned as uint16 bits."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    if nan.any():
        r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r.reshape(a.shape)


def bf16_to_f32(h) -> np.ndarray:
    a = np.ascontiguousarray(np.asarray(h, dtype=np.uint16))
    return (a.astype(np.uint32) << 16).view(np.float32).reshape(a.shape)


def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """Pack integer codes ``[..., K]`` into uint32 words ``[..., K*bits/32]`` (LSB first)."""
    codes = np.asarray(codes)
    K = codes.shape[-1]
    if (K * bits) % 32:
        raise ValueError("row length times bit width must be a multiple of 32")
    if 32 % bits == 0:
        per = 32 // bits
        c = codes.astype(np.uint32).reshape(*codes.shape[:-1], K // per, per)
        shifts = (np.arange(per, dtype=np.uint32) * bits).astype(np.uint32)
        return np.bitwise_or.reduce(c << shifts, axis=-1).astype(np.uint32)
    # generic bit stream (3, 5, 6 bits): 32 codes fill exactly `bits` words
    c = codes.astype(np.uint64).reshape(-1, K)
    words = np.zeros((c.shape[0], K * bits // 32), dtype=np.uint64)
    for j in range(K):
        bit = j * bits
        w, s = divmod(bit, 32)
        words[:, w] |= (c[:, j] << np.uint64(s)) & np.uint64(0xFFFFFFFF)
        if s + bits > 32:
            words[:, w + 1] |= c[:, j] >> np.uint64(32 - s)
    return words.astype(np.uint32).reshape(*codes.shape[:-1], K * bits // 32)


def unpack_codes(words: np.ndarray, bits: int, K: int) -> np.ndarray:
    words = np.asarray(words, dtype=np.uint32)
    if 32 % bits == 0:
        per = 32 // bits
        shifts = (np.arange(per, dtype=np.uint32) * bits).astype(np.uint32)
        c = (words[..., :, None] >> shifts) & np.uint32((1 << bits) - 1)
        return c.reshape(*words.shape[:-1], K)
    flat = words.reshape(-1, words.shape[-1]).astype(np.uint64)
    out = np.zeros((flat.shape[0], K), dtype=np.uint32)
    for j in range(K):
        bit = j * bits
        w, s = divmod(bit, 32)
        v = flat[:, w] >> np.uint64(s)
        if s + bits > 32:
            v |= flat[:, w + 1] << np.uint64(32 - s)
        out[:, j] = (v & np.uint64((1 << bits) - 1)).astype(np.uint32)
    return out.reshape(*words.shape[:-1], K)


@dataclass
class AffineWeights:
    """One stacked affine projection in MLX layout (numpy or torch arrays)."""

    w: object
    scales: object
    biases: object
    bits: int
    group_size: int

    @property
    def experts(self) -> int:
        return int(self.w.shape[0])

    @property
    def out_features(self) -> int:
        return int(self.w.shape[1])

    @property
    def in_features(self) -> int:
        return int(self.w.shape[2]) * 32 // self.bits

    def map(self, fn) -> "AffineWeights":
        return AffineWeights(fn(self.w), fn(self.scales), fn(self.biases), self.bits,
                             self.group_size)

    @property
    def nbytes(self) -> int:
        def nb(a):
            return int(a.numel() * a.element_size()) if hasattr(a, "numel") else int(a.nbytes)
        return nb(self.w) + nb(self.scales) + nb(self.biases)


@dataclass
class MoeLayerWeights:
    """All tensors of one Qwen3.5/3.6-MoE block (feed_forward_weights.rs:17-24)."""

    hidden: int
    num_experts: int
    top_k: int
    intermediate: int
    shared_intermediate: int
    normalize_top_k: bool
    router_w: Optional[object]            # bf16 [E, H] (unquantized router)
    gate_up: Optional[AffineWeights]      # fused [E, 2I, ...]
    down: AffineWeights                   # [E, H, ...]
    gate: Optional[AffineWeights] = None  # separate gate/up pages
    up: Optional[AffineWeights] = None
    router_q: Optional[AffineWeights] = None
    router_bias: Optional[object] = None  # harness-only logit bias, bf16 [E]
    shared_gate: Optional[AffineWeights] = None
    shared_up: Optional[AffineWeights] = None
    shared_down: Optional[AffineWeights] = None
    shared_expert_gate: Optional[AffineWeights] = None
    extras: dict = field(default_factory=dict)
    # compact paged pages: u32 [E] global expert id -> slot of the routed arrays, 0xffffffff
    # for experts the page does not hold (page_slot_by_global_expert_id,
    # quantized_expert_manifest.rs:212-220); None for resident arrays
    slot_of_expert: Optional[object] = None

    def map(self, fn) -> "MoeLayerWeights":
        def m(a):
            return None if a is None else (a.map(fn) if isinstance(a, AffineWeights) else fn(a))
        return MoeLayerWeights(
            self.hidden, self.num_experts, self.top_k, self.intermediate,
            self.shared_intermediate, self.normalize_top_k, m(self.router_w), m(self.gate_up),
            m(self.down), m(self.gate), m(self.up), m(self.router_q), m(self.router_bias),
            m(self.shared_gate), m(self.shared_up), m(self.shared_down),
            m(self.shared_expert_gate), dict(self.extras), m(self.slot_of_expert))

    def page_bytes(self) -> int:
        """Bytes of one routed expert's gate/up + down page (scales and biases included)."""
        gu = self.gate_up if self.gate_up is not None else None
        parts = [gu] if gu is not None else [self.gate, self.up]
        total = 0
        for p in parts + [self.down]:
            total += p.nbytes // p.experts
        return total

    def shared_page_bytes(self) -> int:
        if not self.shared_intermediate:
            return 0
        return sum(p.nbytes for p in (self.shared_gate, self.shared_up, self.shared_down))
