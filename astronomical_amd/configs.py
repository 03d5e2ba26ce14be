"""Synthetic layer configurations of the benchmark and parity suite.

c0  small CPU-runnable layer (parity config): H1024 E32 k4 I256, no shared, 4-bit g64, T=16.
c1  Qwen3.6-35B-A3B-shaped decode: H2048 E256 k8 I512, shared Is512, 4-bit g64, B in {1,2,4,8}.
c2  c1 shapes, prefill of 2048 tokens (sorted path).
c3  c1 shapes, 4096 tokens with Zipf(s=1.1)-biased router logits (skewed load).
c4  Qwen3-30B-A3B-shaped 8-bit: H2048 E128 k8 I768, no shared, 8-bit g32, 48 stacked
    layers, decode B=1 and 512-token prefill.
"""
from __future__ import annotations

from dataclasses import dataclass, replace
from typing import Tuple


@dataclass(frozen=True)
class LayerConfig:
    name: str
    hidden: int
    experts: int
    top_k: int
    intermediate: int
    shared_intermediate: int
    bits: int
    group_size: int
    scale_range: Tuple[float, float]
    bias_noise: float
    seed: int
    normalize_top_k: bool = True
    zipf_s: float = 0.0
    zipf_scale: float = 0.0
    layers: int = 1

    def with_(self, **kw) -> "LayerConfig":
        return replace(self, **kw)

    @property
    def page_bytes(self) -> int:
        """Routed expert page: gate/up + down codes, scales and biases."""
        H, I, b, g = self.hidden, self.intermediate, self.bits, self.group_size
        per_elem = b / 8 + 4 / g
        return int(round(3 * H * I * per_elem))

    @property
    def shared_page_bytes(self) -> int:
        if not self.shared_intermediate:
            return 0
        H, I, b, g = self.hidden, self.shared_intermediate, self.bits, self.group_size
        return int(round(3 * H * I * (b / 8 + 4 / g)))

    def flops_per_token(self) -> int:
        H, E, k, I, Is = self.hidden, self.experts, self.top_k, self.intermediate, self.shared_intermediate
        f = 2 * k * (2 * I * H + H * I) + 2 * H * E
        if Is:
            f += 2 * (2 * Is * H + H * Is) + 2 * H
        return f


C0 = LayerConfig("c0", 1024, 32, 4, 256, 0, 4, 64, (0.002, 0.02), 1e-3, seed=0xC0)
C1 = LayerConfig("c1", 2048, 256, 8, 512, 512, 4, 64, (0.002, 0.02), 1e-3, seed=0xC1)
C2 = C1.with_(name="c2", seed=0xC2)
C3 = C1.with_(name="c3", seed=0xC3, zipf_s=1.1, zipf_scale=2.0)
C4 = LayerConfig("c4", 2048, 128, 8, 768, 0, 8, 32, (1e-4, 1e-3), 0.0, seed=0xC4, layers=48)

CONFIGS = {c.name: c for c in (C0, C1, C2, C3, C4)}

TOKENS = {"c0": (16,), "c1": (1, 2, 4, 8), "c2": (2048,), "c3": (4096,), "c4": (1, 512)}
