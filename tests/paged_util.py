"""Compact expert pages built from a resident synthetic layer (test helper).

A page holds the routed arrays of a chosen list of global experts in slot order, with gate and
up as separate pages (paged_execution.rs:232-245), and the map global id -> slot
(page_slot_by_global_expert_id, quantized_expert_manifest.rs:212-220; 0xffffffff = absent).
"""
import dataclasses

import numpy as np

from astronomical_amd.layout import AffineWeights

SLOT_ABSENT = 0xFFFFFFFF


def _take(w: AffineWeights, experts, rows=None) -> AffineWeights:
    e = np.asarray(experts, dtype=np.int64)
    sl = slice(None) if rows is None else rows
    return AffineWeights(np.ascontiguousarray(w.w[e][:, sl]), np.ascontiguousarray(w.scales[e][:, sl]),
                         np.ascontiguousarray(w.biases[e][:, sl]), w.bits, w.group_size)


def page_arrays(L, experts):
    """(gate, up, down) of the page holding `experts` in slot order (numpy AffineWeights)."""
    I = L.intermediate
    if L.gate_up is not None:
        gate = _take(L.gate_up, experts, slice(0, I))
        up = _take(L.gate_up, experts, slice(I, 2 * I))
    else:
        gate, up = _take(L.gate, experts), _take(L.up, experts)
    return gate, up, _take(L.down, experts)


def slot_map(num_experts, experts):
    m = np.full(num_experts, SLOT_ABSENT, dtype=np.uint32)
    m[np.asarray(experts, dtype=np.int64)] = np.arange(len(experts), dtype=np.uint32)
    return m


def paged_layer(L, experts):
    """The layer L with its routed arrays replaced by the page of `experts` (slot order)."""
    gate, up, down = page_arrays(L, experts)
    return dataclasses.replace(L, gate_up=None, gate=gate, up=up, down=down,
                               slot_of_expert=slot_map(L.num_experts, experts))
