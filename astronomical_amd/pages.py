"""Expert pages from safetensors checkpoints: the host API of the reference's expert paging,
over the C ABI (every check, manifest and read runs in libastro_moe.so).

Reference names kept (crates/model-serving/src/lib.rs:279-301 re-exports the first four):
  build_quantized_expert_layer_plan          quantized_expert_layer_plan.rs:29-214
  build_quantized_expert_page_manifest_from_plan  quantized_expert_manifest.rs:401-418
  contiguous_selected_runs                   source_manifests.rs:77-99
  load_quantized_expert_page                 bounded_expert_reader.rs:35-61
  load_resident_expert_layer                 resident_expert_loading.rs:141-155 with the gate/up
                                             fusion of resident_gate_up_fusion.rs:109-268
A loaded page is a set of AffineWeights in the block's layout: torch device tensors (bf16 as
torch.bfloat16, u32 codes as torch.int32) or, with device=None, numpy host arrays.
"""
from __future__ import annotations

import ctypes as C
import json
import os
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple, Union

import numpy as np

from . import _lib
from .layout import AffineWeights

PROJECTIONS = ("gate_proj", "up_proj", "down_proj")
PARAMETERS = ("weight", "scales", "biases")
SLOT_ABSENT = 0xFFFFFFFF

_NP = {"U32": np.uint32, "BF16": np.uint16, "F16": np.float16, "F32": np.float32}


def _check(rc: int) -> None:
    if rc != _lib.OK:
        raise _lib.AstroMoeError(rc, _lib.lib().astro_moe_last_error().decode())


def read_weight_map(model_dir: str) -> Dict[str, str]:
    """tensor name -> shard file, from model.safetensors.index.json (a single-file checkpoint
    without an index maps every tensor of model.safetensors)."""
    idx = os.path.join(model_dir, "model.safetensors.index.json")
    if os.path.exists(idx):
        with open(idx) as f:
            return dict(json.load(f)["weight_map"])
    single = os.path.join(model_dir, "model.safetensors")
    with open(single, "rb") as f:
        n = int.from_bytes(f.read(8), "little")
        header = json.loads(f.read(n))
    return {k: "model.safetensors" for k in header if k != "__metadata__"}


def safetensors_tensor(path: str, tensor_name: str) -> dict:
    """One tensor's header entry after the reference's header checks (file-relative offset)."""
    dt, rank = C.c_int32(), C.c_int32()
    shape = (C.c_int64 * 8)()
    off, nbytes = C.c_uint64(), C.c_uint64()
    _check(_lib.lib().astro_moe_safetensors_tensor(path.encode(), tensor_name.encode(), C.byref(dt),
                                                   C.byref(rank), shape, C.byref(off), C.byref(nbytes)))
    return {"dtype": _lib.DTYPES[dt.value], "shape": list(shape[: rank.value]),
            "data_start_offset": off.value, "data_end_offset": off.value + nbytes.value}


@dataclass
class QuantizedTensorSource:
    """quantized_expert_manifest.rs:300-315."""
    tensor_name: str
    projection_name: str
    parameter_name: str
    quantization_bits: int
    quantization_group_size: int
    source_file: str
    source_file_size_bytes: int
    dtype: str
    full_shape: List[int]
    tensor_payload_offset: int
    bytes_per_expert: int
    expert_capacity: int


class QuantizedExpertLayerPlan:
    """Startup-validated geometry of one layer's nine expert tensors (quantized_expert_manifest.rs:317-398)."""

    def __init__(self, layer_prefix: str, c_plan: "_lib.ExpertLayerPlan"):
        self.layer_prefix = layer_prefix
        self._c = c_plan
        self.expert_capacity = int(c_plan.expert_capacity)
        self.gate_up_fusable = bool(c_plan.gate_up_fusable)
        self.gate_up_incompatibility_reason = c_plan.gate_up_separate_reason.decode() or None
        self.tensor_sources: List[QuantizedTensorSource] = []
        for p, proj in enumerate(PROJECTIONS):
            for q, param in enumerate(PARAMETERS):
                s = c_plan.src[p][q]
                self.tensor_sources.append(QuantizedTensorSource(
                    f"{layer_prefix}.switch_mlp.{proj}.{param}", proj, param, int(c_plan.bits[p]),
                    int(c_plan.group_size[p]), s.source_file.decode(), int(s.file_size),
                    _lib.DTYPES[s.dtype], [int(d) for d in s.shape], int(s.file_offset),
                    int(s.bytes_per_expert), int(s.shape[0])))

    def source(self, projection: str, parameter: str) -> QuantizedTensorSource:
        return self.tensor_sources[PROJECTIONS.index(projection) * 3 + PARAMETERS.index(parameter)]

    def expert_payload_byte_count(self) -> int:
        return sum(s.bytes_per_expert for s in self.tensor_sources)

    def complete_expert_payload_byte_count(self) -> int:
        return self.expert_payload_byte_count() * self.expert_capacity


def _per_projection(v: Union[int, Sequence[int], Dict[str, int]]) -> List[int]:
    if isinstance(v, dict):
        return [int(v[p]) for p in PROJECTIONS]
    if isinstance(v, (list, tuple)):
        return [int(x) for x in v]
    return [int(v)] * 3


def build_quantized_expert_layer_plan(model_dir: str, weight_map: Dict[str, str], layer_prefix: str,
                                      bits: Union[int, Sequence[int], Dict[str, int]] = 4,
                                      group_size: Union[int, Sequence[int], Dict[str, int]] = 64
                                      ) -> QuantizedExpertLayerPlan:
    """bits / group_size: the quantization profile, one value or one per projection."""
    names = list(weight_map)
    n = len(names)
    arr_names = (C.c_char_p * max(n, 1))(*[k.encode() for k in names])
    arr_files = (C.c_char_p * max(n, 1))(*[weight_map[k].encode() for k in names])
    b = (C.c_int32 * 3)(*_per_projection(bits))
    g = (C.c_int32 * 3)(*_per_projection(group_size))
    plan = _lib.ExpertLayerPlan()
    _check(_lib.lib().astro_moe_build_expert_layer_plan(model_dir.encode(), arr_names, arr_files, n,
                                                        layer_prefix.encode(), b, g, C.byref(plan)))
    return QuantizedExpertLayerPlan(layer_prefix, plan)


@dataclass
class QuantizedExpertSourceInterval:
    """source_manifests.rs:46-58; virtual_payload_offset is relative to the tensor's compact page."""
    tensor_name: str
    expert_start: int
    expert_count: int
    first_page_slot: int
    source_file_offset: int
    source_byte_count: int
    virtual_payload_offset: int


@dataclass
class QuantizedExpertPageManifest:
    """quantized_expert_manifest.rs:192-200."""
    expert_ids: List[int]
    page_slot_by_global_expert_id: np.ndarray  # uint32 [capacity]
    source_intervals: List[QuantizedExpertSourceInterval]
    payload_byte_count: int

    def contains_every_expert(self, selected_expert_ids: Sequence[int]) -> bool:
        s = self.page_slot_by_global_expert_id
        return all(0 <= e < len(s) and s[e] != SLOT_ABSENT for e in selected_expert_ids)

    def missing_expert_ids(self, selected_expert_ids: Sequence[int]) -> List[int]:
        s = self.page_slot_by_global_expert_id
        return [e for e in selected_expert_ids if not (0 <= e < len(s)) or s[e] == SLOT_ABSENT]


def _manifest(c_plan, layer_prefix: str, expert_ids: Sequence[int]) -> QuantizedExpertPageManifest:
    ids = np.ascontiguousarray(np.asarray(expert_ids, dtype=np.int64))
    if ids.size and (ids.min() < -(1 << 31) or ids.max() >= (1 << 31)):
        raise _lib.AstroMoeError(_lib.INVALID_ARGUMENT, "expert IDs exceed the int32 range")
    ids32 = ids.astype(np.int32)
    n = int(ids32.size)
    cap = max(int(c_plan.expert_capacity), 1)
    slots = np.empty(cap, dtype=np.uint32)
    ivs = (_lib.PageInterval * max(9 * n, 1))()
    niv, payload = C.c_int32(), C.c_uint64()
    _check(_lib.lib().astro_moe_build_expert_page_manifest(
        C.byref(c_plan), ids32.ctypes.data_as(C.POINTER(C.c_int32)), n, slots.ctypes.data, ivs,
        max(9 * n, 1), C.byref(niv), C.byref(payload)))
    intervals = [QuantizedExpertSourceInterval(
        f"{layer_prefix}.switch_mlp.{PROJECTIONS[iv.projection]}.{PARAMETERS[iv.parameter]}",
        iv.expert_start, iv.expert_count, iv.first_page_slot, iv.file_offset, iv.byte_count,
        iv.virtual_offset) for iv in ivs[: niv.value]]
    return QuantizedExpertPageManifest([int(x) for x in ids32], slots, intervals, int(payload.value))


def build_quantized_expert_page_manifest_from_plan(plan: QuantizedExpertLayerPlan,
                                                   expert_ids: Sequence[int]) -> QuantizedExpertPageManifest:
    return _manifest(plan._c, plan.layer_prefix, expert_ids)


def contiguous_selected_runs(expert_ids: Sequence[int]) -> List[Tuple[int, int, int]]:
    """(first expert, run length, first page slot) of each run of consecutive ids, from the
    library's manifest of a one-byte-per-expert stand-in plan (no file is touched)."""
    ids = [int(e) for e in expert_ids]
    if not ids:
        return []
    c_plan = _lib.ExpertLayerPlan()
    c_plan.expert_capacity = max(max(ids) + 1, 1)
    for p in range(3):
        for q in range(3):
            c_plan.src[p][q].bytes_per_expert = 1
    m = _manifest(c_plan, "", ids)
    first = [iv for iv in m.source_intervals if iv.tensor_name.endswith("gate_proj.weight")]
    return [(iv.expert_start, iv.expert_count, iv.first_page_slot) for iv in first]


@dataclass
class QuantizedExpertPage:
    """A loaded page in the block's layout: gate_up (fused) or gate and up, and down, each
    [n, out, inner] in page-slot order; slot_of_expert maps global ids to slots."""
    expert_ids: List[int]
    gate_up: Optional[AffineWeights]
    gate: Optional[AffineWeights]
    up: Optional[AffineWeights]
    down: AffineWeights
    slot_of_expert: np.ndarray
    bytes_read: int


def _alloc(shape, dtype_name: str, device):
    if device is None:
        return np.empty(shape, dtype=_NP[dtype_name])
    import torch
    tdt = {"U32": torch.int32, "BF16": torch.bfloat16, "F16": torch.float16, "F32": torch.float32}[dtype_name]
    return torch.empty(shape, dtype=tdt, device=device)


def _addr(a) -> int:
    return a.ctypes.data if isinstance(a, np.ndarray) else a.data_ptr()


def load_quantized_expert_page(plan: QuantizedExpertLayerPlan, expert_ids: Sequence[int],
                               device: Optional[str] = "cuda", fuse_gate_up: bool = False,
                               staging=None) -> QuantizedExpertPage:
    """Reads exactly the selected experts' bytes of the nine tensors.  fuse_gate_up concatenates
    gate and up rows per expert, the resident layout.  staging: optional pinned host tensor
    (>= 1 MiB) reused across calls for device destinations."""
    m = build_quantized_expert_page_manifest_from_plan(plan, expert_ids)
    n = len(m.expert_ids)
    bufs = [[None] * 3 for _ in range(3)]
    for p, proj in enumerate(PROJECTIONS):
        for q, param in enumerate(PARAMETERS):
            s = plan.source(proj, param)
            if fuse_gate_up and p == 1:
                continue
            rows = s.full_shape[1] * (2 if fuse_gate_up and p == 0 else 1)
            bufs[p][q] = _alloc((n, rows, s.full_shape[2]), s.dtype, device)
    ptrs = (C.c_void_p * 9)(*[_addr(bufs[p][q]) if bufs[p][q] is not None else None
                              for p in range(3) for q in range(3)])
    stream = None
    if device is not None:
        import torch
        stream = torch.cuda.current_stream(torch.device(device)).cuda_stream
    st_ptr, st_bytes = (None, 0) if staging is None else (_addr(staging), staging.numel() * staging.element_size())
    nread = C.c_uint64()
    ids32 = np.ascontiguousarray(np.asarray(m.expert_ids, dtype=np.int32))
    _check(_lib.lib().astro_moe_load_expert_page(
        C.byref(plan._c), ids32.ctypes.data_as(C.POINTER(C.c_int32)), n, int(fuse_gate_up), ptrs,
        int(device is not None), st_ptr, st_bytes, stream, C.byref(nread)))

    def aff(p):
        return AffineWeights(bufs[p][0], bufs[p][1], bufs[p][2], int(plan._c.bits[p]),
                             int(plan._c.group_size[p]))
    if fuse_gate_up:
        return QuantizedExpertPage(m.expert_ids, aff(0), None, None, aff(2), m.page_slot_by_global_expert_id,
                                   int(nread.value))
    return QuantizedExpertPage(m.expert_ids, None, aff(0), aff(1), aff(2), m.page_slot_by_global_expert_id,
                               int(nread.value))


def load_resident_expert_layer(plan: QuantizedExpertLayerPlan, device: Optional[str] = "cuda",
                               staging=None) -> QuantizedExpertPage:
    """Every expert of the layer, gate and up fused when the plan allows it (otherwise kept
    separate, plan.gate_up_incompatibility_reason says why)."""
    return load_quantized_expert_page(plan, range(plan.expert_capacity), device,
                                      fuse_gate_up=plan.gate_up_fusable, staging=staging)
