"""Synthetic safetensors checkpoints for the expert-page loader tests, written by the
`safetensors` package (an independent writer of the format the loader parses)."""
import json
import os

import numpy as np
import torch
from safetensors.torch import save_file

from astronomical_amd.layout import AffineWeights

PREFIX = "language_model.model.layers.{}.mlp"


def _t(a: np.ndarray) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32)).view(torch.uint32)
    if a.dtype == np.uint16:  # bf16 bit patterns
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)
    return torch.from_numpy(a)


def projection_tensors(prefix: str, proj: str, w: AffineWeights) -> dict:
    base = f"{prefix}.switch_mlp.{proj}"
    return {f"{base}.weight": _t(w.w), f"{base}.scales": _t(w.scales), f"{base}.biases": _t(w.biases)}


def write_checkpoint(root: str, layers: dict, extra: dict = None) -> dict:
    """layers: {layer index: (gate, up, down) AffineWeights (numpy)}.  Gate projections go to
    shard 1, up and down to shard 2 (a projection family split across shards); writes
    model.safetensors.index.json and returns the weight map."""
    os.makedirs(root, exist_ok=True)
    s1, s2 = {}, {}
    for li, (gate, up, down) in layers.items():
        p = PREFIX.format(li)
        s1.update(projection_tensors(p, "gate_proj", gate))
        s2.update(projection_tensors(p, "up_proj", up))
        s2.update(projection_tensors(p, "down_proj", down))
    s2.update(extra or {})
    names = {"model-00001-of-00002.safetensors": s1, "model-00002-of-00002.safetensors": s2}
    weight_map = {}
    for fname, tensors in names.items():
        save_file(tensors, os.path.join(root, fname), metadata={"format": "mlx"})
        weight_map.update({k: fname for k in tensors})
    with open(os.path.join(root, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": weight_map}, f)
    return weight_map


def header_entries(path: str) -> dict:
    """tensor -> (dtype, shape, file-relative start, end), parsed here with json."""
    with open(path, "rb") as f:
        n = int.from_bytes(f.read(8), "little")
        h = json.loads(f.read(n))
    return {k: (v["dtype"], v["shape"], 8 + n + v["data_offsets"][0], 8 + n + v["data_offsets"][1])
            for k, v in h.items() if k != "__metadata__"}


def raw_file(path: str, header: bytes, payload: bytes = b"", length: int = None) -> str:
    """A hand-made safetensors file: little-endian length (default len(header)), header, payload."""
    with open(path, "wb") as f:
        f.write((len(header) if length is None else length).to_bytes(8, "little"))
        f.write(header)
        f.write(payload)
    return path
