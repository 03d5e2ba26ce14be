"""Expert pages from safetensors (CPU): header checks, the layer plan, the page manifest and
bounded reads into host memory, against files written by the `safetensors` package.

Reference behaviour followed: safetensors_header.rs:171-429, quantized_expert_layer_plan.rs,
quantized_expert_validation.rs, source_manifests.rs, bounded_expert_reader.rs,
resident_gate_up_fusion.rs; manifest cases from
tests/direct_mlx/qwen3_5_moe/expert_paging/quantized_expert_manifest/contracts.rs:16-460."""
import json
import os

import numpy as np
import pytest
import torch

from astronomical_amd import configs as CF
from astronomical_amd import pages as P
from astronomical_amd import synthetic as S
from astronomical_amd._lib import AstroMoeError, INVALID_ARGUMENT
from astronomical_amd.layout import AffineWeights
from pages_util import PREFIX, header_entries, raw_file, write_checkpoint, _t

SLOT_ABSENT = 0xFFFFFFFF


def _layer(cfg=CF.C0, layer=0):
    L = S.make_layer(cfg, layer, keep_separate=True)
    return L, (L.gate, L.up, L.down)


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    root = str(tmp_path_factory.mktemp("ckpt"))
    L0, t0 = _layer(CF.C0, 0)
    L1, t1 = _layer(CF.C0, 1)
    wm = write_checkpoint(root, {0: t0, 1: t1})
    return root, wm, {0: L0, 1: L1}


def _err(fn, match):
    with pytest.raises(AstroMoeError, match=match) as ei:
        fn()
    return ei.value


# ------------------------------------------------------------------ headers

def test_header_entries_match_an_independent_parse(ckpt):
    root, wm, _ = ckpt
    for fname in sorted(set(wm.values())):
        path = os.path.join(root, fname)
        for name, (dt, shape, start, end) in header_entries(path).items():
            e = P.safetensors_tensor(path, name)
            assert (e["dtype"], e["shape"], e["data_start_offset"], e["data_end_offset"]) == (dt, shape, start, end)


def test_header_checks(tmp_path):
    d = str(tmp_path)
    _err(lambda: P.safetensors_tensor(os.path.join(d, "absent.safetensors"), "x"), "safetensors file does not exist")
    p = os.path.join(d, "tiny.safetensors")
    open(p, "wb").write(b"\x01\x02\x03\x04")
    _err(lambda: P.safetensors_tensor(p, "x"), "too small to contain a header length prefix: 4 bytes")
    p = raw_file(os.path.join(d, "huge.safetensors"), b"{}", length=(64 << 20) + 1)
    _err(lambda: P.safetensors_tensor(p, "x"), "exceeds the safety limit of 67108864 bytes")
    p = raw_file(os.path.join(d, "beyond.safetensors"), b"{}", length=100)
    _err(lambda: P.safetensors_tensor(p, "x"), "header extends beyond the file: header ends at 108 but file is 10 bytes")
    p = raw_file(os.path.join(d, "bad.safetensors"), b'{"a": ')
    _err(lambda: P.safetensors_tensor(p, "a"), "must contain valid JSON")
    dup = b'{"a":{"dtype":"U8","shape":[1],"data_offsets":[0,1]},"a":{"dtype":"U8","shape":[1],"data_offsets":[0,1]}}'
    p = raw_file(os.path.join(d, "dup.safetensors"), dup, b"\x00")
    _err(lambda: P.safetensors_tensor(p, "a"), "must contain valid JSON")
    p = raw_file(os.path.join(d, "notobj.safetensors"), b'{"a": 5}')
    _err(lambda: P.safetensors_tensor(p, "a"), "must be a JSON object, got 5")
    p = raw_file(os.path.join(d, "dtype.safetensors"), b'{"a":{"dtype":"F64","shape":[1],"data_offsets":[0,8]}}', bytes(8))
    _err(lambda: P.safetensors_tensor(p, "a"), 'unsupported dtype: "F64"')
    p = raw_file(os.path.join(d, "shape.safetensors"), b'{"a":{"dtype":"U8","shape":[-1],"data_offsets":[0,1]}}', b"\x00")
    _err(lambda: P.safetensors_tensor(p, "a"), "invalid shape")
    p = raw_file(os.path.join(d, "offs.safetensors"), b'{"a":{"dtype":"U8","shape":[1],"data_offsets":[1,0]}}', b"\x00")
    _err(lambda: P.safetensors_tensor(p, "a"), "invalid data_offsets")
    p = raw_file(os.path.join(d, "outside.safetensors"), b'{"a":{"dtype":"U8","shape":[4],"data_offsets":[0,4]}}', b"\x00")
    _err(lambda: P.safetensors_tensor(p, "a"), r"outside the file payload: \[0, 4\) vs payload size 1")
    p = raw_file(os.path.join(d, "count.safetensors"), b'{"a":{"dtype":"U32","shape":[2],"data_offsets":[0,4]}}', bytes(4))
    _err(lambda: P.safetensors_tensor(p, "a"), "byte count mismatch: header declares 4 bytes but shape.*dtype expects 8 bytes")
    # __metadata__ is not a tensor; a valid file parses
    p = raw_file(os.path.join(d, "ok.safetensors"),
                 b'{"__metadata__":{"format":"mlx"},"a":{"dtype":"BF16","shape":[2,1],"data_offsets":[0,4]}}', bytes(4))
    e = P.safetensors_tensor(p, "a")
    assert e["dtype"] == "BF16" and e["shape"] == [2, 1] and e["data_end_offset"] - e["data_start_offset"] == 4
    _err(lambda: P.safetensors_tensor(p, "__metadata__"), "is not in the safetensors header")


# ------------------------------------------------------------------ layer plan

def test_plan_from_two_shards(ckpt):
    root, wm, Ls = ckpt
    plan = P.build_quantized_expert_layer_plan(root, wm, PREFIX.format(1), 4, 64)
    L = Ls[1]
    assert plan.expert_capacity == CF.C0.experts
    assert plan.gate_up_fusable and plan.gate_up_incompatibility_reason is None
    for proj, w in zip(P.PROJECTIONS, (L.gate, L.up, L.down)):
        for param, a in zip(P.PARAMETERS, (w.w, w.scales, w.biases)):
            s = plan.source(proj, param)
            path = os.path.join(root, wm[s.tensor_name])
            dt, shape, start, end = header_entries(path)[s.tensor_name]
            assert (s.source_file, s.dtype, s.full_shape, s.tensor_payload_offset) == (path, dt, shape, start)
            assert s.bytes_per_expert * s.expert_capacity == end - start == a.nbytes
    # exact payload of a complete layer (quantized_expert_manifest.rs:329-398)
    total = sum(a.nbytes for w in (L.gate, L.up, L.down) for a in (w.w, w.scales, w.biases))
    assert plan.complete_expert_payload_byte_count() == total


def _write_one(tmp_path, gate, up, down, extra_map=None):
    root = str(tmp_path)
    wm = write_checkpoint(root, {0: (gate, up, down)})
    wm.update(extra_map or {})
    return root, wm


def test_plan_errors(tmp_path):
    L, (g, u, d) = _layer()
    pre = PREFIX.format(0)
    root, wm = _write_one(tmp_path / "a", g, u, d)
    bad = dict(wm)
    del bad[f"{pre}.switch_mlp.up_proj.scales"]
    _err(lambda: P.build_quantized_expert_layer_plan(root, bad, pre), "missing index entry for tensor .*up_proj.scales")
    bad = dict(wm)
    bad[f"{pre}.switch_mlp.up_proj.scales"] = "model-00001-of-00002.safetensors"
    _err(lambda: P.build_quantized_expert_layer_plan(root, bad, pre), 'missing ".*up_proj.scales" in shard header')
    # quantization contract (quantized_expert_validation.rs:37-62)
    _err(lambda: P.build_quantized_expert_layer_plan(root, wm, pre, 0, 64), "quantization bits must be a positive integer")
    _err(lambda: P.build_quantized_expert_layer_plan(root, wm, pre, 4, 0), "group_size must be a positive integer")
    _err(lambda: P.build_quantized_expert_layer_plan(root, wm, pre, 3, 16),
         "must pack into whole U32 elements: bits=3, group_size=16")
    # a profile that disagrees with the stored packing
    _err(lambda: P.build_quantized_expert_layer_plan(root, wm, pre, 8, 64),
         r'"gate_proj" has an invalid packed weight width: expected 256, got 128')
    # dtypes, rank, shapes
    as_i32 = AffineWeights(g.w.view(np.int32), g.scales, g.biases, 4, 64)
    root, wm = _write_one(tmp_path / "b", as_i32, u, d)
    _err(lambda: P.build_quantized_expert_layer_plan(root, wm, pre), "gate_proj.weight\" must use U32 but has I32")
    i32_scales = AffineWeights(g.w, g.scales.astype(np.int32), g.biases, 4, 64)
    root, wm = _write_one(tmp_path / "c", i32_scales, u, d)
    _err(lambda: P.build_quantized_expert_layer_plan(root, wm, pre), "must use float16, bfloat16, or float32 but has I32")
    rank2 = AffineWeights(g.w[0], g.scales[0], g.biases[0], 4, 64)
    root, wm = _write_one(tmp_path / "d", rank2, u, d)
    _err(lambda: P.build_quantized_expert_layer_plan(root, wm, pre), "must have a non-empty rank-three shape")
    mism = AffineWeights(g.w, g.scales, g.biases[:, :-1], 4, 64)
    root, wm = _write_one(tmp_path / "e", mism, u, d)
    _err(lambda: P.build_quantized_expert_layer_plan(root, wm, pre), '"gate_proj" scales and biases must share a shape')
    batch = AffineWeights(g.w[:, :-1], g.scales, g.biases, 4, 64)
    root, wm = _write_one(tmp_path / "f", batch, u, d)
    _err(lambda: P.build_quantized_expert_layer_plan(root, wm, pre), '"gate_proj" weight/scales batch dimensions differ')
    fewer = AffineWeights(d.w[:-1], d.scales[:-1], d.biases[:-1], 4, 64)
    root, wm = _write_one(tmp_path / "g", g, u, fewer)
    _err(lambda: P.build_quantized_expert_layer_plan(root, wm, pre), r"must share one expert capacity, found \[32, 31\]")


def test_gate_up_fusion_plan(tmp_path):
    """resident_gate_up_fusion.rs:119-163: fused only with equal shapes, dtypes and profile."""
    L, (g, u, d) = _layer()
    pre = PREFIX.format(0)
    u8 = S.affine(CF.C0.with_(bits=8), CF.C0.seed, "u8", CF.C0.experts, CF.C0.intermediate, CF.C0.hidden)
    root, wm = _write_one(tmp_path / "a", g, u8, d)
    plan = P.build_quantized_expert_layer_plan(root, wm, pre, (4, 8, 4), 64)
    assert not plan.gate_up_fusable and plan.gate_up_incompatibility_reason == "gate and up tensor shapes differ"
    _err(lambda: P.load_quantized_expert_page(plan, [0], device=None, fuse_gate_up=True),
         "gate and up cannot be fused: gate and up tensor shapes differ")
    page = P.load_resident_expert_layer(plan, device=None)  # kept separate
    assert page.gate_up is None and np.array_equal(page.up.w, u8.w)
    f16 = AffineWeights(u.w, u.scales.view(np.float16), u.biases.view(np.float16), 4, 64)
    root, wm = _write_one(tmp_path / "b", g, f16, d)
    plan = P.build_quantized_expert_layer_plan(root, wm, pre)
    assert plan.gate_up_incompatibility_reason == "gate and up tensor data types differ"


# ------------------------------------------------------------------ manifest

def _plan8(tmp_path):
    cfg = CF.C0.with_(experts=8)
    L = S.make_layer(cfg, keep_separate=True)
    root, wm = _write_one(tmp_path, L.gate, L.up, L.down)
    return P.build_quantized_expert_layer_plan(root, wm, PREFIX.format(0)), L


def test_manifest_contract_cases(tmp_path):
    plan, L = _plan8(tmp_path)
    m = P.build_quantized_expert_page_manifest_from_plan(plan, [0, 7])
    assert m.expert_ids == [0, 7] and len(m.page_slot_by_global_expert_id) == 8
    assert m.page_slot_by_global_expert_id[0] == 0 and m.page_slot_by_global_expert_id[7] == 1
    assert m.page_slot_by_global_expert_id[3] == SLOT_ABSENT
    assert m.contains_every_expert([0, 7]) and not m.contains_every_expert([0, 3])
    assert m.missing_expert_ids([3, 0, 5]) == [3, 5]
    m = P.build_quantized_expert_page_manifest_from_plan(plan, [3, 5, 7])
    assert list(m.page_slot_by_global_expert_id[[3, 5, 7]]) == [0, 1, 2]
    assert m.payload_byte_count == 3 * plan.expert_payload_byte_count()
    assert P.build_quantized_expert_page_manifest_from_plan(plan, [7]).expert_ids == [7]  # capacity boundary
    _err(lambda: P.build_quantized_expert_page_manifest_from_plan(plan, []), "must select at least one expert")
    _err(lambda: P.build_quantized_expert_page_manifest_from_plan(plan, [5, 3]), "unique and strictly ascending")
    _err(lambda: P.build_quantized_expert_page_manifest_from_plan(plan, [3, 3]), "unique and strictly ascending")
    _err(lambda: P.build_quantized_expert_page_manifest_from_plan(plan, [0, 8]),
         "exceed the quantized layer's expert capacity: max 8, got 8")
    _err(lambda: P.build_quantized_expert_page_manifest_from_plan(plan, [-1]), "must be non-negative integers")


def test_manifest_intervals(tmp_path):
    plan, L = _plan8(tmp_path)
    ids = [0, 1, 2, 5, 6]
    m = P.build_quantized_expert_page_manifest_from_plan(plan, ids)
    assert len(m.source_intervals) == 9 * 2
    for iv in m.source_intervals:
        s = next(t for t in plan.tensor_sources if t.tensor_name == iv.tensor_name)
        assert iv.source_file_offset == s.tensor_payload_offset + iv.expert_start * s.bytes_per_expert
        assert iv.source_byte_count == iv.expert_count * s.bytes_per_expert
        assert iv.virtual_payload_offset == iv.first_page_slot * s.bytes_per_expert
        assert ids[iv.first_page_slot] == iv.expert_start
    # per tensor: the intervals tile its compact payload without gaps (validate_virtual_intervals)
    for s in plan.tensor_sources:
        mine = sorted((iv for iv in m.source_intervals if iv.tensor_name == s.tensor_name),
                      key=lambda iv: iv.virtual_payload_offset)
        at = 0
        for iv in mine:
            assert iv.virtual_payload_offset == at
            at += iv.source_byte_count
        assert at == len(ids) * s.bytes_per_expert


def test_contiguous_selected_runs():
    assert P.contiguous_selected_runs([0, 1, 2, 5, 6, 9]) == [(0, 3, 0), (5, 2, 3), (9, 1, 5)]
    assert P.contiguous_selected_runs([4]) == [(4, 1, 0)]
    assert P.contiguous_selected_runs([]) == []
    assert P.contiguous_selected_runs(list(range(10))) == [(0, 10, 0)]


# ------------------------------------------------------------------ bounded reads

def _sel(a, ids):
    return np.ascontiguousarray(a[np.asarray(ids)])


def test_load_page_into_host_memory(ckpt):
    root, wm, Ls = ckpt
    L = Ls[1]
    plan = P.build_quantized_expert_layer_plan(root, wm, PREFIX.format(1))
    ids = [1, 2, 3, 10, 20, 31]
    page = P.load_quantized_expert_page(plan, ids, device=None)
    for got, ref in ((page.gate, L.gate), (page.up, L.up), (page.down, L.down)):
        for a, b in ((got.w, ref.w), (got.scales, ref.scales), (got.biases, ref.biases)):
            assert a.dtype == b.dtype and np.array_equal(a, _sel(b, ids))
    assert page.bytes_read == P.build_quantized_expert_page_manifest_from_plan(plan, ids).payload_byte_count
    assert list(page.slot_of_expert[ids]) == list(range(len(ids)))
    fused = P.load_quantized_expert_page(plan, ids, device=None, fuse_gate_up=True)
    for a, b in ((fused.gate_up.w, L.gate_up.w), (fused.gate_up.scales, L.gate_up.scales),
                 (fused.gate_up.biases, L.gate_up.biases)):
        assert np.array_equal(a, _sel(b, ids))  # concat(gate, up) on the output axis, per expert


def test_resident_layer_matches_the_fused_layout(ckpt):
    root, wm, Ls = ckpt
    L = Ls[0]
    plan = P.build_quantized_expert_layer_plan(root, wm, PREFIX.format(0))
    page = P.load_resident_expert_layer(plan, device=None)
    assert page.gate is None and page.up is None
    for a, b in ((page.gate_up.w, L.gate_up.w), (page.gate_up.scales, L.gate_up.scales),
                 (page.gate_up.biases, L.gate_up.biases), (page.down.w, L.down.w)):
        assert np.array_equal(a, b)
    assert page.bytes_read == plan.complete_expert_payload_byte_count()


def test_read_weight_map(ckpt, tmp_path):
    root, wm, _ = ckpt
    assert P.read_weight_map(root) == wm
    from safetensors.torch import save_file
    save_file({"a": torch.zeros(2), "b": torch.ones(3)}, str(tmp_path / "model.safetensors"))
    assert P.read_weight_map(str(tmp_path)) == {"a": "model.safetensors", "b": "model.safetensors"}
