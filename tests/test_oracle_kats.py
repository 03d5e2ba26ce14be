"""The oracle against the known-answer vectors of the reference's own tests (CPU only).

The reference tests feed float32 arrays; the block's dtype is bf16, so inputs are
rounded to bf16 first.  Integer-valued vectors stay exact; fractional ones are compared
at bf16 resolution (the tolerance is stated at each assertion).
"""
import math

import numpy as np
import pytest

from astronomical_amd.layout import AffineWeights, bf16_to_f32, f32_to_bf16


def _aff(d):
    w = np.array(d["w"], dtype=np.uint32).reshape(d["w_shape"])
    if w.ndim == 2:
        w = w[None]
    sb_shape = d.get("sb_shape", [1, w.shape[1], len(d["scales"]) // w.shape[1]])
    s = f32_to_bf16(np.array(d["scales"], np.float32)).reshape(sb_shape)
    b = f32_to_bf16(np.array(d["biases"], np.float32)).reshape(sb_shape)
    return AffineWeights(w, s, b, d["bits"], d["group"])


@pytest.mark.parametrize("name", ["qmm_4bit_g64", "qmm_8bit_g64", "qmm_5bit_g32_zeros"])
def test_quantized_matmul_kats(orc, kats, name):
    d = kats[name]
    x = f32_to_bf16(np.array(d["x"], np.float32).reshape(d["x_shape"]))
    y = orc.qmm(x, _aff(d))
    assert bf16_to_f32(y).reshape(-1).tolist() == d["expected"]


def test_gather_qmm_kat(orc, kats):
    d = kats["gather_qmm_4bit"]
    x = f32_to_bf16(np.array(d["x"], np.float32).reshape(d["x_shape"]))
    y = orc.gather_qmm(x, _aff(d), np.array(d["ids"], np.uint32), x_rows=np.zeros(2, np.uint32))
    assert bf16_to_f32(y).tolist() == d["expected"]


def test_dequantize_selected_rows_kat(orc, kats):
    d = kats["dequantize_8bit_rows"]
    w = np.array(d["w"], np.uint32).reshape(d["w_shape"])
    rows = np.array(d["take"])
    aff = AffineWeights(w[rows][None], f32_to_bf16(np.array(d["scales"], np.float32))[rows].reshape(1, 2, 1),
                        f32_to_bf16(np.array(d["biases"], np.float32))[rows].reshape(1, 2, 1),
                        d["bits"], d["group"])
    assert bf16_to_f32(orc.dequantize(aff)).tolist() == d["expected_rows"]


def test_route_and_combine_kat(orc, kats):
    d = kats["route_and_combine"]
    logits = f32_to_bf16(np.array([d["logits"]], np.float32))
    idx, sc = orc.route_topk(logits, d["top_k"], d["normalize"])
    assert sorted(idx[0].tolist()) == [2, 3]
    # the selected slice is emitted ascending in (probability, index)
    assert idx[0].tolist() == [2, 3]
    scores = np.sort(bf16_to_f32(sc[0]))
    # bf16 inputs and outputs: within one bf16 ulp (2**-9 relative) of 3/7 and 4/7
    assert np.allclose(scores, d["expected_sorted_scores"], rtol=2 ** -8, atol=0)
    eo = f32_to_bf16(np.array(d["expert_outputs"], np.float32))
    selected = eo[idx[0]][None]
    sparse = orc.unsorted_weighted_sum(selected, sc)
    y = orc.combine_shared(sparse, f32_to_bf16(np.array([d["shared_output"]], np.float32)),
                           f32_to_bf16(np.array([d["shared_gate_logit"]], np.float32)))
    assert np.allclose(bf16_to_f32(y)[0], d["expected_combined"], rtol=2 ** -7, atol=0)


def test_sort_and_restore_kat(orc, kats):
    d = kats["sort_and_restore"]
    ids = np.array(d["ids"], np.uint32)
    so, inv, sid, off = orc.sort_assignments(ids, 6)
    hidden = np.array(d["hidden"], np.float32)
    assert hidden[so // d["top_k"]].tolist() == d["expected_sorted_states"]
    assert sid.tolist() == d["expected_sorted_ids"]
    assert inv.tolist() == d["expected_inverse"]
    assert off.tolist() == [0, 1, 2, 3, 4, 5, 6]
    sorted_outputs = np.array(d["sorted_outputs"], np.float32)
    assert sorted_outputs[inv].tolist() == d["expected_restored"]


def test_sorted_weighted_sum_kat(orc, kats):
    d = kats["sorted_weighted_sum"]
    so = f32_to_bf16(np.array(d["sorted_outputs"], np.float32))
    sc = f32_to_bf16(np.array(d["scores"], np.float32))
    y = orc.sorted_weighted_sum(so, np.array(d["inverse"], np.uint32), sc)
    # the bf16 scores 0.1/0.2/0.7 carry up to 2**-9 relative error; outputs are bf16
    assert np.allclose(bf16_to_f32(y), d["expected"], rtol=2 ** -7, atol=0)
    # restored-unsorted reduction agrees (sparse_experts.rs:146-166)
    restored = so[np.array(d["inverse"])].reshape(2, 3, 2)
    y2 = orc.unsorted_weighted_sum(restored, sc)
    assert np.allclose(bf16_to_f32(y2), d["expected"], rtol=2 ** -7, atol=0)


def test_unsorted_weighted_sum_kat(orc, kats):
    d = kats["unsorted_weighted_sum"]
    y = orc.unsorted_weighted_sum(f32_to_bf16(np.array(d["outputs"], np.float32)),
                                  f32_to_bf16(np.array(d["scores"], np.float32)))
    assert bf16_to_f32(y).tolist() == d["expected"]


def test_invert_assignment_order_kat(orc, kats):
    d = kats["invert_assignment_order"]
    assert orc.invert_assignment_order(np.array(d["sorted_order"])).tolist() == d["expected"]
    assert orc.invert_assignment_order(np.array(d["empty"], np.uint32)).tolist() == []
    with pytest.raises(orc.OracleError, match="duplicate"):
        orc.invert_assignment_order(np.array(d["duplicate"]))
    with pytest.raises(orc.OracleError, match="out-of-range"):
        orc.invert_assignment_order(np.array(d["out_of_range"]))


def test_argpartition_top1_kat(orc, kats):
    d = kats["argpartition_top1"]
    idx, _ = orc.route_topk(f32_to_bf16(np.array(d["scores"], np.float32)), 1, normalize=False)
    assert idx[:, 0].tolist() == d["expected_top_index"]
    assert np.array(d["scores"])[[0, 1], idx[:, 0]].tolist() == d["expected_top_score"]


def test_swiglu_kat_matches_closed_form(orc, kats):
    for case in kats["swiglu"]["cases"]:
        g = f32_to_bf16(np.array(case["gate"], np.float32))
        u = f32_to_bf16(np.array(case["up"], np.float32))
        got = bf16_to_f32(orc.swiglu(g, u)).astype(np.float64)
        gf, uf = bf16_to_f32(g).astype(np.float64), bf16_to_f32(u).astype(np.float64)
        want = gf / (1.0 + np.exp(-gf)) * uf
        # three bf16 roundings (sigmoid, g*s, *u): within 3 half-ulps of bf16
        assert np.all(np.abs(got - want) <= 3 * 2 ** -9 * np.maximum(np.abs(want), 1e-30)), (got, want)


def test_empty_assignments_kat(orc, kats):
    so, inv, sid, off = orc.sort_assignments(np.zeros(0, np.uint32), 4)
    assert so.shape == (0,) and inv.shape == (0,) and off.tolist() == [0] * 5
    y = orc.unsorted_weighted_sum(np.zeros((1, 0, 2), np.uint16), np.zeros((1, 0), np.uint16))
    assert bf16_to_f32(y).tolist() == [kats["empty_assignments"]["expected_reduction"]]
