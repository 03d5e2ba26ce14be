"""Writes reference_kats.json: the known-answer vectors the reference's own tests hold
for the MoE block, transcribed as data (inputs and expected outputs) with the file:line
of the reference test each one comes from.  Run: python tests/golden/make_reference_kats.py
"""
import json
import math
import os

k = {}
src = "crates/runtime-integration/tests/direct_mlx/quantized_operations.rs"
k["qmm_4bit_g64"] = dict(source=src + ":5-61", x=list(range(1, 65)), x_shape=[1, 64],
    w=[0x11111111] * 8 + [0x22222222] * 8, w_shape=[1, 2, 8], scales=[1.0, 1.0], biases=[0.0, 0.0],
    sb_shape=[1, 2, 1], bits=4, group=64, expected=[2080.0, 4160.0])
k["qmm_8bit_g64"] = dict(source=src + ":63-135", x=list(range(1, 65)), x_shape=[1, 64],
    w=[0x01010101] * 16 + [0x02020202] * 16, w_shape=[1, 2, 16], scales=[1.0, 1.0], biases=[0.0, 0.0],
    sb_shape=[1, 2, 1], bits=8, group=64, expected=[2080.0, 4160.0])
k["qmm_5bit_g32_zeros"] = dict(source=src + ":137-172", x=[1.0] * 64, x_shape=[1, 64],
    w=[0] * 20, w_shape=[1, 2, 10], scales=[1.0] * 4, biases=[0.0] * 4, sb_shape=[1, 2, 2],
    bits=5, group=32, expected=[0.0, 0.0])
k["gather_qmm_4bit"] = dict(source=src + ":255-306", x=list(range(1, 65)), x_shape=[1, 64],
    w=[0x11111111] * 8 + [0x22222222] * 8 + [0x55555555] * 8 + [0x66666666] * 8
      + [0x33333333] * 8 + [0x44444444] * 8,
    w_shape=[3, 2, 8], scales=[1.0] * 6, biases=[0.0] * 6, sb_shape=[3, 2, 1], bits=4, group=64,
    ids=[2, 0], expected=[[6240.0, 8320.0], [2080.0, 4160.0]])
k["dequantize_8bit_rows"] = dict(source=src + ":306-340",
    w=[0x01010101] * 16 + [0x02020202] * 16, w_shape=[2, 16], scales=[1.0, 1.0], biases=[0.0, 0.0],
    bits=8, group=64, take=[1, 0], expected_rows=[[2.0] * 64, [1.0] * 64])
rc = "crates/model-serving/tests/direct_mlx/qwen3_5_moe/routing_and_combination.rs"
k["route_and_combine"] = dict(source=rc + ":12-68",
    logits=[0.0, math.log(2.0), math.log(3.0), math.log(4.0)], top_k=2, normalize=True,
    expected_sorted_scores=[3 / 7, 4 / 7],
    expert_outputs=[[0.0, 0.0], [0.0, 0.0], [7.0, 14.0], [14.0, 21.0]],
    shared_output=[2.0, 4.0], shared_gate_logit=0.0, expected_combined=[12.0, 20.0],
    note="the reference test sorts the scores: the order inside the selected slice is not pinned")
k["sort_and_restore"] = dict(source=rc + ":109-182",
    hidden=[[10.0, 11.0], [20.0, 21.0]], ids=[5, 0, 4, 1, 3, 2], top_k=3,
    expected_sorted_states=[[10.0, 11.0], [20.0, 21.0], [20.0, 21.0], [20.0, 21.0], [10.0, 11.0], [10.0, 11.0]],
    expected_sorted_ids=[0, 1, 2, 3, 4, 5], expected_inverse=[5, 0, 4, 1, 3, 2],
    sorted_outputs=[[100.0, 101.0], [110.0, 111.0], [120.0, 121.0], [130.0, 131.0], [140.0, 141.0], [150.0, 151.0]],
    expected_restored=[[150.0, 151.0], [100.0, 101.0], [140.0, 141.0], [110.0, 111.0], [130.0, 131.0], [120.0, 121.0]])
k["sorted_weighted_sum"] = dict(
    source=rc + ":184-226; crates/model-serving/tests/direct_mlx/sparse_experts.rs:86-173",
    sorted_outputs=[[100.0, 101.0], [110.0, 111.0], [120.0, 121.0], [130.0, 131.0], [140.0, 141.0], [150.0, 151.0]],
    inverse=[5, 0, 4, 1, 3, 2], scores=[[0.1, 0.2, 0.7], [0.25, 0.25, 0.5]],
    expected=[[133.0, 134.0], [120.0, 121.0]])
k["unsorted_weighted_sum"] = dict(source="crates/model-serving/tests/direct_mlx/sparse_experts.rs:34-64",
    outputs=[[[2.0, 4.0], [6.0, 8.0]]], scores=[[0.25, 0.75]], expected=[[5.0, 7.0]])
hs = "crates/model-serving/tests/hermetic/sparse_experts.rs"
k["invert_assignment_order"] = dict(source=hs + ":5-36", sorted_order=[1, 3, 5, 4, 2, 0],
    expected=[5, 0, 4, 1, 3, 2], empty=[], duplicate=[0, 0], out_of_range=[0, 2])
k["argpartition_top1"] = dict(
    source="crates/runtime-integration/tests/direct_mlx/array_operations/numeric_operations.rs:268-300",
    scores=[[1.0, 5.0, 3.0, 2.0], [4.0, 0.0, 7.0, 6.0]], expected_top_index=[1, 2],
    expected_top_score=[5.0, 7.0])
k["swiglu"] = dict(source="crates/runtime-integration/tests/direct_mlx/compiled_swiglu.rs:1-52",
    cases=[dict(gate=[-1.0, 0.0, 1.0, 0.5], up=[2.0, 3.0, 4.0, 5.0], shape=[1, 2, 2]),
           dict(gate=[2.0, -2.0, 0.5, -0.5, 1.5, -1.5, 0.25, -0.25, 3.0, -3.0],
                up=[1.0, 2.0, 3.0, 4.0, 0.5, 1.5, 2.5, 3.5, 0.75, 1.25], shape=[1, 5, 2])])
k["empty_assignments"] = dict(source="crates/model-serving/tests/direct_mlx/sparse_experts.rs:175-236",
    hidden=[1.0, 2.0], expected_sorted_states_shape=[0, 1, 2], expected_reduction=[0.0, 0.0])

if __name__ == "__main__":
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_kats.json")
    with open(out, "w") as f:
        json.dump(k, f, indent=1)
    print(out, len(k))
