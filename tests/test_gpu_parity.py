"""HIP path vs the CPU oracle, through the C ABI, on an MI355X.

Bars: integer and index outputs (routing ids, permutation, offsets) bit-exact; the
deterministic elementwise stages (SwiGLU, weighted sums, shared combine) bit-exact;
matmul outputs (bf16 out, fp32 accumulation; the MFMA path rounds dequantised weights
to bf16) within rel-L2 1e-2 and a median of 2 bf16 ulps (moe_testutil)."""
import os

import numpy as np
import pytest

from astronomical_amd import configs as CF
from astronomical_amd import synthetic as S
from astronomical_amd.layout import AffineWeights, bf16_to_f32, f32_to_bf16, pack_codes

from conftest import GOLDEN
from moe_testutil import assert_bf16_close, ulp_distance

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ops():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    from astronomical_amd import ops as O
    O._lib.lib()
    return O


def _dev_bf16(a):
    from astronomical_amd.ops import _bf16_dev
    return _bf16_dev(a)


def _dev_u32(a):
    from astronomical_amd.ops import _u32_dev
    return _u32_dev(a)


def _np(t):
    from astronomical_amd.ops import bf16_to_numpy, u32_to_numpy
    return bf16_to_numpy(t) if t.dtype == torch.bfloat16 else u32_to_numpy(t)


# ------------------------------------------------------------------ routing

@pytest.mark.parametrize("T,E,k", [(1, 256, 8), (8, 256, 8), (2048, 256, 8), (16, 32, 4),
                                   (33, 128, 8), (5, 70, 3), (3, 1024, 64)])
def test_route_topk_bit_exact(ops, orc, T, E, k):
    rng = np.random.default_rng(T * 7 + E)
    logits = f32_to_bf16((rng.standard_normal((T, E)) * 0.9).astype(np.float32))
    logits[T // 2:] = f32_to_bf16(np.round(bf16_to_f32(logits[T // 2:]) * 4) / 4)  # many ties
    want_idx, want_sc = orc.route_topk(logits, k, True)
    idx, sc = ops.qwen3_5_moe_route_experts(_dev_bf16(logits), k, True)
    assert np.array_equal(_np(idx), want_idx)
    assert np.array_equal(_np(sc), want_sc)
    want_idx2, want_sc2 = orc.route_topk(logits, k, False)
    idx2, sc2 = ops.qwen3_5_moe_route_experts(_dev_bf16(logits), k, False)
    assert np.array_equal(_np(idx2), want_idx2) and np.array_equal(_np(sc2), want_sc2)


def test_route_ties_fixture(ops):
    fx = np.load(os.path.join(GOLDEN, "route_ties.npz"), allow_pickle=False)
    for E, k in ((256, 8), (32, 4)):
        idx, _ = ops.qwen3_5_moe_route_experts(_dev_bf16(fx[f"logits_E{E}_k{k}"]), k, True)
        assert np.array_equal(_np(idx), fx[f"indices_E{E}_k{k}"])


def test_route_and_combine_kat(ops, kats):
    d = kats["route_and_combine"]
    idx, sc = ops.qwen3_5_moe_route_experts(_dev_bf16(f32_to_bf16(np.array([d["logits"]], np.float32))), 2, True)
    assert _np(idx)[0].tolist() == [2, 3]
    assert np.allclose(np.sort(bf16_to_f32(_np(sc)[0])), d["expected_sorted_scores"], rtol=2 ** -8)
    eo = f32_to_bf16(np.array(d["expert_outputs"], np.float32))
    selected = _dev_bf16(eo[_np(idx)[0].astype(np.int64)][None])
    y = ops.qwen3_5_moe_combine_experts(selected, sc, _dev_bf16(f32_to_bf16(np.array([d["shared_output"]], np.float32))),
                                        _dev_bf16(f32_to_bf16(np.array([d["shared_gate_logit"]], np.float32))))
    assert np.allclose(bf16_to_f32(_np(y))[0], d["expected_combined"], rtol=2 ** -7)


# ------------------------------------------------------------------ sort

@pytest.mark.parametrize("A,E", [(6, 6), (64, 32), (16384, 256), (32768, 256), (4096, 128), (1, 4),
                                 (5000, 1024), (2048, 1)])
def test_sort_bit_exact(ops, orc, A, E):
    rng = np.random.default_rng(A + E)
    if A == 32768:  # skewed: most assignments on a few experts, many experts empty
        ids = np.minimum(rng.zipf(1.3, size=A) - 1, E - 1).astype(np.uint32)
    else:
        ids = rng.integers(0, E, size=A).astype(np.uint32)
    so, inv, sid, off = orc.sort_assignments(ids, E)
    r = ops.sort_expert_assignments(_dev_u32(ids), E)
    assert np.array_equal(_np(r.sorted_order), so)
    assert np.array_equal(_np(r.inverse_order), inv)
    assert np.array_equal(_np(r.sorted_indices), sid)
    assert np.array_equal(_np(r.expert_offsets), off)


def test_sort_puts_out_of_range_ids_last(ops):
    """ids >= E (E = 1024 uses the extra bucket past the workgroup's 1024 threads) sort after
    every expert, stably; checked against numpy's stable argsort of the clipped ids."""
    rng = np.random.default_rng(7)
    E, A = 1024, 6000
    ids = rng.integers(0, E + 80, size=A).astype(np.uint32)
    r = ops.sort_expert_assignments(_dev_u32(ids), E)
    want = np.argsort(np.minimum(ids, E), kind="stable").astype(np.uint32)
    assert np.array_equal(_np(r.sorted_order), want)
    assert np.array_equal(_np(r.sorted_indices), ids[want])
    inv = np.empty(A, np.uint32)
    inv[want] = np.arange(A, dtype=np.uint32)
    assert np.array_equal(_np(r.inverse_order), inv)
    counts = np.bincount(np.minimum(ids, E), minlength=E + 1)
    assert np.array_equal(_np(r.expert_offsets)[: E + 1], np.concatenate([[0], np.cumsum(counts[:E])]).astype(np.uint32))


def test_sort_kat(ops, kats):
    d = kats["sort_and_restore"]
    r = ops.sort_expert_assignments(_dev_u32(np.array(d["ids"], np.uint32).reshape(2, 3)), 6)
    assert _np(r.sorted_indices).tolist() == d["expected_sorted_ids"]
    assert _np(r.inverse_order).tolist() == d["expected_inverse"]
    hidden = np.array(d["hidden"])
    assert hidden[_np(r.sorted_order) // 3].tolist() == d["expected_sorted_states"]


# ------------------------------------------------------------------ quantized matmuls

def _aff_from_kat(d):
    w = np.array(d["w"], np.uint32).reshape(d["w_shape"])
    s = f32_to_bf16(np.array(d["scales"], np.float32)).reshape(d["sb_shape"])
    b = f32_to_bf16(np.array(d["biases"], np.float32)).reshape(d["sb_shape"])
    return AffineWeights(_dev_u32(w), _dev_bf16(s), _dev_bf16(b), d["bits"], d["group"])


@pytest.mark.parametrize("name", ["qmm_4bit_g64", "qmm_8bit_g64"])
def test_quantized_matmul_kats(ops, kats, name):
    d = kats[name]
    x = _dev_bf16(f32_to_bf16(np.array(d["x"], np.float32).reshape(d["x_shape"])))
    y = ops.quantized_matmul_affine(x, _aff_from_kat(d))
    assert bf16_to_f32(_np(y)).reshape(-1).tolist() == d["expected"]


def test_gather_qmm_kat(ops, kats):
    d = kats["gather_qmm_4bit"]
    x = _dev_bf16(f32_to_bf16(np.array(d["x"], np.float32).reshape(d["x_shape"])))
    y = ops.gather_expert_projection(x, _aff_from_kat(d), _dev_u32(np.array(d["ids"], np.uint32)),
                                     token_rows=_dev_u32(np.zeros(2, np.uint32)))
    assert bf16_to_f32(_np(y)).tolist() == d["expected"]


def _random_affine(rng, E, N, K, bits, group):
    codes = rng.integers(0, 1 << bits, size=(E, N, K))
    w = pack_codes(codes, bits)
    s = f32_to_bf16(rng.uniform(0.002, 0.02, size=(E, N, K // group)).astype(np.float32))
    b = f32_to_bf16((-(1 << (bits - 1)) * bf16_to_f32(s) + rng.normal(0, 1e-3, s.shape)).astype(np.float32))
    return AffineWeights(w, s, b, bits, group)


@pytest.mark.parametrize("bits,group", [(4, 32), (4, 64), (4, 128), (8, 32), (8, 64), (8, 128)])
@pytest.mark.parametrize("sorted_ids", [False, True])
def test_gather_qmm_matches_oracle(ops, orc, bits, group, sorted_ids):
    rng = np.random.default_rng(bits * 100 + group)
    E, N, K, rows = 9, 192, 512, 300
    aff = _random_affine(rng, E, N, K, bits, group)
    x = f32_to_bf16(rng.standard_normal((rows, K)).astype(np.float32))
    ids = rng.integers(0, E, size=rows).astype(np.uint32)
    ids[:40] = 3  # one expert with more than one tile of rows
    if sorted_ids:
        ids = np.sort(ids)
    want = orc.gather_qmm(x, aff, ids)
    daff = aff.map(lambda a: _dev_u32(a) if a.dtype == np.uint32 else _dev_bf16(a))
    order = ops.ExpertAssignmentOrder.SORTED_BY_EXPERT if sorted_ids else ops.ExpertAssignmentOrder.ORIGINAL
    got = _np(ops.gather_expert_projection(_dev_bf16(x), daff, _dev_u32(ids), order))
    assert_bf16_close(got, want, f"gather_qmm {bits}-bit g{group}")


@pytest.mark.parametrize("bits,group", [(4, 32), (4, 64), (8, 32), (8, 64)])
@pytest.mark.parametrize("K", [64, 576])
def test_gather_qmm_odd_and_single_k_steps(ops, orc, bits, group, K):
    """The 4-wave grouped GEMM's two load stages over one K step (K = 64) and an odd number of
    steps (K = 576, a tail step after the pairs), with a partial last column tile (N = 130) and
    experts of 1-70 rows."""
    rng = np.random.default_rng(bits * 1000 + group + K)
    E, N, rows = 5, 130, 160
    aff = _random_affine(rng, E, N, K, bits, group)
    x = f32_to_bf16(rng.standard_normal((rows, K)).astype(np.float32))
    ids = np.sort(np.concatenate([np.full(70, 1), np.full(1, 2), rng.integers(0, E, size=rows - 71)]))
    ids = ids.astype(np.uint32)
    want = orc.gather_qmm(x, aff, ids)
    daff = aff.map(lambda a: _dev_u32(a) if a.dtype == np.uint32 else _dev_bf16(a))
    got = _np(ops.gather_expert_projection(_dev_bf16(x), daff, _dev_u32(ids),
                                           ops.ExpertAssignmentOrder.SORTED_BY_EXPERT))
    assert_bf16_close(got, want, f"gather_qmm {bits}-bit g{group} K{K}")


# ------------------------------------------------------------------ elementwise stages

def test_swiglu_bit_exact(ops, orc):
    rng = np.random.default_rng(2)
    g = f32_to_bf16((rng.standard_normal(100003) * 4).astype(np.float32))
    u = f32_to_bf16((rng.standard_normal(100003) * 4).astype(np.float32))
    g[:6] = f32_to_bf16(np.array([0.0, -0.0, 90.0, -90.0, 1e-30, -200.0], np.float32))
    assert np.array_equal(_np(ops.apply_compiled_swiglu(_dev_bf16(g), _dev_bf16(u))), orc.swiglu(g, u))


def test_swiglu_every_gate_value(ops, orc):
    """The kernels' sigmoid takes a hardware exp2/reciprocal path away from bf16 rounding
    midpoints and the exact one near them: every one of the 2^16 bf16 gate values (signed
    zeros, denormals, infinities, NaNs included) against the oracle, with up = 1 (the output is
    bf16(g * bf16(sigmoid(g))) itself), with random up values, and with up values that overflow
    or underflow the product.  NaN outputs compare as NaN (their payload is not specified)."""
    g = np.arange(1 << 16, dtype=np.uint16)
    rng = np.random.default_rng(7)
    ups = [np.full(g.size, 0x3F80, np.uint16),
           f32_to_bf16((rng.standard_normal(g.size) * 3).astype(np.float32)),
           f32_to_bf16(np.full(g.size, 3.0e38, np.float32)),
           f32_to_bf16(np.full(g.size, -1.5e-38, np.float32))]
    for i, u in enumerate(ups):
        got = _np(ops.apply_compiled_swiglu(_dev_bf16(g), _dev_bf16(u)))
        want = orc.swiglu(g, u)
        nan_want = (want & 0x7FFF) > 0x7F80
        nan_got = (got & 0x7FFF) > 0x7F80
        assert np.array_equal(nan_got, nan_want), f"up set {i}: NaN positions differ"
        bad = np.flatnonzero((got != want) & ~nan_want)
        assert bad.size == 0, f"up set {i}: {bad.size} gate values differ, first g=0x{g[bad[0]]:04x}"


def test_bf16_rounding_selftest(ops):
    """gfx950's fp32 -> bf16 conversion, which every kernel rounds with, equals round-to-nearest-
    even on the bit pattern (the oracle's rounding) for all 2^32 fp32 patterns."""
    assert ops.selftest_bf16_rounding() == 0


def test_weighted_sums_bit_exact(ops, orc, kats):
    rng = np.random.default_rng(4)
    T, k, D = 37, 8, 2048
    out = f32_to_bf16(rng.standard_normal((T * k, D)).astype(np.float32))
    sc = f32_to_bf16(rng.dirichlet(np.ones(k), size=T).astype(np.float32))
    perm = rng.permutation(T * k).astype(np.uint32)
    sorted_out = np.empty_like(out)
    sorted_out[perm] = out
    got = ops.sorted_expert_weighted_sum(_dev_bf16(sorted_out), _dev_u32(perm), _dev_bf16(sc))
    assert np.array_equal(_np(got), orc.sorted_weighted_sum(sorted_out, perm, sc))
    got_u = ops.unsorted_expert_weighted_sum(_dev_bf16(out.reshape(T, k, D)), _dev_bf16(sc))
    assert np.array_equal(_np(got_u), orc.unsorted_weighted_sum(out.reshape(T, k, D), sc))
    d = kats["sorted_weighted_sum"]
    y = ops.sorted_expert_weighted_sum(_dev_bf16(f32_to_bf16(np.array(d["sorted_outputs"], np.float32))),
                                       _dev_u32(np.array(d["inverse"], np.uint32)),
                                       _dev_bf16(f32_to_bf16(np.array(d["scores"], np.float32))))
    assert np.allclose(bf16_to_f32(_np(y)), d["expected"], rtol=2 ** -7)
    d = kats["unsorted_weighted_sum"]
    y = ops.unsorted_expert_weighted_sum(_dev_bf16(f32_to_bf16(np.array(d["outputs"], np.float32))),
                                         _dev_bf16(f32_to_bf16(np.array(d["scores"], np.float32))))
    assert bf16_to_f32(_np(y)).tolist() == d["expected"]


def test_combine_shared_bit_exact(ops, orc):
    rng = np.random.default_rng(8)
    T, D = 19, 1024
    sp = f32_to_bf16(rng.standard_normal((T, D)).astype(np.float32))
    so = f32_to_bf16(rng.standard_normal((T, D)).astype(np.float32))
    z = f32_to_bf16(rng.standard_normal(T).astype(np.float32) * 3)
    got = ops.combine_sparse_and_shared_experts(_dev_bf16(sp), _dev_bf16(so), _dev_bf16(z))
    assert np.array_equal(_np(got), orc.combine_shared(sp, so, z))


# ------------------------------------------------------------------ whole block

def _device_layer(ops, L):
    return ops.to_device(L)


def _check_block(ops, orc, L, x, what):
    """GPU block vs oracle: routing bit-exact on the GPU's logits, outputs to the FP bar."""
    dL = _device_layer(ops, L)
    blk = ops.MoeBlock(dL)
    T = x.shape[0]
    y = _np(blk(_dev_bf16(x)))
    tr = blk.trace(T)
    # router projection: fp32 accumulation in another order -> within one bf16 ulp
    want_logits = None
    if L.router_bias is None and L.router_q is not None:
        # affine router: the decode kernels (T <= 8) and the prefill router GEMM both keep the
        # codes exact and factor each group's terms as s * sum((MAG + q) x) + (b - MAG s) *
        # sum(x) in fp32 -> bounded by the magnitudes those terms carry
        want_logits = orc.qmm(x, L.router_q)
        rq = L.router_q
        deq = bf16_to_f32(orc.dequantize(rq)).astype(np.float64)
        g = rq.group_size
        sc = np.repeat(bf16_to_f32(rq.scales[0]).astype(np.float64), g, axis=1)
        xf = bf16_to_f32(x).astype(np.float64)
        mag = np.abs(xf) @ (np.abs(deq) + (1 << rq.bits) * sc).T
        ref = bf16_to_f32(want_logits).astype(np.float64)
        got = bf16_to_f32(tr["logits"]).astype(np.float64)
        ulp = np.abs(np.spacing(ref.astype(np.float32)).astype(np.float64)) * 2 ** 16
        assert np.all(np.abs(got - ref) <= ulp + 2.0 ** -16 * mag), what
        assert np.mean(ulp_distance(tr["logits"], want_logits) <= 1) > 0.99, what
        want_logits = None
    elif L.router_bias is None:
        want_logits = orc.router_logits(x, L.router_w)
    if want_logits is not None:
        # two fp32 accumulation orders differ by a few 2^-24 * sum|x*w| (absolute), then
        # each result is rounded to bf16: |diff| <= ulp(ref) + 2^-18 * sum|x*w|
        xa = np.abs(bf16_to_f32(x).astype(np.float64))
        wa = np.abs(bf16_to_f32(L.router_w).astype(np.float64))
        mag = xa @ wa.T
        ref = bf16_to_f32(want_logits).astype(np.float64)
        got = bf16_to_f32(tr["logits"]).astype(np.float64)
        ulp = np.abs(np.spacing(ref.astype(np.float32)).astype(np.float64)) * 2 ** 16
        assert np.all(np.abs(got - ref) <= ulp + 2.0 ** -18 * mag), what
        assert np.mean(ulp_distance(tr["logits"], want_logits) <= 1) > 0.999, what
    # routing and permutation bit-exact given identical logits
    y_ref, ref = orc.moe_block_forward(L, x, logits_override=tr["logits"], trace=True)
    assert np.array_equal(tr["indices"], ref["indices"]), what
    assert np.array_equal(tr["scores"], ref["scores"]), what
    A = T * L.top_k
    so, inv, sid, off = orc.sort_assignments(tr["indices"].reshape(-1), L.num_experts)
    assert np.array_equal(tr["sorted_order"], so) and np.array_equal(tr["inverse_order"], inv)
    assert np.array_equal(tr["sorted_ids"], sid) and np.array_equal(tr["expert_offsets"], off)
    assert tr["sorted_path"] == (A >= 64) == ref["used_sorted_path"]
    # the combine is deterministic: bit-exact against the oracle's combine of the device's
    # own expert outputs, scores and shared expert
    eo = tr["expert_out_sorted"]
    if tr["sorted_path"]:
        sparse_ref = orc.sorted_weighted_sum(eo, tr["inverse_order"], tr["scores"])
    else:
        sparse_ref = orc.unsorted_weighted_sum(eo[tr["inverse_order"]].reshape(T, L.top_k, -1), tr["scores"])
    assert np.array_equal(tr["sparse"], sparse_ref), what + " sparse combine"
    if L.shared_intermediate:
        assert np.array_equal(y, orc.combine_shared(sparse_ref, tr["shared_out"], tr["shared_gate_logits"])), \
            what + " shared combine"
    else:
        assert np.array_equal(y, sparse_ref), what + " combine"
    # intermediates and output
    act = tr["activated_sorted"][inv]  # back to assignment order
    stats = {"act": assert_bf16_close(act, ref["activated"], what + " activated")}
    stats["expert_out"] = assert_bf16_close(tr["expert_out_sorted"][inv], ref["expert_out"], what + " expert_out")
    stats["y"] = assert_bf16_close(y, y_ref, what + " y")
    if L.shared_intermediate:
        stats["shared"] = assert_bf16_close(tr["shared_out"], ref["shared_out"], what + " shared")
    # end-to-end routing with the oracle's own router: tokens whose top-k set differs
    _, ref2 = orc.moe_block_forward(L, x, trace=True)
    differ = int(np.sum(np.any(np.sort(ref2["indices"], 1) != np.sort(tr["indices"], 1), axis=1)))
    stats["tokens_with_different_topk_set"] = differ
    assert differ <= max(1, T // 200), (what, differ)
    print(what, stats)
    return stats


def test_block_c0_golden(ops, orc):
    fx = np.load(os.path.join(GOLDEN, "c0_block.npz"), allow_pickle=False)
    L = S.make_layer(CF.C0)
    _check_block(ops, orc, L, fx["x"], "c0")
    blk = ops.MoeBlock(_device_layer(ops, L))
    y = _np(blk(_dev_bf16(fx["x"])))
    assert_bf16_close(y, fx["y"], "c0 vs committed fixture")


@pytest.fixture(scope="module")
def c1_layer():
    return S.make_layer(CF.C1)


@pytest.mark.parametrize("T", [1, 2, 4, 8])
def test_block_c1_decode(ops, orc, c1_layer, T):
    _check_block(ops, orc, c1_layer, S.make_tokens(CF.C1, T), f"c1 B={T}")


@pytest.mark.parametrize("group", [2, 3, 5])
def test_block_c1_decode_tied_router_rows(ops, orc, c1_layer, group):
    """Router rows repeated in runs of `group` experts: those experts' logits and bf16
    probabilities are equal, so the top-k set and its order rest on the index tie rule (ties
    toward the higher index) in every routing path the decode kernels take -- the single-token
    set of the gate/up workgroups, the batch routing kernel and the published MLX order."""
    import copy
    L = copy.copy(c1_layer)
    w = np.array(c1_layer.router_w, copy=True)
    w[:] = w[(np.arange(w.shape[0]) // group) * group]
    L.router_w = w
    for i, T in enumerate((1, 1, 1, 2, 8)):
        x = S.make_tokens(CF.C1, T, step=100 * group + i)
        _check_block(ops, orc, L, x, f"c1 tied rows x{group} B={T}")


@pytest.fixture(scope="module")
def c1_affine_router_layers():
    return {bits: S.make_layer(CF.C1, router_bits=bits) for bits in (4, 8)}


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("T", [1, 2, 4, 8, 64])
def test_block_c1_affine_router(ops, orc, c1_affine_router_layers, bits, T):
    """The reference's certified Qwen3.5/3.6-MoE checkpoints quantize mlp.gate
    (tests/common/qwen3_5_moe.rs:299-308): the router runs as quantized_linear
    (forward.rs:53-58).  T <= 8 takes the decode kernels' affine router, T = 64 the grouped
    GEMM."""
    _check_block(ops, orc, c1_affine_router_layers[bits], S.make_tokens(CF.C1, T), f"c1 affine router {bits}-bit T={T}")


def test_block_c2_prefill_subset(ops, orc, c1_layer):
    _check_block(ops, orc, c1_layer, S.make_tokens(CF.C2, 256), "c2 T=256")


def test_block_c3_skewed_subset(ops, orc):
    L = S.make_layer(CF.C3)
    _check_block(ops, orc, L, S.make_tokens(CF.C3, 512), "c3 T=512 (Zipf)")


def test_block_c4_8bit(ops, orc):
    """8-bit g32 without a shared expert: T <= 8 takes the decode kernels (two participants per
    down-kernel wave, two input chunks per lane), T = 64 the grouped GEMMs."""
    L = S.make_layer(CF.C4)
    for T in (1, 2, 8, 64):
        _check_block(ops, orc, L, S.make_tokens(CF.C4, T), f"c4 T={T}")


@pytest.mark.parametrize("T", [1, 2, 8])
def test_block_c0_decode(ops, orc, T):
    """c0's shapes (4-bit, top-4 of 32, no shared expert) through the decode kernels: one, two
    and four output rows per quarter-wave in the down kernel."""
    L = S.make_layer(CF.C0)
    _check_block(ops, orc, L, S.make_tokens(CF.C0, T), f"c0 T={T}")


def test_fused_and_separate_gate_up_are_bit_identical(ops):
    """resident_gate_up_fusion.rs:13-90 on the device."""
    L = S.make_layer(CF.C0, keep_separate=True)
    x = _dev_bf16(S.make_tokens(CF.C0, 40))
    fused = ops.MoeBlock(_device_layer(ops, L))
    Ls = L.map(lambda a: a)
    Ls.gate_up = None
    sep = ops.MoeBlock(_device_layer(ops, Ls))
    assert np.array_equal(_np(fused(x)), _np(sep(x)))


def test_attributed_forward_matches_forward(ops, c1_layer):
    """The attributed entry point computes the same bits and reports the stages it ran:
    three kernels on the decode path; on the sorted path every stage but the shared expert's
    output gate, which the route kernel computes."""
    blk = ops.MoeBlock(_device_layer(ops, c1_layer))
    for T, expect in ((1, {"router", "gate_up", "down"}), (128, set(ops._lib.STAGES) - {"shared"})):
        x = _dev_bf16(S.make_tokens(CF.C1, T))
        y = _np(blk(x))
        y2, st = blk.forward_attributed(x)
        assert np.array_equal(_np(y2), y)
        assert {k for k, v in st.items() if v > 0} == expect, (T, st)
        assert all(0 <= v < 50 for v in st.values()), st


def test_empty_token_batch(ops):
    L = S.make_layer(CF.C0)
    blk = ops.MoeBlock(_device_layer(ops, L))
    y = blk(torch.empty(0, L.hidden, dtype=torch.bfloat16, device="cuda"))
    assert y.shape == (0, L.hidden)


def test_device_generator_matches_numpy(ops):
    from astronomical_amd import device_synthetic as DS
    cfg = CF.C0
    host = S.make_layer(cfg)
    dev = DS.make_layer_device(cfg)
    assert np.array_equal(_np(dev.gate_up.w), host.gate_up.w)
    assert np.array_equal(_np(dev.down.w), host.down.w)
    for a, b in ((dev.gate_up.scales, host.gate_up.scales), (dev.gate_up.biases, host.gate_up.biases),
                 (dev.router_w, host.router_w)):
        assert np.mean(_np(a) == b) > 0.9999
    xd = _np(DS.make_tokens_device(cfg, 16))
    assert np.mean(xd == S.make_tokens(cfg, 16)) > 0.9999


def _adversarial_logits(orc, E, k):
    """Logits whose probabilities order the experts as orc.adversarial_ranks does, so the
    slice order comes out of libstdc++'s heap selection: the E largest-spaced bf16 values
    in [-40, 0] whose softmax probabilities stay distinct in bf16."""
    ranks = orc.adversarial_ranks(E, E - k)
    cand = np.unique(f32_to_bf16(-np.linspace(0, 40, 40 * 64 + 1).astype(np.float32)))
    vals = np.sort(bf16_to_f32(cand))[::-1]  # descending from 0
    chosen, last_p = [], None
    for v in vals:
        p = np.float32(np.exp(np.float64(v)))
        pb = f32_to_bf16(np.array([p], np.float32))[0]
        if last_p is None or pb != last_p:
            chosen.append(v)
            last_p = pb
        if len(chosen) == E:
            break
    levels = np.array(chosen[::-1], np.float32)  # ascending
    return f32_to_bf16(levels[ranks])[None]


@pytest.mark.parametrize("E,k", [(64, 4), (256, 8), (512, 16)])
def test_route_topk_adversarial_rows_take_the_heap_selection(ops, orc, E, k):
    from nth_element_model import nth_element
    logits = _adversarial_logits(orc, E, k)
    want_idx, want_sc, p = orc.route_topk(logits, k, True, with_probabilities=True)
    keys = [(int(v), i) for i, v in enumerate(p[0])]
    _, used_heap = nth_element(keys, E - k)
    assert used_heap and len(set(p[0].tolist())) == E
    idx, sc = ops.qwen3_5_moe_route_experts(_dev_bf16(logits), k, True)
    assert np.array_equal(_np(idx), want_idx)
    assert np.array_equal(_np(sc), want_sc)
