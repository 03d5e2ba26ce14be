"""The routing slice order: MLX's CPU argpartition is std::nth_element on the index vector with
the (value, index) comparator (CPU only).

The oracle calls the C++ library's std::nth_element (oracle/argpartition.cc).  Pinned here by
the reference's argpartition KAT (numeric_operations.rs:267-305), the partition property, two
slices traced by hand through libstdc++'s introselect, a plain-Python restatement of that
algorithm (tests/nth_element_model.py) on random, tied and adversarial rows — a dropped tie
break, a wrong kth or a transposed comparator fails them — and rows that reach the heap
selection."""
import numpy as np
import pytest

from astronomical_amd.layout import bf16_to_f32, f32_to_bf16

from nth_element_model import argpartition_slice, nth_element


def _keys(v):
    f = bf16_to_f32(v)
    return [(float(x), i) for i, x in enumerate(f)]


def test_reference_argpartition_kat(orc):
    """should_copy_strided_top_indices_and_select_scores: argpartition(kth = -1) of
    [[1, 5, 3, 2], [4, 0, 7, 6]] along the rows puts 1 and 2 last."""
    rows = f32_to_bf16(np.array([[1, 5, 3, 2], [4, 0, 7, 6]], np.float32))
    assert [int(orc.argpartition_bf16(r, 3)[3]) for r in rows] == [1, 2]


def test_hand_traced_slices(orc):
    """logits [0, 2, 0.5, 2, -1, 0.25, 2, 1] (experts 1, 3, 6 tie at the top), traced through
    libstdc++'s introselect by hand.  kth = 6: the median of (1, 4, 7) is 7, swapped to 0; the
    partition around it swaps positions 1 <-> 7 and 3 <-> 5 (cut 5 <= 6), leaving [3, 6, 1] in
    [5, 8), insertion-sorted to [1, 3, 6]: slice [3, 6].  kth = 4: after the same first
    partition (cut 5 > 4) the range is [0, 5); the median of (0, 2, 4) is 0 at position 1;
    the partition swaps positions 1 <-> 4 (cut 2), and [2, 5) = [2, 5, 7] sorts to [5, 2, 7]:
    slice [7, 3, 6, 1]."""
    v = f32_to_bf16(np.array([0.0, 2.0, 0.5, 2.0, -1.0, 0.25, 2.0, 1.0], np.float32))
    assert orc.argpartition_bf16(v, 6)[6:].tolist() == [3, 6]
    assert orc.argpartition_bf16(v, 4)[4:].tolist() == [7, 3, 6, 1]
    assert orc.argpartition_bf16(v, 4).tolist() == [0, 4, 5, 2, 7, 3, 6, 1]
    # the oracle's routing takes the same slices from the softmax of these logits
    idx, _ = orc.route_topk(v[None], 2, True)
    assert idx[0].tolist() == [3, 6]
    idx, _ = orc.route_topk(v[None], 4, True)
    assert idx[0].tolist() == [7, 3, 6, 1]


@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 17, 32, 64, 100, 256, 1000, 1024])
def test_partition_property_and_python_model(orc, n):
    rng = np.random.default_rng(n)
    for trial in range(20):
        if trial % 3 == 0:  # many exact ties
            vals = f32_to_bf16(rng.integers(0, 4, n).astype(np.float32))
        else:
            vals = f32_to_bf16(rng.standard_normal(n).astype(np.float32))
        kth = int(rng.integers(0, n))
        idx = orc.argpartition_bf16(vals, kth)
        assert sorted(idx.tolist()) == list(range(n))
        keys = _keys(vals)
        kk = [keys[i] for i in idx]
        assert all(x < kk[kth] for x in kk[:kth]) and all(kk[kth] < x for x in kk[kth + 1:])
        want, _ = nth_element(keys, kth)
        assert [i for _, i in want] == idx.tolist(), (n, trial, kth)


def test_ranges_of_three_or_fewer_come_back_sorted(orc):
    for n in (1, 2, 3):
        for perm in np.random.default_rng(n).permuted(np.tile(np.arange(n), (6, 1)), axis=1):
            v = f32_to_bf16(perm.astype(np.float32))
            for kth in range(n):
                assert orc.argpartition_bf16(v, kth).tolist() == np.argsort(perm, kind="stable").tolist()


@pytest.mark.parametrize("n,k", [(64, 8), (256, 8), (256, 1), (1000, 16), (1024, 64)])
def test_adversarial_rows_reach_the_heap_selection(orc, n, k):
    """Ranks from the lazily-deciding comparator make every partition unbalanced, so the
    library switches to its heap selection; the oracle, the Python restatement and the
    partition property agree there too."""
    ranks = orc.adversarial_ranks(n, n - k)
    assert sorted(ranks.tolist()) == list(range(n))
    keys = [(int(r), i) for i, r in enumerate(ranks)]
    want, used_heap = nth_element(keys, n - k)
    assert used_heap
    vals = f32_to_bf16(ranks.astype(np.float32))  # bf16 holds integer ranks exactly up to 256
    if n <= 256:
        assert orc.argpartition_bf16(vals, n - k).tolist() == [i for _, i in want]


def test_routing_slice_is_the_argpartition_slice(orc):
    """route_topk's indices = argpartition_slice of its own probabilities (Python model)."""
    rng = np.random.default_rng(5)
    for E, k in ((32, 4), (256, 8), (70, 3), (1024, 64)):
        logits = f32_to_bf16((rng.standard_normal((6, E)) * 0.9).astype(np.float32))
        logits[3:] = f32_to_bf16(np.round(bf16_to_f32(logits[3:]) * 2) / 2)
        idx, _, p = orc.route_topk(logits, k, True, with_probabilities=True)
        for t in range(6):
            assert idx[t].tolist() == argpartition_slice(bf16_to_f32(p[t]).tolist(), k), (E, k, t)
