"""CPU oracle of the paged callers (paged_execution.rs, split_page_route.rs), pinned against
the resident block: a page holding every routed expert, in any slot order, reproduces the
resident sparse output bit for bit; the slot remap refuses absent experts like the reference;
the bf16 add matches the oracle's scalar fp32 -> bf16 rounding."""
import numpy as np
import pytest

from astronomical_amd import configs as CF
from astronomical_amd import synthetic as S
from astronomical_amd.layout import bf16_to_f32, f32_to_bf16

from moe_testutil import rel_l2
from paged_util import SLOT_ABSENT, page_arrays, slot_map


def test_remap_expert_page_slots(orc):
    m = slot_map(8, [5, 1, 6])
    assert orc.remap_expert_page_slots(np.array([[1, 6], [5, 5]], np.uint32), m).tolist() == [[1, 2], [0, 0]]
    with pytest.raises(orc.OracleError):
        orc.remap_expert_page_slots(np.array([1, 2], np.uint32), m)   # expert 2 has no slot
    with pytest.raises(orc.OracleError):
        orc.remap_expert_page_slots(np.array([9], np.uint32), m)      # past the map
    assert m[2] == SLOT_ABSENT


def test_add_bf16_matches_scalar_rounding(orc):
    rng = np.random.default_rng(3)
    a = f32_to_bf16((rng.standard_normal(4096) * 10 ** rng.uniform(-3, 3, 4096)).astype(np.float32))
    b = f32_to_bf16((rng.standard_normal(4096) * 10 ** rng.uniform(-3, 3, 4096)).astype(np.float32))
    got = orc.add_bf16(a, b)
    want = np.array([orc.f32_to_bf16_scalar(float(np.float32(x) + np.float32(y)))
                     for x, y in zip(bf16_to_f32(a), bf16_to_f32(b))], np.uint16)
    assert np.array_equal(got, want)
    assert np.array_equal(orc.add_bf16(a, b), orc.add_bf16(b, a))


@pytest.mark.parametrize("T", [16, 8])  # A = 64 (sorted path) and 32 (unsorted)
def test_streamed_sparse_equals_resident_sparse(orc, T):
    cfg = CF.C0
    L = S.make_layer(cfg)
    x = S.make_tokens(cfg, T)
    _, tr = orc.moe_block_forward(L, x, trace=True)
    rng = np.random.default_rng(T)
    experts = rng.permutation(L.num_experts)          # every expert, shuffled slots
    gate, up, down = page_arrays(L, experts)
    m = slot_map(L.num_experts, experts)
    slots = orc.remap_expert_page_slots(tr["indices"], m)
    sparse = orc.streamed_sparse_forward(x, gate, up, down, slots, tr["scores"])
    assert np.array_equal(sparse, tr["sparse"])
    # a compact page of just the routed experts gives the same output
    used = np.unique(tr["indices"])
    gate, up, down = page_arrays(L, used[::-1])
    m = slot_map(L.num_experts, used[::-1])
    sparse2 = orc.streamed_sparse_forward(x, gate, up, down, orc.remap_expert_page_slots(tr["indices"], m),
                                          tr["scores"])
    assert np.array_equal(sparse2, tr["sparse"])


def test_split_paged_forward_consistency(orc):
    cfg = CF.C1
    L = S.make_layer(cfg)
    x = S.make_tokens(cfg, 1)
    y_res, tr = orc.moe_block_forward(L, x, trace=True)
    ids = tr["indices"].reshape(-1)
    ret_pos, mis_pos = [0, 2, 5], [1, 3, 4, 6, 7]
    ret_e, mis_e = ids[ret_pos], ids[mis_pos]
    pages = {}
    for name, ex in (("r", list(ret_e) + [int((ids.max() + 1) % L.num_experts)]), ("m", list(mis_e[::-1]))):
        pages[name] = (page_arrays(L, ex), slot_map(L.num_experts, ex))
    y = orc.split_paged_forward(L, x, tr["indices"], tr["scores"], ret_pos, mis_pos,
                                pages["r"][0], pages["r"][1], pages["m"][0], pages["m"][1])
    # the sides swapped give the same sum (the bf16 add is commutative)
    y_sw = orc.split_paged_forward(L, x, tr["indices"], tr["scores"], mis_pos, ret_pos,
                                   pages["m"][0], pages["m"][1], pages["r"][0], pages["r"][1])
    assert np.array_equal(y, y_sw)
    # the split rounds two partial sums instead of one: close to the resident block
    assert rel_l2(y, y_res) < 1e-2
    # a side that routes to an expert its page lacks is refused
    with pytest.raises(orc.OracleError):
        orc.split_paged_forward(L, x, tr["indices"], tr["scores"], ret_pos, mis_pos,
                                pages["m"][0], pages["m"][1], pages["r"][0], pages["r"][1])
