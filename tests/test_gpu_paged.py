"""Paged callers on the HIP path vs the CPU oracle (paged_execution.rs, split_page_route.rs).

A block whose routed arrays are a compact page (slot_of_expert set) routes exactly like the
resident block and sorts by page slot; with every routed expert in the page its output equals
the resident block's bit for bit (same weights, same rows; only the row order of the sorted
buffers changes).  The streamed sparse graph and the split-page decode meet the oracle to the
matmul bar; slot remap, assignment gather and the bf16 add are bit-exact."""
import numpy as np
import pytest

from astronomical_amd import configs as CF
from astronomical_amd import synthetic as S
from astronomical_amd.layout import f32_to_bf16

from moe_testutil import assert_bf16_close
from paged_util import SLOT_ABSENT, page_arrays, paged_layer, slot_map

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ops():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    from astronomical_amd import ops as O
    O._lib.lib()
    return O


def _np(t):
    from astronomical_amd.ops import bf16_to_numpy, u32_to_numpy
    return bf16_to_numpy(t) if t.dtype == torch.bfloat16 else u32_to_numpy(t)


def _bf(a):
    from astronomical_amd.ops import _bf16_dev
    return _bf16_dev(a)


def _u32(a):
    from astronomical_amd.ops import _u32_dev
    return _u32_dev(a)


# T <= 8 at c1 takes the decode kernels (one token: the routed workgroups' own slot ranks; two:
# the in-workgroup table; 4 and 8: the routing kernel's table), larger batches the sorted path
@pytest.mark.parametrize("cfg,T", [(CF.C1, 128), (CF.C0, 16), (CF.C1, 1), (CF.C1, 2), (CF.C1, 4), (CF.C1, 8)])
def test_paged_block(ops, orc, cfg, T):
    L = S.make_layer(cfg)
    x = S.make_tokens(cfg, T)
    res = ops.MoeBlock(ops.to_device(L))
    y_res = _np(res(_bf(x)))
    tr_res = res.trace(T)
    used = np.unique(tr_res["indices"])
    rng = np.random.default_rng(T)
    extra = [e for e in rng.permutation(L.num_experts) if e not in set(used.tolist())][:3]
    experts = rng.permutation(np.concatenate([used, np.array(extra, dtype=used.dtype)]))
    PL = paged_layer(L, experts)
    blk = ops.MoeBlock(ops.to_device(PL))
    y = _np(blk(_bf(x)))
    tr = blk.trace(T)
    what = f"{cfg.name} T={T} paged ({len(experts)} slots)"
    assert tr["missing_slots"] == 0, what
    assert np.array_equal(tr["indices"], tr_res["indices"]) and np.array_equal(tr["scores"], tr_res["scores"]), what
    assert np.array_equal(tr["expert_slots"], PL.slot_of_expert[tr["indices"]]), what
    so, inv, sid, off = orc.sort_assignments(tr["expert_slots"].reshape(-1), len(experts))
    assert np.array_equal(tr["sorted_order"], so) and np.array_equal(tr["inverse_order"], inv), what
    assert np.array_equal(tr["sorted_ids"], sid), what
    if not tr_res["sorted_path"] and T * L.top_k < 64 and T <= 8:
        # the resident block took the decode kernels: compare both with the oracle instead
        y_ref = orc.moe_block_forward(L, x, logits_override=tr["logits"])
        assert_bf16_close(y, y_ref, what)
    else:
        assert np.array_equal(y, y_res), what
    # the paged graph of the oracle on the same routing
    gate, up, down = page_arrays(L, experts)
    sparse_ref = orc.streamed_sparse_forward(x, gate, up, down, tr["expert_slots"], tr["scores"])
    assert_bf16_close(tr["sparse"], sparse_ref, what + " sparse")


@pytest.mark.parametrize("cfg,T", [(CF.C0, 16), (CF.C1, 1), (CF.C1, 4)])
def test_paged_block_missing_expert_counted(ops, cfg, T):
    """Experts absent from the page are counted (the sorted path's remap kernel, or the decode
    kernels' routing publisher)."""
    L = S.make_layer(cfg)
    x = S.make_tokens(cfg, T)
    res = ops.MoeBlock(ops.to_device(L))
    res(_bf(x))
    used = np.unique(res.trace(T)["indices"])
    drop = int(used[0])
    n_drop = int((res.trace(T)["indices"] == drop).sum())
    blk = ops.MoeBlock(ops.to_device(paged_layer(L, used[1:])))
    blk(_bf(x))
    assert blk.trace(T)["missing_slots"] == n_drop
    # the operator API refuses the route like the reference
    ids = torch.tensor(res.trace(T)["indices"].astype(np.int32), device="cuda")
    with pytest.raises(ops.AstroMoeError, match="absent from the streamed page manifest"):
        ops.qwen3_5_moe_remap_expert_page_slots(ids, _u32(slot_map(L.num_experts, used[1:])))


@pytest.mark.parametrize("cfg,T,kk", [(CF.C1, 1, 3), (CF.C1, 16, 8), (CF.C0, 32, 4)])
def test_streamed_sparse_forward(ops, orc, cfg, T, kk):
    L = S.make_layer(cfg)
    x = S.make_tokens(cfg, T)
    rng = np.random.default_rng(T * 31 + kk)
    experts = rng.permutation(L.num_experts)[: max(2 * kk, 24)]
    slots = np.stack([rng.choice(len(experts), size=kk, replace=False) for _ in range(T)]).astype(np.uint32)
    scores = f32_to_bf16(rng.uniform(0.02, 0.4, size=(T, kk)).astype(np.float32))
    gate, up, down = page_arrays(L, experts)
    PL = paged_layer(L, experts)
    got = _np(ops.forward_moe_with_streamed_weights(_bf(x), ops.to_device(PL), _u32(slots), _bf(scores)))
    want = orc.streamed_sparse_forward(x, gate, up, down, slots, scores)
    assert_bf16_close(got, want, f"{cfg.name} streamed T={T} kk={kk}")


def test_split_paged_decode(ops, orc):
    cfg = CF.C1
    L = S.make_layer(cfg)
    x = S.make_tokens(cfg, 1)
    _, tr = orc.moe_block_forward(L, x, trace=True)
    ids = tr["indices"].reshape(-1)
    ret_pos, mis_pos = [0, 2, 5], [1, 3, 4, 6, 7]
    ret_e = list(ids[ret_pos]) + [int((ids.max() + 7) % L.num_experts)]
    mis_e = list(ids[mis_pos][::-1])
    want = orc.split_paged_forward(L, x, tr["indices"], tr["scores"], ret_pos, mis_pos,
                                   page_arrays(L, ret_e), slot_map(L.num_experts, ret_e),
                                   page_arrays(L, mis_e), slot_map(L.num_experts, mis_e))
    dL = ops.to_device(L)
    got = ops.forward_moe_split_paged(_bf(x), dL, ops.to_device(paged_layer(L, ret_e)),
                                      ops.to_device(paged_layer(L, mis_e)), _u32(tr["indices"]),
                                      _bf(tr["scores"]), ret_pos, mis_pos)
    assert_bf16_close(_np(got), want, "split-page decode c1")
    with pytest.raises(ops.AstroMoeError, match="appears more than once"):
        ops.Qwen3_5MoESplitPageRoute.build(_u32(tr["indices"]), _bf(tr["scores"]), [0, 0, 1], [2, 3, 4, 5, 6],
                                           _u32(slot_map(L.num_experts, ret_e)), _u32(slot_map(L.num_experts, mis_e)))


def test_gather_assignments_and_add_bit_exact(ops, orc):
    rng = np.random.default_rng(11)
    ids = rng.integers(0, 256, 64).astype(np.uint32)
    sc = f32_to_bf16(rng.uniform(0, 1, 64).astype(np.float32))
    pos = rng.permutation(64)[:20].astype(np.uint32)
    out_ids = torch.empty(20, dtype=torch.int32, device="cuda")
    out_sc = torch.empty(20, dtype=torch.bfloat16, device="cuda")
    from astronomical_amd._lib import call
    from astronomical_amd.ops import _ptr, _stream
    dids, dsc, dpos = _u32(ids), _bf(sc), _u32(pos)
    call("astro_moe_gather_assignments", _ptr(dids), _ptr(dsc), _ptr(dpos), 20, _ptr(out_ids), _ptr(out_sc), _stream())
    assert np.array_equal(_np(out_ids), ids[pos]) and np.array_equal(_np(out_sc), sc[pos])
    a = f32_to_bf16((rng.standard_normal(10007) * 50).astype(np.float32))
    b = f32_to_bf16((rng.standard_normal(10007) * 0.01).astype(np.float32))
    assert np.array_equal(_np(ops.add(_bf(a), _bf(b))), orc.add_bf16(a, b))
