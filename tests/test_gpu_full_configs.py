"""The block at every configuration's stated size against the CPU oracle, on an MI355X.

c2 (2048 tokens, near-uniform routing) puts 65-96 rows on about half of the experts, so their
rows span a full 64-row tile and a partial one, and the tile table lists the light last tiles
after the heavy ones; c3 (4096 tokens, Zipf-skewed logits) puts
every token on its top expert (64 whole tiles of one expert) and leaves most experts empty;
c4 (512 tokens, 8-bit g32) runs the 8-bit grouped GEMMs at about 32 rows per expert, alone and
as a two-layer residual chain (h <- h + MoE_l(rms_norm(h)), the decoder step of
decoder_layer_forward.rs:111-174).  Bars as in test_gpu_parity: routing and permutation
bit-exact, the combine bit-exact given the stage inputs, projections within rel-L2 1e-2 and a
median of 2 bf16 ulps."""
import ctypes as C

import numpy as np
import pytest

from astronomical_amd import configs as CF
from astronomical_amd import synthetic as S
from astronomical_amd.layout import bf16_to_f32, f32_to_bf16

from moe_testutil import assert_bf16_close
from test_gpu_parity import _check_block, _dev_bf16, _np, ops  # noqa: F401  (fixture)

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


TILE_ROWS = 64  # rows of a grouped-GEMM tile (kGemmBM)


def _tile_checks(tr, what):
    """The tile table covers every sorted row once, in tiles of at most 64 rows of one
    expert, with every tile of more than 32 rows before the smaller last tiles."""
    off = tr["expert_offsets"].astype(np.int64)
    te, tr0 = tr["tile_expert"].astype(np.int64), tr["tile_row0"].astype(np.int64)
    rows = np.minimum(TILE_ROWS, off[te + 1] - tr0)
    assert np.all(rows > 0), what
    covered = np.zeros(int(off[-1]), np.int32)
    for e, r0, n in zip(te, tr0, rows):
        assert off[e] <= r0 < off[e + 1], what
        covered[r0:r0 + n] += 1
    assert np.all(covered == 1), what
    big = rows > TILE_ROWS // 2
    first_small = int(np.argmin(big)) if not big.all() else len(big)
    assert big[:first_small].all() and not big[first_small:].any(), what
    return rows


def test_block_c2_full(ops, orc):
    L = S.make_layer(CF.C1)
    T = 2048
    stats = _check_block(ops, orc, L, S.make_tokens(CF.C2, T), "c2 T=2048")
    blk = ops.MoeBlock(ops.to_device(L))
    blk(_dev_bf16(S.make_tokens(CF.C2, T)))
    tr = blk.trace(T)
    rows = _tile_checks(tr, "c2 tiles")
    counts = np.diff(tr["expert_offsets"][:L.num_experts + 1].astype(np.int64))
    # experts of more than one tile, partial tiles of every size class, and small last tiles
    # ordered after the heavy ones are all exercised
    assert np.sum(counts > TILE_ROWS) >= 64, counts
    assert np.sum(rows == TILE_ROWS) >= 64 and np.sum(rows <= TILE_ROWS // 2) >= 32, rows
    print("c2 full", stats)


def test_block_c2_full_affine_router(ops, orc):
    """c2 with a 4-bit affine router (the certified checkpoints' quantized mlp.gate): the
    router projection runs on the grouped GEMM."""
    L = S.make_layer(CF.C1, router_bits=4)
    stats = _check_block(ops, orc, L, S.make_tokens(CF.C2, 2048), "c2 T=2048 affine router")
    print("c2 full affine router", stats)


def test_block_c3_full(ops, orc):
    L = S.make_layer(CF.C3)
    T = 4096
    x = S.make_tokens(CF.C3, T)
    stats = _check_block(ops, orc, L, x, "c3 T=4096 (Zipf)")
    blk = ops.MoeBlock(ops.to_device(L))
    blk(_dev_bf16(x))
    tr = blk.trace(T)
    _tile_checks(tr, "c3 tiles")
    counts = np.diff(tr["expert_offsets"][:L.num_experts + 1].astype(np.int64))
    assert counts.max() > 1024 and np.sum(counts == 0) >= 100, (counts.max(), np.sum(counts == 0))
    print("c3 full", stats)


def test_block_c4_full(ops, orc):
    L = S.make_layer(CF.C4)
    stats = _check_block(ops, orc, L, S.make_tokens(CF.C4, 512), "c4 T=512 (8-bit g32)")
    print("c4 full", stats)


def test_block_c4_two_layer_chain(ops, orc):
    """Two distinct 8-bit layers chained through the decoder step at 512 tokens
    (h <- h + MoE_l(rms_norm(h))).  Each layer is checked on the device's own input, the
    previous layer's device output: the residual and the RMS norm bit-exact, routing bit-exact
    on the device's router logits, the step's output within the FP bar.  (Fed the oracle's own
    previous output instead, a few tokens of the second layer route differently, as any two
    implementations whose logits differ in the last bit do.)"""
    T, eps = 512, 1e-6
    w = f32_to_bf16(np.ones(CF.C4.hidden, np.float32))
    dev_w = _dev_bf16(w)
    h = S.make_tokens(CF.C4, T, step=3)
    for l in range(2):
        L = S.make_layer(CF.C4, layer=l)
        blk = ops.MoeBlock(ops.to_device(L))
        need = C.c_size_t()
        ops._lib.call("astro_moe_decoder_ffn_workspace_bytes", C.byref(blk._struct), T, C.byref(need))
        ws = torch.empty(need.value, dtype=torch.uint8, device="cuda")
        r_dev = torch.empty(T, CF.C4.hidden, dtype=torch.bfloat16, device="cuda")
        out = _np(blk.decoder_feed_forward(_dev_bf16(h), dev_w, eps, residual=r_dev, workspace=ws))
        tr = blk.trace(T, workspace=ws)
        r_ref, n_ref = orc.add_rms_norm(h, w, eps)
        assert np.array_equal(_np(r_dev), r_ref), l
        y_ref, ref = orc.moe_block_forward(L, n_ref, logits_override=tr["logits"], trace=True)
        assert np.array_equal(tr["indices"], ref["indices"]), l
        assert np.array_equal(tr["inverse_order"], ref["inverse_order"]), l
        want = f32_to_bf16(bf16_to_f32(r_ref) + bf16_to_f32(y_ref))
        stats = assert_bf16_close(out, want, f"c4 chain layer {l}")
        print("c4 chain layer", l, stats)
        h = out
