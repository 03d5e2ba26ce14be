"""The decoder step around the block and Laguna's sigmoid router on the GPU, against the oracle:
RMS norm and routing bit-exact (the kernels and the oracle share the summation order and
the exp), the whole feed-forward step to the FP bar on the device's own logits."""
import numpy as np
import pytest
import torch

from astronomical_amd import configs as CF
from astronomical_amd import ops
from astronomical_amd import synthetic as S
from astronomical_amd.layout import bf16_to_f32, f32_to_bf16
from moe_testutil import assert_bf16_close

pytestmark = pytest.mark.gpu


def _bf(a):
    return f32_to_bf16(np.asarray(a, np.float32))


@pytest.mark.parametrize("T,H,with_attn", [(5, 2048, True), (1, 1024, False), (3, 4096, True), (2, 96, True)])
def test_add_rms_norm_bit_exact(orc, T, H, with_attn):
    rng = np.random.default_rng(T * H)
    h = _bf(rng.standard_normal((T, H)) * 1.5)
    a = _bf(rng.standard_normal((T, H))) if with_attn else None
    w = _bf(1.0 + 0.1 * rng.standard_normal(H))
    r_ref, n_ref = orc.add_rms_norm(h, w, 1e-6, a)
    r = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    n = ops.rms_norm(ops._bf16_dev(h), ops._bf16_dev(w), 1e-6,
                     attention_out=None if a is None else ops._bf16_dev(a), residual_out=r)
    assert np.array_equal(ops.bf16_to_numpy(r), r_ref)
    assert np.array_equal(ops.bf16_to_numpy(n), n_ref)


@pytest.mark.parametrize("cfg,T,router_bits", [(CF.C0, 16, None), (CF.C1, 1, None), (CF.C1, 8, None),
                                               (CF.C0, 40, None), (CF.C1, 1, 4), (CF.C1, 4, 8)])
def test_decoder_ffn_forward(orc, cfg, T, router_bits):
    """The fused decode step (the router kernel forms r and n itself) also with an affine
    router."""
    L = S.make_layer(cfg, router_bits=router_bits)
    rng = np.random.default_rng(T)
    h = _bf(rng.standard_normal((T, cfg.hidden)))
    a = _bf(rng.standard_normal((T, cfg.hidden)) * 0.5)
    w = _bf(1.0 + 0.05 * rng.standard_normal(cfg.hidden))
    blk = ops.MoeBlock(ops.to_device(L))
    n_ws = blk.workspace_bytes(T) + 3 * ((T * cfg.hidden * 2 + 255) // 256 * 256) + 256
    ws = torch.empty(n_ws, dtype=torch.uint8, device="cuda")
    r = torch.empty((T, cfg.hidden), dtype=torch.bfloat16, device="cuda")
    out = ops.bf16_to_numpy(blk.decoder_feed_forward(ops._bf16_dev(h), ops._bf16_dev(w), 1e-6,
                                                     attention_out=ops._bf16_dev(a), residual=r, workspace=ws))
    r_ref, n_ref = orc.add_rms_norm(h, w, 1e-6, a)
    assert np.array_equal(ops.bf16_to_numpy(r), r_ref)
    tr = blk.trace(T, workspace=ws)  # the block's workspace leads the step's
    y_ref, ref = orc.moe_block_forward(L, n_ref, logits_override=tr["logits"], trace=True)
    assert np.array_equal(tr["indices"], ref["indices"])
    out_ref = _bf(bf16_to_f32(r_ref) + bf16_to_f32(y_ref))
    assert_bf16_close(out, out_ref, f"{cfg.name} T={T}")


def test_laguna_router_kats():
    """The reference's router KATs (laguna_hermetic/routing.rs:8-58) on the device."""
    def route(lg, k, bias=None, cap=0.0, norm=False):
        i, s = ops.route_laguna_experts(ops._bf16_dev(_bf(lg)), k,
                                        None if bias is None else torch.tensor(bias, device="cuda"), cap, norm)
        return ops.u32_to_numpy(i).tolist(), s.cpu().numpy()
    i, s = route([[0.0, 2.0, -2.0, 0.5]], 2, [2.0, 0.0, 0.0, 0.0])
    assert i == [[0, 1]] and abs(s[0, 0] - 0.5) < 1e-6 and abs(s[0, 1] - 1 / (1 + np.exp(-2.0))) < 1e-6
    assert route([[0.0, 0.0, -4.0]], 1)[0] == [[0]]
    assert route([[30.0, 0.0]], 1)[1][0, 0] > route([[30.0, 0.0]], 1, cap=2.0)[1][0, 0]
    assert abs(route([[1.0, 0.0, -1.0]], 2, norm=True)[1].sum() - 1.0) < 1e-6


@pytest.mark.parametrize("T,E,k,bias,cap,norm,ties", [
    (7, 256, 8, True, 0.0, True, False), (33, 128, 10, False, 2.0, True, True), (1, 64, 1, True, 30.0, False, False),
    (5, 1000, 16, True, 0.0, False, True), (9, 4, 4, False, 0.0, True, False)])
def test_laguna_router_bit_exact(orc, T, E, k, bias, cap, norm, ties):
    rng = np.random.default_rng(E + k)
    lg = rng.standard_normal((T, E)) * 2.0
    if ties:
        lg = np.round(lg * 2) / 2  # many equal scores: ties go to the lower expert id
    lg = _bf(lg)
    b = (rng.standard_normal(E) * 0.2).astype(np.float32) if bias else None
    i_ref, s_ref = orc.laguna_route(lg, k, b, cap, norm)
    i, s = ops.route_laguna_experts(ops._bf16_dev(lg), k, None if b is None else torch.from_numpy(b).cuda(), cap, norm)
    assert np.array_equal(ops.u32_to_numpy(i), i_ref)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
