"""The multi-token QMV of MTP target-verification windows on the GPU: every output row bit-equal
to the one-token projection of its own row (the reference's test,
direct_mlx/qwen3_5/target_verification_quantized_linear.rs:21-166), against the oracle to the
FP bar, the bf16 small-batch quantized matmul bit-equal to it, and the block's decode path
token-local the way verification windows need (resident_execution.rs:161-162)."""
import numpy as np
import pytest
import torch

from astronomical_amd import configs as CF
from astronomical_amd import synthetic as S
from verify_util import FALLBACK, FALLBACK_F32, SUPPORTED, random_inputs, reference_inputs, rel_l2, ulps

pytestmark = pytest.mark.gpu

# FP bar for one rounding to bf16 / binary16 after fp32 accumulation
REL_L2_TOL = 1e-2
MEDIAN_ULP_TOL = 2.0


@pytest.fixture(scope="module")
def ops():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    from astronomical_amd import ops as O
    O._lib.lib()
    return O


def _dt(f16):
    return torch.float16 if f16 else torch.bfloat16


def _dev(a, f16):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint16).view(np.int16)).cuda().view(_dt(f16))


def _host(t):
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _dev_weights(w, f16):
    codes = torch.from_numpy(np.ascontiguousarray(np.asarray(w.w)[0]).view(np.int32)).cuda()
    return codes, _dev(np.asarray(w.scales)[0], f16), _dev(np.asarray(w.biases)[0], f16)


def _project(ops, x, w, f16):
    codes, s, b = _dev_weights(w, f16)
    return ops.qwen3_5_target_verification_quantized_linear(_dev(x, f16), codes, s, b, w.group_size, w.bits)


def _check_token_local(ops, x, w, f16, whole):
    codes, s, b = _dev_weights(w, f16)
    xd = _dev(x, f16)
    for t in range(x.shape[1]):
        one = ops.qwen3_5_target_verification_quantized_linear(xd[:, t:t + 1].contiguous(), codes, s, b,
                                                               w.group_size, w.bits)
        assert np.array_equal(_host(one.projected_activations)[:, 0], whole[:, t]), f"token {t}"


def _check_oracle(orc, x, w, f16, got, what):
    want = orc.verification_quantized_linear(x, w, f16=f16)
    u = ulps(got, want)
    stats = dict(rel_l2=rel_l2(got, want, f16), median_ulp=float(np.median(u)), max_ulp=int(u.max()))
    assert stats["rel_l2"] <= REL_L2_TOL and stats["median_ulp"] <= MEDIAN_ULP_TOL, (what, stats)


@pytest.mark.parametrize("geo", SUPPORTED + FALLBACK[1:], ids=lambda g: f"T{g.tokens}K{g.input_dimension}"
                         f"N{g.output_dimension}{'f16' if g.f16 else 'bf16'}b{g.bits}g{g.group_size}")
@pytest.mark.parametrize("batch", [1, 2])
def test_reference_geometries_are_token_local(ops, orc, geo, batch):
    x, w = reference_inputs(geo, batch)
    proj = _project(ops, x, w, geo.f16)
    want_dispatch = (ops.TargetVerificationProjectionDispatch.OPTIMIZED_METAL if geo in SUPPORTED
                     else ops.TargetVerificationProjectionDispatch.TOKEN_LOCAL_MLX_FALLBACK)
    assert proj.dispatch == want_dispatch
    whole = _host(proj.into_projected_activations())
    assert whole.shape == (batch, geo.tokens, geo.output_dimension)
    _check_token_local(ops, x, w, geo.f16, whole)
    _check_oracle(orc, x, w, geo.f16, whole, geo)


def test_unsupported_widths_and_dtypes_raise(ops):
    x, w = reference_inputs(FALLBACK[0])  # 6-bit codes
    with pytest.raises(ops.AstroMoeError) as e:
        _project(ops, x, w, False)
    assert e.value.status == ops._lib.UNSUPPORTED
    g = FALLBACK_F32
    x32 = torch.zeros(1, g.tokens, g.input_dimension, dtype=torch.float32, device="cuda")
    codes = torch.zeros(g.output_dimension, g.input_dimension * g.bits // 32, dtype=torch.int32, device="cuda")
    s = torch.zeros(g.output_dimension, g.input_dimension // g.group_size, dtype=torch.float32, device="cuda")
    with pytest.raises(ops.AstroMoeError) as e:
        ops.qwen3_5_target_verification_quantized_linear(x32, codes, s, s, g.group_size, g.bits)
    assert e.value.status == ops._lib.UNSUPPORTED


@pytest.mark.parametrize("bits,f16,group", [(4, False, 64), (4, True, 32), (5, False, 64), (5, True, 128),
                                            (8, False, 32), (8, True, 64)])
@pytest.mark.parametrize("batch,tokens,K,N", [(1, 4, 2048, 1000), (3, 8, 1024, 272), (1, 1, 4096, 300),
                                              (2, 7, 512, 129)])
def test_random_codes_match_oracle_and_are_token_local(ops, orc, bits, f16, group, batch, tokens, K, N):
    print(f"verify qmv bits={bits} f16={f16} g={group} B={batch} T={tokens} K={K} N={N}", flush=True)
    rng = np.random.default_rng(bits * 1000 + K + N)
    x, w = random_inputs(rng, batch, tokens, K, N, bits, group, f16)
    whole = _host(_project(ops, x, w, f16).projected_activations)
    _check_oracle(orc, x, w, f16, whole, (bits, f16, group, batch, tokens, K, N))
    _check_token_local(ops, x, w, f16, whole)


@pytest.mark.parametrize("bits,f16,group,batch,tokens,K,N", [
    (4, False, 128, 1, 3, 128, 17),   # one ring stage; one group per row (scalar affine staging)
    (4, True, 64, 2, 2, 384, 1),      # K not a multiple of 256 (4-step stages), a single output row
    (5, False, 32, 1, 5, 640, 40),    # 20 groups per row (scalar staging), 8-token fragment
    (8, True, 128, 1, 12, 1152, 33),  # 16-token fragment, 9 groups per row
])
def test_edge_geometries_match_oracle_and_are_token_local(ops, orc, bits, f16, group, batch, tokens, K, N):
    print(f"verify qmv edge bits={bits} f16={f16} g={group} B={batch} T={tokens} K={K} N={N}", flush=True)
    rng = np.random.default_rng(K + N)
    x, w = random_inputs(rng, batch, tokens, K, N, bits, group, f16)
    whole = _host(_project(ops, x, w, f16).projected_activations)
    _check_oracle(orc, x, w, f16, whole, (bits, f16, group, batch, tokens, K, N))
    _check_token_local(ops, x, w, f16, whole)


@pytest.mark.parametrize("bits", [4, 8])
def test_small_batch_quantized_matmul_equals_verification(ops, bits):
    """quantized_matmul_affine of each row alone == the verification projection of the window."""
    rng = np.random.default_rng(bits)
    x, w = random_inputs(rng, 1, 6, 2048, 512, bits, 64, False)
    whole = _host(_project(ops, x, w, False).projected_activations)[0]
    wd = w.map(lambda a: torch.from_numpy(np.ascontiguousarray(a).view(
        np.int32 if np.asarray(a).dtype == np.uint32 else np.int16)).cuda())
    wd = wd.map(lambda t: t.view(torch.bfloat16) if t.dtype == torch.int16 else t)
    xd = _dev(x[0], False)
    batch = _host(ops.quantized_matmul_affine(xd, wd))
    assert np.array_equal(batch, whole)
    for t in range(x.shape[1]):
        assert np.array_equal(_host(ops.quantized_matmul_affine(xd[t:t + 1].contiguous(), wd))[0], whole[t])


@pytest.fixture(scope="module")
def c1_block(ops):
    return ops.MoeBlock(ops.to_device(S.make_layer(CF.C1)))


@pytest.mark.parametrize("T", [2, 4, 8, 13])
def test_block_verification_window_is_token_local(ops, c1_block, T):
    """A verification window through the block: row t equals the one-token block of row t,
    also where the window's assignments reach the sorted threshold (8 x 8 = 64) or span
    several decode pieces (13 tokens)."""
    x = S.make_tokens(CF.C1, T)
    whole = _host(c1_block.target_verification_forward(ops._bf16_dev(x)))
    for t in range(T):
        assert np.array_equal(_host(c1_block(ops._bf16_dev(x[t:t + 1])))[0], whole[t]), f"token {t} of {T}"


def test_block_verification_window_matches_oracle(ops, orc, c1_block):
    """The unsorted combine at A = 64 against the oracle's one-token blocks (on the device's
    router logits, as the other block tests)."""
    from moe_testutil import assert_bf16_close
    L = S.make_layer(CF.C1)
    x = S.make_tokens(CF.C1, 8)
    ws = torch.empty(1 << 26, dtype=torch.uint8, device="cuda")
    got = _host(c1_block.target_verification_forward(ops._bf16_dev(x), workspace=ws))
    logits = c1_block.trace(8, workspace=ws)["logits"]  # one piece of 8 tokens
    want = np.concatenate([orc.moe_block_forward(L, x[t:t + 1], logits_override=logits[t:t + 1])
                           for t in range(8)])
    assert_bf16_close(got, want, "c1 verification window of 8")


@pytest.mark.parametrize("T", [2, 4])
def test_block_decode_below_the_sorted_threshold_is_token_local(ops, c1_block, T):
    """Below 64 assignments the production path is unsorted too, hence token-local."""
    x = S.make_tokens(CF.C1, T)
    whole = _host(c1_block(ops._bf16_dev(x)))
    for t in range(T):
        assert np.array_equal(_host(c1_block(ops._bf16_dev(x[t:t + 1])))[0], whole[t]), f"token {t} of {T}"


def test_block_verification_window_keeps_the_unsorted_combine_at_top_64(ops, orc):
    """top_k = 64 leaves the decode kernels (k <= 8), so the window runs one token at a time
    through the grouped-GEMM path with 64 assignments per token; the verification contract
    (resident_execution.rs:146-208) still asks for the unsorted reduction there: the device's
    sparse output equals the oracle's unsorted weighted sum of the device's own expert outputs
    bit for bit, and y is within the FP bar of it."""
    from moe_testutil import assert_bf16_close
    cfg = CF.C0.with_(name="c0_k64", experts=128, top_k=64)
    L = S.make_layer(cfg)
    blk = ops.MoeBlock(ops.to_device(L))
    x = S.make_tokens(cfg, 3)
    ws = torch.empty(1 << 24, dtype=torch.uint8, device="cuda")
    got = _host(blk.target_verification_forward(ops._bf16_dev(x), workspace=ws))
    tr = blk.trace(1, workspace=ws)  # the last piece: token 2 alone
    eo = tr["expert_out_sorted"][tr["inverse_order"]].reshape(1, 64, -1)
    want_sparse = orc.unsorted_weighted_sum(eo, tr["scores"])
    assert np.array_equal(tr["sparse"], want_sparse)
    assert np.array_equal(got[2:3], want_sparse)
    sorted_sparse = orc.sorted_weighted_sum(tr["expert_out_sorted"], tr["inverse_order"], tr["scores"])
    assert not np.array_equal(sorted_sparse, want_sparse)  # the two roundings differ here
    assert_bf16_close(got[2:3], orc.moe_block_forward(L, x[2:3], logits_override=tr["logits"]),
                      "k=64 verification token")
    for t in range(3):  # token-local: each row equals its one-token window
        one = _host(blk.target_verification_forward(ops._bf16_dev(x[t:t + 1])))
        assert np.array_equal(one[0], got[t]), t
