"""The oracle's decoder step (residual add + RMS norm around the block) and Laguna's sigmoid
router (CPU): pinned by the reference's router KATs, float64 closed forms and invariants."""
import math

import numpy as np
import pytest

from astronomical_amd import configs as CF
from astronomical_amd import synthetic as S
from astronomical_amd.layout import bf16_to_f32, f32_to_bf16
from moe_testutil import ulp_distance


def _bf(a):
    return f32_to_bf16(np.asarray(a, np.float32))


def _sig(v):
    return 1.0 / (1.0 + math.exp(-v))


# ------------------------------------------------------------------ Laguna router KATs

def test_laguna_bias_only_selects_and_original_scores_are_gathered(orc):
    """laguna_hermetic/routing.rs:8-21: expert 0 wins only through the bias; its weight stays 0.5."""
    idx, sc = orc.laguna_route(_bf([[0.0, 2.0, -2.0, 0.5]]), 2, np.array([2, 0, 0, 0], np.float32), 0.0, False)
    assert idx.tolist() == [[0, 1]]
    assert abs(sc[0, 0] - _sig(0.0)) < 1e-6 and abs(sc[0, 1] - _sig(2.0)) < 1e-6


def test_laguna_ties_go_to_the_lower_expert(orc):
    """laguna_hermetic/routing.rs:23-29."""
    idx, _ = orc.laguna_route(_bf([[0.0, 0.0, -4.0]]), 1, None, 0.0, False)
    assert idx.tolist() == [[0]]


def test_laguna_softcap_before_sigmoid(orc):
    """laguna_hermetic/routing.rs:31-44: a positive cap bounds the logit to c * tanh(l / c)."""
    _, raw = orc.laguna_route(_bf([[30.0, 0.0]]), 1, None, 0.0, False)
    _, capped = orc.laguna_route(_bf([[30.0, 0.0]]), 1, None, 2.0, False)
    assert raw[0, 0] > capped[0, 0]
    assert abs(capped[0, 0] - _sig(2.0 * math.tanh(15.0))) < 1e-6


def test_laguna_normalisation(orc):
    """laguna_hermetic/routing.rs:46-58 and direct_mlx/laguna/routing.rs:63-122."""
    _, raw = orc.laguna_route(_bf([[1.0, 0.0, -1.0]]), 2, None, 0.0, False)
    _, nrm = orc.laguna_route(_bf([[1.0, 0.0, -1.0]]), 2, None, 0.0, True)
    assert abs(float(nrm.sum()) - 1.0) < 1e-6
    assert abs(nrm[0, 0] - raw[0, 0] / raw.sum()) < 1e-6
    idx, sc = orc.laguna_route(_bf([[0.0, 2.0, -2.0, 0.5]]), 2, np.array([2, 0, 0, 0], np.float32), 0.0, True)
    s0, s1 = _sig(0.0), _sig(2.0)
    assert idx.tolist() == [[0, 1]]
    assert abs(sc[0, 0] - s0 / (s0 + s1)) < 1e-6 and abs(sc[0, 1] - s1 / (s0 + s1)) < 1e-6


def test_laguna_rejects_invalid_geometry(orc):
    """laguna_hermetic/routing.rs:61-66 (k > E, negative cap)."""
    with pytest.raises(RuntimeError):
        orc.laguna_route(_bf([[0.0, 0.0]]), 3)
    with pytest.raises(RuntimeError):
        orc.laguna_route(_bf([[0.0, 0.0]]), 1, None, -1.0)


@pytest.mark.parametrize("softcap", [0.0, 3.0])
def test_laguna_matches_float64_brute_force(orc, softcap):
    rng = np.random.default_rng(11)
    T, E, k = 9, 96, 6
    lg = _bf(rng.standard_normal((T, E)) * 3.0)
    bias = (rng.standard_normal(E) * 0.3).astype(np.float32)
    idx, sc = orc.laguna_route(lg, k, bias, softcap, True)
    l64 = bf16_to_f32(lg).astype(np.float64)
    if softcap:
        l64 = np.tanh(l64 / softcap) * softcap
    s64 = 1.0 / (1.0 + np.exp(-l64))
    sel = s64 + bias.astype(np.float64)
    for t in range(T):
        order = sorted(range(E), key=lambda e: (-sel[t, e], e))[:k]
        assert idx[t].tolist() == order
        want = s64[t, order] / s64[t, order].sum()
        assert np.allclose(sc[t], want, rtol=2e-6, atol=0)


# ------------------------------------------------------------------ RMS norm and the decoder step

def _row_norm64(r, w, eps):
    r = bf16_to_f32(r).astype(np.float64)
    inv = 1.0 / np.sqrt(np.mean(r * r, axis=-1, keepdims=True) + eps)
    return bf16_to_f32(w).astype(np.float64) * r * inv


def test_rms_norm_float64_closed_form(orc):
    rng = np.random.default_rng(3)
    T, H = 6, 2048
    h = _bf(rng.standard_normal((T, H)) * 2.0)
    w = _bf(1.0 + 0.1 * rng.standard_normal(H))
    r, n = orc.add_rms_norm(h, w, 1e-6)
    assert np.array_equal(r, h)
    want = f32_to_bf16(_row_norm64(h, w, 1e-6).astype(np.float32))
    # two bf16 roundings (x * inv, then w * that): at most 2 ulp from the exact value
    assert ulp_distance(n, want).max() <= 2 and np.mean(ulp_distance(n, want) == 0) > 0.5


def test_rms_norm_invariants(orc):
    rng = np.random.default_rng(4)
    H = 1024
    ones = _bf(np.ones(H))
    h = _bf(rng.standard_normal((4, H)))
    _, n = orc.add_rms_norm(h, ones, 0.0)
    ms = np.mean(bf16_to_f32(n).astype(np.float64) ** 2, axis=1)
    assert np.allclose(ms, 1.0, rtol=1e-2)  # unit RMS without a weight
    # a zero row stays zero (eps > 0 keeps the normaliser finite)
    _, n0 = orc.add_rms_norm(np.zeros((1, H), np.uint16), ones, 1e-6)
    assert not np.any(bf16_to_f32(n0))
    # eps much larger than mean(r^2): n = r / sqrt(eps) (eps inside the root)
    _, nb = orc.add_rms_norm(h, ones, 1e6)
    assert ulp_distance(nb, _bf(bf16_to_f32(h) / 1000.0)).max() <= 1
    # the mean, not the sum: a row repeated twice normalises to the same values
    hh = np.concatenate([h, h], axis=1)
    _, n2 = orc.add_rms_norm(hh, _bf(np.ones(2 * H)), 1e-6)
    _, n1 = orc.add_rms_norm(h, ones, 1e-6)
    assert ulp_distance(n2[:, :H], n1).max() <= 1


def test_residual_add_then_norm(orc):
    rng = np.random.default_rng(5)
    h = _bf(rng.standard_normal((3, 512)))
    a = _bf(rng.standard_normal((3, 512)))
    w = _bf(np.ones(512))
    r, n = orc.add_rms_norm(h, w, 1e-6, a)
    assert np.array_equal(r, _bf(bf16_to_f32(h) + bf16_to_f32(a)))
    _, n_of_r = orc.add_rms_norm(r, w, 1e-6)
    assert np.array_equal(n, n_of_r)


def test_decoder_ffn_is_the_composition(orc):
    L = S.make_layer(CF.C0)
    rng = np.random.default_rng(6)
    h = _bf(rng.standard_normal((16, CF.C0.hidden)))
    a = _bf(rng.standard_normal((16, CF.C0.hidden)) * 0.5)
    w = _bf(1.0 + 0.05 * rng.standard_normal(CF.C0.hidden))
    out, r = orc.decoder_ffn_forward(L, h, w, 1e-6, a)
    r2, n = orc.add_rms_norm(h, w, 1e-6, a)
    y = orc.moe_block_forward(L, n)
    assert np.array_equal(r, r2)
    assert np.array_equal(out, _bf(bf16_to_f32(r2) + bf16_to_f32(y)))
