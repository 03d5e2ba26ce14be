"""The oracle reproduces the committed golden fixtures bit for bit (CPU only)."""
import os

import numpy as np

from astronomical_amd import configs as CF
from astronomical_amd import synthetic as S

from conftest import GOLDEN


def _load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def test_c0_block_fixture_is_reproduced(orc):
    import sys
    sys.path.insert(0, GOLDEN)
    from make_fixtures import layer_checksum
    fx = _load("c0_block.npz")
    L = S.make_layer(CF.C0)
    assert layer_checksum(L) == str(fx["layer_sha256"])
    x = S.make_tokens(CF.C0, 16)
    assert np.array_equal(x, fx["x"])
    y, tr = orc.moe_block_forward(L, x, trace=True)
    assert bool(fx["used_sorted_path"]) and tr["used_sorted_path"]
    for name in ("logits", "probabilities", "indices", "scores", "sorted_order", "inverse_order",
                 "sorted_ids", "expert_offsets", "activated", "expert_out", "sparse"):
        assert np.array_equal(tr[name], fx[name]), name
    assert np.array_equal(y, fx["y"])


def test_route_ties_fixture(orc):
    fx = _load("route_ties.npz")
    for E, k in ((256, 8), (32, 4)):
        idx, _ = orc.route_topk(fx[f"logits_E{E}_k{k}"], k, True)
        assert np.array_equal(idx, fx[f"indices_E{E}_k{k}"])
