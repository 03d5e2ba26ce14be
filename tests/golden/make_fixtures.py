"""Writes the committed golden fixtures (data only):

* c0_block.npz — config c0 (H1024 E32 k4 I256, 4-bit g64, 16 tokens): the seeded inputs
  (x; the weights are regenerated from the seeded generator and pinned by checksum) and
  the oracle's outputs of every stage.
* route_ties.npz — router logits with exact ties at the top-k boundary (E=256 k=8 and
  E=32 k=4) and the expected ids: the slice of MLX's CPU argpartition of each row's
  probabilities (oracle.argpartition_bf16, libstdc++'s std::nth_element with the (value,
  index) comparator), i.e. the k largest (probability, index) keys in that order.

Run: python tests/golden/make_fixtures.py   (needs the oracle library: make -C oracle)
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "oracle")]

import oracle  # noqa: E402
from astronomical_amd import configs as CF  # noqa: E402
from astronomical_amd import synthetic as S  # noqa: E402
from astronomical_amd.layout import f32_to_bf16  # noqa: E402


def layer_checksum(L) -> str:
    h = hashlib.sha256()
    for a in (L.router_w, L.gate_up.w, L.gate_up.scales, L.gate_up.biases, L.down.w,
              L.down.scales, L.down.biases):
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def make_c0():
    L = S.make_layer(CF.C0)
    x = S.make_tokens(CF.C0, 16)
    y, tr = oracle.moe_block_forward(L, x, trace=True)
    out = {k: v for k, v in tr.items() if isinstance(v, np.ndarray)}
    out.update(x=x, y=y, used_sorted_path=np.array(tr["used_sorted_path"]),
               layer_sha256=np.array(layer_checksum(L)))
    np.savez_compressed(os.path.join(HERE, "c0_block.npz"), **out)


def make_ties():
    rng = np.random.default_rng(20261201)
    cases = {}
    for E, k in ((256, 8), (32, 4)):
        T = 64
        lg = (rng.standard_normal((T, E)) * 0.9).astype(np.float32)
        for t in range(T):
            order = np.argsort(-lg[t])
            # tie the k-th and (k+1)-th largest, and for odd t a block of four around it
            span = 4 if t % 2 else 2
            lg[t, order[k - span // 2:k + span // 2]] = lg[t, order[k - 1]]
        logits = f32_to_bf16(lg)
        _, _, p = oracle.route_topk(logits, k, True, with_probabilities=True)
        expected = np.stack([oracle.argpartition_bf16(row, E - k)[E - k:] for row in p]).astype(np.uint32)
        cases[f"logits_E{E}_k{k}"] = logits
        cases[f"indices_E{E}_k{k}"] = expected
    np.savez_compressed(os.path.join(HERE, "route_ties.npz"), **cases)


if __name__ == "__main__":
    oracle.lib()
    make_c0()
    make_ties()
    print("fixtures written to", HERE)
