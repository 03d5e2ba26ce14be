"""Expert pages loaded from safetensors into HIP memory (GPU): the device bytes equal the host
read, and blocks whose routed arrays come from the loaded pages reproduce the resident block
bit for bit (resident fused gate/up, and a streamed page of separate gate/up with its slot map).
"""
import dataclasses

import numpy as np
import pytest
import torch

from astronomical_amd import configs as CF
from astronomical_amd import ops
from astronomical_amd import pages as P
from astronomical_amd import synthetic as S
from paged_util import slot_map
from pages_util import PREFIX, write_checkpoint

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    root = str(tmp_path_factory.mktemp("gpu_ckpt"))
    L = S.make_layer(CF.C0, 0, keep_separate=True)
    wm = write_checkpoint(root, {0: (L.gate, L.up, L.down)})
    return L, P.build_quantized_expert_layer_plan(root, wm, PREFIX.format(0))


def _host(a):
    if isinstance(a, np.ndarray):
        return a
    return ops.u32_to_numpy(a) if a.dtype == torch.int32 else ops.bf16_to_numpy(a)


def _same(dev_aff, host_aff, what):
    for d, h in ((dev_aff.w, host_aff.w), (dev_aff.scales, host_aff.scales), (dev_aff.biases, host_aff.biases)):
        assert np.array_equal(_host(d), h), what


def _dev_layer(L):
    Ld = ops.to_device(dataclasses.replace(L, gate=None, up=None))
    return Ld


def test_device_load_equals_host_load(ckpt):
    L, plan = ckpt
    ids = [0, 3, 4, 5, 17, 31]
    host = P.load_quantized_expert_page(plan, ids, device=None)
    hostf = P.load_quantized_expert_page(plan, ids, device=None, fuse_gate_up=True)
    staging = torch.empty(1 << 20, dtype=torch.uint8).pin_memory()  # 1 MiB: many staging fills
    for st in (None, staging):
        dev = P.load_quantized_expert_page(plan, ids, device="cuda", staging=st)
        for name in ("gate", "up", "down"):
            _same(getattr(dev, name), getattr(host, name), f"{name} staging={st is not None}")
        assert dev.bytes_read == host.bytes_read
        devf = P.load_quantized_expert_page(plan, ids, device="cuda", fuse_gate_up=True, staging=st)
        _same(devf.gate_up, hostf.gate_up, f"fused staging={st is not None}")
        _same(devf.down, hostf.down, f"fused down staging={st is not None}")


@pytest.mark.parametrize("T", [16, 4, 1])
def test_block_from_resident_checkpoint(ckpt, T):
    L, plan = ckpt
    page = P.load_resident_expert_layer(plan, "cuda")
    assert page.gate_up is not None
    Ld = _dev_layer(L)
    Lf = dataclasses.replace(Ld, gate_up=page.gate_up, down=page.down)
    x = ops._bf16_dev(S.make_tokens(CF.C0, T, step=T))
    y_ref = ops.bf16_to_numpy(ops.MoeBlock(Ld)(x))
    y = ops.bf16_to_numpy(ops.MoeBlock(Lf)(x))
    assert np.array_equal(y, y_ref), f"T={T}"


def test_block_from_streamed_page(ckpt):
    L, plan = ckpt
    T = 16  # T * k = 64: the sorted path
    x = ops._bf16_dev(S.make_tokens(CF.C0, T))
    Ld = _dev_layer(L)
    res = ops.MoeBlock(Ld)
    y_res = ops.bf16_to_numpy(res(x))
    used = np.unique(res.trace(T)["indices"])
    spare = [e for e in range(L.num_experts) if e not in set(used.tolist())][:3]
    ids = sorted(used.tolist() + spare)
    page = P.load_quantized_expert_page(plan, ids, device="cuda")
    assert np.array_equal(page.slot_of_expert, slot_map(L.num_experts, ids))
    PL = dataclasses.replace(Ld, gate_up=None, gate=page.gate, up=page.up, down=page.down,
                             slot_of_expert=ops._u32_dev(page.slot_of_expert))
    blk = ops.MoeBlock(PL)
    y = ops.bf16_to_numpy(blk(x))
    assert blk.trace(T)["missing_slots"] == 0
    assert np.array_equal(y, y_res)
