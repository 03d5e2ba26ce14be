"""astro_moe_block_forward_no_alloc (the block on the library's static per-GPU scratch, for
callers that cannot allocate) against astro_moe_block_forward with a caller workspace, through
the C ABI: bit-identical outputs on two calls in a row, the second with fewer tokens (the
scratch keeps the first call's contents), on the decode path and the sorted path; and the
size limit."""
import ctypes as C

import numpy as np
import pytest

from astronomical_amd import configs as CF
from astronomical_amd import synthetic as S

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

SCRATCH_BYTES = 32 << 20  # ASTRO_MOE_STATIC_SCRATCH_BYTES


@pytest.fixture(scope="module")
def ops():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    from astronomical_amd import ops as O
    O._lib.lib()
    return O


def _no_alloc(ops, blk, x):
    x2 = x.contiguous().view(torch.bfloat16).reshape(-1, blk.weights.hidden)
    y = torch.empty_like(x2)
    ops._lib.call("astro_moe_block_forward_no_alloc", C.byref(blk._struct), ops._ptr(x2), x2.shape[0],
                  ops._ptr(y), ops._stream(blk.device))
    return y


@pytest.mark.parametrize("first,second", [(8, 1), (256, 96)])
def test_no_alloc_matches_the_workspace_entry_point(ops, first, second):
    L = S.make_layer(CF.C1)
    blk = ops.MoeBlock(ops.to_device(L))
    for T in (first, second):
        x = ops._bf16_dev(S.make_tokens(CF.C1, T, step=T))
        want = ops.bf16_to_numpy(blk(x))
        got = ops.bf16_to_numpy(_no_alloc(ops, blk, x))
        torch.cuda.synchronize()
        assert np.array_equal(got, want), (first, second, T)


def test_no_alloc_rejects_calls_beyond_the_static_scratch(ops):
    L = S.make_layer(CF.C1)
    blk = ops.MoeBlock(ops.to_device(L))
    T = 2048
    assert blk.workspace_bytes(T) > SCRATCH_BYTES
    x = torch.zeros(T, L.hidden, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ops._lib.AstroMoeError) as err:
        _no_alloc(ops, blk, x)
    assert err.value.status == ops._lib.WORKSPACE_TOO_SMALL
    assert f"allowed_bytes={SCRATCH_BYTES}" in err.value.message
    # the largest token count that fits still runs and matches
    T = 1
    while blk.workspace_bytes(2 * T) <= SCRATCH_BYTES:
        T *= 2
    x = ops._bf16_dev(S.make_tokens(CF.C1, T))
    assert np.array_equal(ops.bf16_to_numpy(_no_alloc(ops, blk, x)), ops.bf16_to_numpy(blk(x)))
