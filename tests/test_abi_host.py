"""The C-ABI library loads, exports every symbol the header declares, and rejects invalid
arguments with the reference's messages — host-side only, no kernel runs (CPU)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "astro_moe.h")


@pytest.fixture(scope="module")
def L():
    from astronomical_amd import _lib
    return _lib


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(astro_(?:moe|synth)_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported(L):
    lib = L.lib()
    names = _declared()
    assert len(names) >= 20
    for n in names:
        assert hasattr(lib, n), n
    # and the binding declares exactly those
    assert sorted(L.EXPORTS) == names
    assert lib.astro_moe_abi_version() == 6


def test_invert_assignment_order_host_entry_point(L):
    from astronomical_amd import ops
    assert ops.invert_assignment_order([1, 3, 5, 4, 2, 0]) == [5, 0, 4, 1, 3, 2]
    assert ops.invert_assignment_order([]) == []
    with pytest.raises(L.AstroMoeError, match="duplicate slot"):
        ops.invert_assignment_order([0, 0])
    with pytest.raises(L.AstroMoeError, match="out-of-range slot"):
        ops.invert_assignment_order([0, 2])


def test_route_validation_messages(L):
    lib = L.lib()
    rc = lib.astro_moe_route_topk(None, 1, 4, 5, 1, None, None, None)
    assert rc == L.INVALID_ARGUMENT
    assert "selected expert count must be positive and no larger than the router dimension" in \
        lib.astro_moe_last_error().decode()
    assert lib.astro_moe_route_topk(None, 1, 4, 0, 1, None, None, None) == L.INVALID_ARGUMENT
    assert lib.astro_moe_route_topk(None, 1, 2048, 8, 1, None, None, None) == L.UNSUPPORTED


def test_sort_rejects_more_than_1024_experts(L):
    lib = L.lib()
    need = C.c_size_t()
    assert lib.astro_moe_sort_workspace_bytes(16, 1025, C.byref(need)) == L.UNSUPPORTED
    assert "at most 1024 experts" in lib.astro_moe_last_error().decode()
    assert lib.astro_moe_sort_workspace_bytes(16, 1024, C.byref(need)) == 0


def _affine(bits=4, group=64, E=2, out=8, inp=128):
    from astronomical_amd._lib import Affine
    return Affine(1, 1, 1, E, out, inp, bits, group)  # fake non-null pointers: never dereferenced


def test_gather_qmm_validation_messages(L):
    lib = L.lib()
    w = _affine(bits=7)
    assert lib.astro_moe_gather_qmm(None, None, 1, C.byref(w), None, 0, None, None, 0, None) == L.INVALID_ARGUMENT
    assert "affine bit width must be 2, 3, 4, 5, 6, or 8" in lib.astro_moe_last_error().decode()
    w = _affine(group=16)
    assert lib.astro_moe_gather_qmm(None, None, 1, C.byref(w), None, 0, None, None, 0, None) == L.INVALID_ARGUMENT
    assert "affine group size must be 32, 64, or 128" in lib.astro_moe_last_error().decode()
    w = _affine(bits=5, group=32, inp=64)
    assert lib.astro_moe_gather_qmm(None, None, 1, C.byref(w), None, 0, None, None, 0, None) == L.UNSUPPORTED
    w = _affine(bits=4, group=64, inp=96)
    assert lib.astro_moe_gather_qmm(None, None, 1, C.byref(w), None, 0, None, None, 0, None) == L.INVALID_ARGUMENT
    assert "affine scale and bias shapes do not match the packed weight shape" in lib.astro_moe_last_error().decode()


def test_workspace_too_small_carries_the_active_memory_marker(L):
    """error_handling.rs:81-122 parses this marker into ActiveMemoryLimitExceeded."""
    from astronomical_amd import configs as CF
    from astronomical_amd import synthetic as S
    from astronomical_amd.ops import layer_struct
    import torch
    Lw = S.make_layer(CF.C0)
    # host tensors stand in for device pointers: validation never dereferences them
    Lt = Lw.map(lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16 if a.dtype == np.uint16 else np.int32)))
    s = layer_struct(Lt)
    lib = L.lib()
    need = C.c_size_t()
    assert lib.astro_moe_workspace_bytes(C.byref(s), 16, C.byref(need)) == 0
    assert need.value > 0
    rc = lib.astro_moe_block_forward(C.byref(s), C.c_void_p(8), 16, C.c_void_p(8), C.c_void_p(8), 100, None)
    assert rc == L.WORKSPACE_TOO_SMALL
    msg = lib.astro_moe_last_error().decode()
    m = re.search(r"ASTRONOMICAL_MLX_ACTIVE_MEMORY_LIMIT_EXCEEDED (.*)$", msg)
    assert m, msg
    fields = dict(f.split("=") for f in m.group(1).split())
    assert set(fields) == {"active_bytes", "allocation_bytes", "allowed_bytes"}
    assert int(fields["allocation_bytes"]) == need.value and int(fields["allowed_bytes"]) == 100
    # geometry errors come before any device work
    s.top_k = 40
    assert lib.astro_moe_workspace_bytes(C.byref(s), 16, C.byref(need)) == L.INVALID_ARGUMENT


def test_decoder_step_rejects_a_residual_output_aliasing_its_inputs(L):
    """The fused decode step writes r while other workgroups still read the hidden states and
    the attention output, so r may not overlap either (checked on the host, before any launch)."""
    from astronomical_amd import configs as CF
    from astronomical_amd import synthetic as S
    from astronomical_amd.ops import layer_struct
    import torch
    Lw = S.make_layer(CF.C0)
    Lt = Lw.map(lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16 if a.dtype == np.uint16 else np.int32)))
    s = layer_struct(Lt)
    lib = L.lib()
    need = C.c_size_t()
    T, H = 1, Lw.hidden
    assert lib.astro_moe_decoder_ffn_workspace_bytes(C.byref(s), T, C.byref(need)) == 0
    hidden, attn, out = 1 << 20, 1 << 24, 1 << 28  # fake addresses, never dereferenced
    for r in (hidden, hidden + 64, attn, attn - 2 * T * H + 2):
        rc = lib.astro_moe_decoder_ffn_forward(C.byref(s), C.c_void_p(hidden), C.c_void_p(attn), C.c_void_p(8),
                                               1e-6, T, C.c_void_p(out), C.c_void_p(r), C.c_void_p(8),
                                               need.value, None)
        assert rc == L.INVALID_ARGUMENT, r
        assert "residual output must not overlap" in lib.astro_moe_last_error().decode()
