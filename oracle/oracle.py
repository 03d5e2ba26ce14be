"""ctypes wrapper of the CPU oracle (liboracle_moe.so) — TEST INFRASTRUCTURE ONLY.

Loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker
or the timed CPU baseline; the product path never imports it.  Arrays are numpy:
bf16 as uint16 bit patterns, packed weights as uint32.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# ASTRO_ORACLE_LIB names another build of the same sources (the sanitizer build of the tests)
_LIB_PATH = os.environ.get("ASTRO_ORACLE_LIB") or os.path.join(_HERE, "liboracle_moe.so")

ERRORS = {0: "ok", 1: "invalid geometry", 2: "unsupported", 3: "duplicate slot",
          4: "out-of-range slot", 5: "missing slot"}


class OracleError(RuntimeError):
    def __init__(self, code: int, what: str):
        super().__init__(f"{what}: {ERRORS.get(code, code)}")
        self.code = code


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


class _Affine(C.Structure):
    _fields_ = [("w", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p),
                ("experts", C.c_int32), ("out_features", C.c_int32),
                ("in_features", C.c_int32), ("bits", C.c_int32), ("group_size", C.c_int32)]


class _Layer(C.Structure):
    _fields_ = [("hidden", C.c_int32), ("num_experts", C.c_int32), ("top_k", C.c_int32),
                ("intermediate", C.c_int32), ("shared_intermediate", C.c_int32),
                ("normalize_top_k", C.c_int32), ("router_w", C.c_void_p),
                ("router_q", _Affine), ("router_bias", C.c_void_p),
                ("gate_up", _Affine), ("gate", _Affine), ("up", _Affine), ("down", _Affine),
                ("shared_gate", _Affine), ("shared_up", _Affine), ("shared_down", _Affine),
                ("shared_expert_gate", _Affine)]


class _Trace(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "logits", "probabilities", "indices", "scores", "sorted_order", "inverse_order",
        "sorted_ids", "expert_offsets", "activated", "expert_out", "sparse", "shared_out",
        "shared_gate_logits")] + [("used_sorted_path", C.c_int32)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            if os.environ.get("ASTRO_ORACLE_LIB"):
                raise RuntimeError(f"ASTRO_ORACLE_LIB={_LIB_PATH} does not exist")
            build()
        L = C.CDLL(_LIB_PATH)
        vp, i32, i64 = C.c_void_p, C.c_int32, C.c_int64
        L.orc_f32_to_bf16.argtypes = [C.c_float]
        L.orc_f32_to_bf16.restype = C.c_uint16
        L.orc_expf.argtypes = [C.c_float]
        L.orc_expf.restype = C.c_float
        L.orc_set_threads.argtypes = [C.c_int]
        L.orc_get_threads.restype = C.c_int
        L.orc_router_logits.argtypes = [vp, vp, i32, i32, i32, vp]
        L.orc_route_topk.argtypes = [vp, i32, i32, i32, i32, vp, vp, vp]
        L.orc_argpartition_bf16.argtypes = [vp, i32, i32, vp]
        L.orc_argpartition_bf16.restype = None
        L.orc_adversarial_ranks.argtypes = [i32, i32, vp]
        L.orc_adversarial_ranks.restype = None
        L.orc_sort_assignments.argtypes = [vp, i32, i32, vp, vp, vp, vp]
        L.orc_invert_assignment_order.argtypes = [vp, i32, vp]
        L.orc_dequantize.argtypes = [C.POINTER(_Affine), i32, vp]
        L.orc_qmm.argtypes = [vp, i32, C.POINTER(_Affine), i32, vp]
        L.orc_verification_quantized_linear.argtypes = [vp, i32, C.POINTER(_Affine), i32, vp]
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_gather_qmm.argtypes = [vp, vp, i32, C.POINTER(_Affine), vp, vp]
        L.orc_swiglu.argtypes = [vp, vp, i64, vp]
        L.orc_sorted_weighted_sum.argtypes = [vp, vp, vp, i32, i32, i32, vp]
        L.orc_unsorted_weighted_sum.argtypes = [vp, vp, i32, i32, i32, vp]
        L.orc_combine_shared.argtypes = [vp, vp, vp, i32, i32, vp]
        L.orc_moe_block_forward.argtypes = [C.POINTER(_Layer), vp, i32, vp, vp, C.POINTER(_Trace)]
        L.orc_add_rms_norm.argtypes = [vp, vp, vp, C.c_float, i32, i32, vp, vp]
        L.orc_laguna_route.argtypes = [vp, i32, i32, i32, vp, C.c_float, i32, vp, vp]
        L.orc_decoder_ffn_forward.argtypes = [C.POINTER(_Layer), vp, vp, vp, C.c_float, i32, vp, vp]
        for f in ("orc_route_topk", "orc_sort_assignments", "orc_invert_assignment_order",
                  "orc_dequantize", "orc_qmm", "orc_gather_qmm", "orc_moe_block_forward",
                  "orc_add_rms_norm", "orc_laguna_route", "orc_decoder_ffn_forward"):
            getattr(L, f).restype = C.c_int
        _lib = L
    return _lib


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def _p(a):
    return None if a is None else a.ctypes.data


def _c(a, dtype):
    return np.ascontiguousarray(np.asarray(a, dtype=dtype))


def _check(rc, what):
    if rc:
        raise OracleError(rc, what)


def _affine(w, keep):
    if w is None:
        return _Affine()
    arrs = (_c(w.w, np.uint32), _c(w.scales, np.uint16), _c(w.biases, np.uint16))
    keep.extend(arrs)
    return _Affine(_p(arrs[0]), _p(arrs[1]), _p(arrs[2]), arrs[0].shape[0], arrs[0].shape[1],
                   arrs[0].shape[2] * 32 // w.bits, w.bits, w.group_size)


def expf(x: float) -> float:
    return lib().orc_expf(float(x))


def f32_to_bf16_scalar(x: float) -> int:
    return lib().orc_f32_to_bf16(float(x))


def router_logits(x, w):
    x, w = _c(x, np.uint16), _c(w, np.uint16)
    T, H = x.shape
    E = w.shape[0]
    out = np.empty((T, E), np.uint16)
    lib().orc_router_logits(_p(x), _p(w), T, H, E, _p(out))
    return out


def route_topk(logits, k, normalize=True, with_probabilities=False):
    lg = _c(logits, np.uint16)
    T, E = lg.reshape(-1, lg.shape[-1]).shape
    idx = np.empty((T, k), np.uint32)
    sc = np.empty((T, k), np.uint16)
    pr = np.empty((T, E), np.uint16) if with_probabilities else None
    _check(lib().orc_route_topk(_p(lg), T, E, k, int(bool(normalize)), _p(idx), _p(sc), _p(pr)),
           "route experts")
    return (idx, sc, pr) if with_probabilities else (idx, sc)


def argpartition_bf16(values, kth):
    """MLX CPU argpartition of one bf16 row: the index vector after libstdc++'s
    std::nth_element at kth with the (value, index) comparator."""
    v = _c(values, np.uint16).reshape(-1)
    idx = np.empty(v.shape[0], np.uint32)
    lib().orc_argpartition_bf16(_p(v), v.shape[0], int(kth), _p(idx))
    return idx


def adversarial_ranks(n, kth):
    """A permutation of 0..n-1 that drives std::nth_element(kth) into its heap selection
    (McIlroy's lazily-decided comparator; see argpartition.cc)."""
    r = np.empty(n, np.int32)
    lib().orc_adversarial_ranks(int(n), int(kth), _p(r))
    return r


def sort_assignments(ids, experts):
    ids = _c(ids, np.uint32).reshape(-1)
    A = ids.shape[0]
    so, inv, sid = (np.empty(A, np.uint32) for _ in range(3))
    off = np.empty(experts + 1, np.uint32)
    _check(lib().orc_sort_assignments(_p(ids), A, experts, _p(so), _p(inv), _p(sid), _p(off)),
           "sort expert assignments")
    return so, inv, sid, off


def invert_assignment_order(sorted_order):
    so = _c(sorted_order, np.uint32).reshape(-1)
    inv = np.empty_like(so)
    _check(lib().orc_invert_assignment_order(_p(so), so.shape[0], _p(inv)),
           "invert assignment order")
    return inv


def dequantize(w, expert=0):
    keep = []
    a = _affine(w, keep)
    out = np.empty((a.out_features, a.in_features), np.uint16)
    _check(lib().orc_dequantize(C.byref(a), expert, _p(out)), "dequantize")
    return out


def qmm(x, w, expert=0):
    keep = []
    a = _affine(w, keep)
    x = _c(x, np.uint16)
    M = x.shape[0]
    y = np.empty((M, a.out_features), np.uint16)
    _check(lib().orc_qmm(_p(x), M, C.byref(a), expert, _p(y)), "quantized matmul")
    return y


def verification_quantized_linear(x, w, f16=False):
    """x [..., K] bf16 (or binary16 when f16) bits; w AffineWeights with one expert whose
    scales/biases share x's dtype -> [..., N] of that dtype."""
    keep = []
    a = _affine(w, keep)
    x = _c(x, np.uint16)
    lead = x.shape[:-1]
    x2 = np.ascontiguousarray(x.reshape(-1, x.shape[-1]))
    y = np.empty((x2.shape[0], a.out_features), np.uint16)
    _check(lib().orc_verification_quantized_linear(_p(x2), x2.shape[0], C.byref(a), int(bool(f16)), _p(y)),
           "target-verification quantized linear")
    return y.reshape(*lead, a.out_features)


def f32_to_f16_scalar(x: float) -> int:
    return int(lib().orc_f32_to_f16(float(x)))


def f16_to_f32_scalar(h: int) -> float:
    return float(lib().orc_f16_to_f32(int(h)))


def gather_qmm(x, w, ids, x_rows=None):
    keep = []
    a = _affine(w, keep)
    x = _c(x, np.uint16)
    ids = _c(ids, np.uint32).reshape(-1)
    xr = None if x_rows is None else _c(x_rows, np.uint32).reshape(-1)
    rows = ids.shape[0]
    y = np.empty((rows, a.out_features), np.uint16)
    _check(lib().orc_gather_qmm(_p(x), _p(xr), rows, C.byref(a), _p(ids), _p(y)), "gather_qmm")
    return y


def swiglu(gate, up):
    g, u = _c(gate, np.uint16), _c(up, np.uint16)
    out = np.empty_like(g)
    lib().orc_swiglu(_p(g), _p(u), g.size, _p(out))
    return out


def sorted_weighted_sum(sorted_out, inverse_order, scores):
    so = _c(sorted_out, np.uint16)
    inv = _c(inverse_order, np.uint32)
    sc = _c(scores, np.uint16)
    T, k = sc.shape
    D = so.shape[-1]
    y = np.empty((T, D), np.uint16)
    lib().orc_sorted_weighted_sum(_p(so), _p(inv), _p(sc), T, k, D, _p(y))
    return y


def unsorted_weighted_sum(out, scores):
    o = _c(out, np.uint16)
    sc = _c(scores, np.uint16)
    T, k = sc.shape
    D = o.shape[-1]
    y = np.empty((T, D), np.uint16)
    lib().orc_unsorted_weighted_sum(_p(o), _p(sc), T, k, D, _p(y))
    return y


def combine_shared(sparse, shared_out, gate_logits):
    sp, so = _c(sparse, np.uint16), _c(shared_out, np.uint16)
    z = _c(gate_logits, np.uint16).reshape(-1)
    T, D = sp.shape
    y = np.empty_like(sp)
    lib().orc_combine_shared(_p(sp), _p(so), _p(z), T, D, _p(y))
    return y


def layer_struct(L, keep):
    """Build the orc_layer view of a MoeLayerWeights holding numpy arrays."""
    s = _Layer()
    s.hidden, s.num_experts, s.top_k = L.hidden, L.num_experts, L.top_k
    s.intermediate, s.shared_intermediate = L.intermediate, L.shared_intermediate
    s.normalize_top_k = int(bool(L.normalize_top_k))
    if L.router_w is not None:
        r = _c(L.router_w, np.uint16)
        keep.append(r)
        s.router_w = _p(r)
    s.router_q = _affine(L.router_q, keep)
    if L.router_bias is not None:
        rb = _c(L.router_bias, np.uint16)
        keep.append(rb)
        s.router_bias = _p(rb)
    s.gate_up = _affine(L.gate_up, keep)
    s.gate = _affine(L.gate, keep)
    s.up = _affine(L.up, keep)
    s.down = _affine(L.down, keep)
    s.shared_gate = _affine(L.shared_gate, keep)
    s.shared_up = _affine(L.shared_up, keep)
    s.shared_down = _affine(L.shared_down, keep)
    s.shared_expert_gate = _affine(L.shared_expert_gate, keep)
    return s


def moe_block_forward(L, x, logits_override=None, trace=False):
    """Whole block; returns y (bf16 [T, H]) or (y, dict of intermediates)."""
    keep = []
    s = layer_struct(L, keep)
    x = _c(x, np.uint16)
    T = x.shape[0]
    H, E, k, I = L.hidden, L.num_experts, L.top_k, L.intermediate
    A = T * k
    y = np.empty((T, H), np.uint16)
    lo = None if logits_override is None else _c(logits_override, np.uint16)
    tr = None
    bufs = {}
    if trace:
        bufs = dict(
            logits=np.empty((T, E), np.uint16), probabilities=np.empty((T, E), np.uint16),
            indices=np.empty((T, k), np.uint32), scores=np.empty((T, k), np.uint16),
            sorted_order=np.zeros(A, np.uint32), inverse_order=np.zeros(A, np.uint32),
            sorted_ids=np.zeros(A, np.uint32), expert_offsets=np.zeros(E + 1, np.uint32),
            activated=np.empty((A, I), np.uint16), expert_out=np.empty((A, H), np.uint16),
            sparse=np.empty((T, H), np.uint16))
        if L.shared_intermediate:
            bufs["shared_out"] = np.empty((T, H), np.uint16)
            bufs["shared_gate_logits"] = np.empty(T, np.uint16)
        tr = _Trace(**{n: _p(a) for n, a in bufs.items()})
    _check(lib().orc_moe_block_forward(C.byref(s), _p(x), T, _p(lo), _p(y),
                                       C.byref(tr) if tr is not None else None),
           "moe block forward")
    if trace:
        bufs["used_sorted_path"] = bool(tr.used_sorted_path)
        return y, bufs
    return y


# ------------------------------------------------------------------- the decoder step and Laguna's router

def add_rms_norm(h, w, eps, a=None):
    """(r, n): r = bf16(h + a) (h when a is None), n = RMS norm of r with weight w (bf16 [T, H])."""
    h = _c(h, np.uint16)
    T, H = h.shape
    a = None if a is None else _c(a, np.uint16)
    w = _c(w, np.uint16)
    r = np.empty((T, H), np.uint16)
    n = np.empty((T, H), np.uint16)
    _check(lib().orc_add_rms_norm(_p(h), _p(a), _p(w), float(eps), T, H, _p(r), _p(n)), "add rms norm")
    return r, n


def decoder_ffn_forward(L, h, w, eps, a=None):
    """(out, r): out = bf16(r + MoE(rms_norm(r))), r = bf16(h + a)."""
    keep = []
    s = layer_struct(L, keep)
    h = _c(h, np.uint16)
    T = h.shape[0]
    a = None if a is None else _c(a, np.uint16)
    w = _c(w, np.uint16)
    out = np.empty_like(h)
    r = np.empty_like(h)
    _check(lib().orc_decoder_ffn_forward(C.byref(s), _p(h), _p(a), _p(w), float(eps), T, _p(out), _p(r)),
           "decoder feed-forward step")
    return out, r


def laguna_route(logits, k, bias=None, softcap=0.0, normalize=True):
    """(indices uint32 [T, k], fp32 scores [T, k]) of the CPU selection order."""
    lg = _c(logits, np.uint16)
    T, E = lg.shape
    b = None if bias is None else _c(bias, np.float32)
    idx = np.empty((T, k), np.uint32)
    sc = np.empty((T, k), np.float32)
    _check(lib().orc_laguna_route(_p(lg), T, E, k, _p(b), float(softcap), int(normalize), _p(idx), _p(sc)),
           "laguna route")
    return idx, sc


# ------------------------------------------------------------------- paged callers
# Compositions of the stage functions above, restating the reference's paged graphs.

SLOT_ABSENT = 0xFFFFFFFF


def remap_expert_page_slots(ids, page_slot_by_global_expert_id):
    """qwen3_5_moe_remap_expert_page_slots (split_page_route.rs:79-105): slots = take(map, ids),
    refused when a routed expert has no slot (or lies past the map)."""
    ids = _c(ids, np.uint32)
    m = _c(page_slot_by_global_expert_id, np.uint32).reshape(-1)
    if np.any(ids >= m.shape[0]) or np.any(m[np.minimum(ids, m.shape[0] - 1)] == SLOT_ABSENT):
        raise OracleError(5, "remap expert page slots: a routed expert is absent from the streamed page manifest")
    return m[ids]


def add_bf16(a, b):
    """MLX add of two bf16 arrays: the fp32 sum rounded to nearest even."""
    f = (bf16_to_f32(a) + bf16_to_f32(b)).astype(np.float32)
    return f32_to_bf16(f)


def bf16_to_f32(h):
    return (_c(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f):
    """Round-to-nearest-even of fp32 to bf16 bit patterns (quiet NaN for NaN inputs)."""
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def streamed_sparse_forward(x, gate, up, down, slots, scores):
    """forward_moe_with_streamed_weights (paged_execution.rs:207-281) for T tokens with kk
    assignments each: slots / scores [T, kk] (page slots, bf16 scores); gate, up, down are the
    page's arrays (slot-indexed AffineWeights).  Sorted by slot iff T*kk >= 64 (routing.rs:13,
    sort_expert_assignments over the page's slot count), then up, gate, SwiGLU, down and the
    sorted or unsorted weighted sum.  Returns the sparse output bf16 [T, H]."""
    slots = _c(slots, np.uint32)
    scores = _c(scores, np.uint16)
    T, kk = scores.shape
    A = T * kk
    flat = slots.reshape(-1)
    rows = np.repeat(np.arange(T, dtype=np.uint32), kk)  # assignment a reads token a // kk
    capacity = int(np.asarray(down.w).shape[0])
    if A >= 64:
        so, inv, sid, _ = sort_assignments(flat, capacity)
        ids, x_rows = sid, rows[so]
    else:
        inv, ids, x_rows = None, flat, rows
    up_out = gather_qmm(x, up, ids, x_rows=x_rows)
    gate_out = gather_qmm(x, gate, ids, x_rows=x_rows)
    act = swiglu(gate_out, up_out)
    out = gather_qmm(act, down, ids)
    if A >= 64:
        return sorted_weighted_sum(out, inv, scores)
    return unsorted_weighted_sum(out.reshape(T, kk, -1), scores)


def paged_shared_combine(L, x, sparse):
    """combine_paged_sparse_and_shared_outputs (paged_execution.rs:337-374): the shared
    expert of L on x, then the shared combine (sparse unchanged without a shared expert)."""
    if not L.shared_intermediate:
        return _c(sparse, np.uint16)
    g = qmm(x, L.shared_gate)
    u = qmm(x, L.shared_up)
    o = qmm(swiglu(g, u), L.shared_down)
    z = qmm(x, L.shared_expert_gate).reshape(-1)
    return combine_shared(sparse, o, z)


def split_paged_forward(L, x, indices, scores, retained_positions, missing_positions,
                        retained_page, retained_map, missing_page, missing_map):
    """forward_moe_split_paged_with_performance_attribution (paged_execution.rs:147-205) for
    one decode token: each side takes its assignment positions (split_page_route.rs:28-55),
    remaps them to its page's slots and runs the streamed sparse graph; the two partial
    outputs are added in bf16, then the shared combine.  Pages are (gate, up, down)."""
    ids = _c(indices, np.uint32).reshape(-1)
    sc = _c(scores, np.uint16).reshape(-1)
    parts = []
    for pos, page, m in ((retained_positions, retained_page, retained_map),
                         (missing_positions, missing_page, missing_map)):
        pos = np.asarray(pos, dtype=np.int64)
        slots = remap_expert_page_slots(ids[pos], m)
        parts.append(streamed_sparse_forward(x, page[0], page[1], page[2], slots.reshape(1, -1),
                                             sc[pos].reshape(1, -1)))
    return paged_shared_combine(L, x, add_bf16(parts[0], parts[1]))
