"""ctypes binding of include/astro_moe.h (libastro_moe.so, built in-tree).

The product path is the HIP library only: if it is missing, loading raises — there is
no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libastro_moe.so")
# A host-only build of the library's host code (the sanitizer build the CPU tests run under)
# stands in for it when ASTRO_MOE_HOST_LIB names one; its absent entry points stay unbound, so
# calling one raises AttributeError.
HOST_LIB = os.environ.get("ASTRO_MOE_HOST_LIB")

OK, INVALID_ARGUMENT, UNSUPPORTED, WORKSPACE_TOO_SMALL, HIP_ERROR = 0, 1, 2, 3, 4
STAGES = ("router", "route", "sort", "gate_up", "down", "shared", "combine")


class AstroMoeError(RuntimeError):
    """A failed C-ABI call: status code and the library's thread-local message."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status
        self.message = message


class Affine(C.Structure):
    _fields_ = [("w", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p),
                ("experts", C.c_int32), ("out_features", C.c_int32), ("in_features", C.c_int32),
                ("bits", C.c_int32), ("group_size", C.c_int32)]


class Layer(C.Structure):
    _fields_ = [("hidden", C.c_int32), ("num_experts", C.c_int32), ("top_k", C.c_int32),
                ("intermediate", C.c_int32), ("shared_intermediate", C.c_int32),
                ("normalize_top_k", C.c_int32), ("router_w", C.c_void_p), ("router_q", Affine),
                ("router_bias", C.c_void_p), ("gate_up", Affine), ("gate", Affine), ("up", Affine),
                ("down", Affine), ("shared_gate", Affine), ("shared_up", Affine),
                ("shared_down", Affine), ("shared_expert_gate", Affine),
                ("slot_of_expert", C.c_void_p)]


class WorkspaceView(C.Structure):
    _fields_ = [("total_bytes", C.c_size_t), ("sorted_path", C.c_int32)] + [
        (n, C.c_size_t) for n in ("logits", "indices", "scores", "sorted_order", "inverse_order",
                                  "sorted_ids", "expert_offsets", "activated", "activated_ld", "expert_out",
                                  "sparse", "shared_out", "shared_gate_logits", "expert_slots",
                                  "missing_slots", "tile_expert", "tile_row0", "tile_count", "max_tiles",
                                  "activated_paired")]


PATH_MAX = 1024
DTYPES = ("BOOL", "I8", "U8", "F8_E4M3", "F8_E5M2", "I16", "U16", "F16", "BF16", "I32", "U32",
          "F32", "I64", "U64")


class TensorSource(C.Structure):
    _fields_ = [("source_file", C.c_char * PATH_MAX), ("dtype", C.c_int32), ("shape", C.c_int64 * 3),
                ("file_offset", C.c_uint64), ("bytes_per_expert", C.c_uint64), ("file_size", C.c_uint64)]


class ExpertLayerPlan(C.Structure):
    _fields_ = [("src", (TensorSource * 3) * 3), ("expert_capacity", C.c_int32),
                ("bits", C.c_int32 * 3), ("group_size", C.c_int32 * 3), ("gate_up_fusable", C.c_int32),
                ("gate_up_separate_reason", C.c_char * 96)]


class PageInterval(C.Structure):
    _fields_ = [("projection", C.c_int32), ("parameter", C.c_int32), ("expert_start", C.c_int32),
                ("expert_count", C.c_int32), ("first_page_slot", C.c_int32), ("file_offset", C.c_uint64),
                ("byte_count", C.c_uint64), ("virtual_offset", C.c_uint64)]


EXPORTS = {
    "astro_moe_add_rms_norm": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_float, C.c_int32, C.c_int32,
                                C.c_void_p, C.c_void_p, C.c_void_p], C.c_int),
    "astro_moe_decoder_ffn_workspace_bytes": ([C.POINTER(Layer), C.c_int32, C.POINTER(C.c_size_t)], C.c_int),
    "astro_moe_decoder_ffn_forward": ([C.POINTER(Layer), C.c_void_p, C.c_void_p, C.c_void_p, C.c_float,
                                       C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t,
                                       C.c_void_p], C.c_int),
    "astro_moe_route_laguna": ([C.c_void_p, C.c_int32, C.c_int32, C.c_int32, C.c_void_p, C.c_double,
                                C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p], C.c_int),
    "astro_moe_safetensors_tensor": ([C.c_char_p, C.c_char_p, C.POINTER(C.c_int32), C.POINTER(C.c_int32),
                                      C.POINTER(C.c_int64), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)],
                                     C.c_int),
    "astro_moe_build_expert_layer_plan": ([C.c_char_p, C.POINTER(C.c_char_p), C.POINTER(C.c_char_p),
                                           C.c_int32, C.c_char_p, C.POINTER(C.c_int32),
                                           C.POINTER(C.c_int32), C.POINTER(ExpertLayerPlan)], C.c_int),
    "astro_moe_build_expert_page_manifest": ([C.POINTER(ExpertLayerPlan), C.POINTER(C.c_int32), C.c_int32,
                                              C.c_void_p, C.POINTER(PageInterval), C.c_int32,
                                              C.POINTER(C.c_int32), C.POINTER(C.c_uint64)], C.c_int),
    "astro_moe_load_expert_page": ([C.POINTER(ExpertLayerPlan), C.POINTER(C.c_int32), C.c_int32, C.c_int32,
                                    C.POINTER(C.c_void_p), C.c_int32, C.c_void_p, C.c_size_t, C.c_void_p,
                                    C.POINTER(C.c_uint64)], C.c_int),
    # name: (argtypes, restype)
    "astro_moe_remap_expert_slots": ([C.c_void_p, C.c_int32, C.c_void_p, C.c_int32, C.c_void_p,
                                      C.c_void_p, C.c_void_p], C.c_int),
    "astro_moe_gather_assignments": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p,
                                      C.c_void_p, C.c_void_p], C.c_int),
    "astro_moe_streamed_sparse_workspace_bytes": ([C.POINTER(Layer), C.c_int32, C.c_int32,
                                                   C.POINTER(C.c_size_t)], C.c_int),
    "astro_moe_streamed_sparse_forward": ([C.POINTER(Layer), C.c_void_p, C.c_int32, C.c_void_p,
                                           C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p,
                                           C.c_size_t, C.c_void_p], C.c_int),
    "astro_moe_add": ([C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p], C.c_int),
    "astro_moe_selftest_bf16_rounding": ([C.c_void_p, C.c_void_p], C.c_int),
    "astro_moe_last_error": ([], C.c_char_p),
    "astro_moe_abi_version": ([], C.c_int),
    "astro_moe_workspace_bytes": ([C.POINTER(Layer), C.c_int32, C.POINTER(C.c_size_t)], C.c_int),
    "astro_moe_workspace_layout": ([C.POINTER(Layer), C.c_int32, C.POINTER(WorkspaceView)], C.c_int),
    "astro_moe_block_forward": ([C.POINTER(Layer), C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p,
                                 C.c_size_t, C.c_void_p], C.c_int),
    "astro_moe_block_forward_no_alloc": ([C.POINTER(Layer), C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p],
                                         C.c_int),
    "astro_moe_block_forward_attributed": ([C.POINTER(Layer), C.c_void_p, C.c_int32, C.c_void_p,
                                            C.c_void_p, C.c_size_t, C.c_void_p,
                                            C.POINTER(C.c_float)], C.c_int),
    "astro_moe_verification_workspace_bytes": ([C.POINTER(Layer), C.c_int32, C.POINTER(C.c_size_t)], C.c_int),
    "astro_moe_block_forward_verification": ([C.POINTER(Layer), C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p,
                                              C.c_size_t, C.c_void_p], C.c_int),
    "astro_moe_router_logits": ([C.POINTER(Layer), C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p], C.c_int),
    "astro_moe_route_topk": ([C.c_void_p, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_void_p,
                              C.c_void_p, C.c_void_p], C.c_int),
    "astro_moe_sort_workspace_bytes": ([C.c_int32, C.c_int32, C.POINTER(C.c_size_t)], C.c_int),
    "astro_moe_sort_assignments": ([C.c_void_p, C.c_int32, C.c_int32, C.c_void_p, C.c_void_p,
                                    C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p], C.c_int),
    "astro_moe_invert_assignment_order": ([C.c_void_p, C.c_int32, C.c_void_p], C.c_int),
    "astro_moe_gather_qmm_workspace_bytes": ([C.c_int32, C.c_int32, C.POINTER(C.c_size_t)], C.c_int),
    "astro_moe_gather_qmm": ([C.c_void_p, C.c_void_p, C.c_int32, C.POINTER(Affine), C.c_void_p,
                              C.c_int32, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p], C.c_int),
    "astro_moe_quantized_matmul": ([C.c_void_p, C.c_int32, C.POINTER(Affine), C.c_void_p,
                                    C.c_void_p], C.c_int),
    "astro_moe_verification_quantized_linear": ([C.c_void_p, C.c_int32, C.c_int32, C.c_int32,
                                                 C.POINTER(Affine), C.c_int32, C.c_void_p, C.c_void_p],
                                                C.c_int),
    "astro_moe_swiglu": ([C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p], C.c_int),
    "astro_moe_sorted_weighted_sum": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32,
                                       C.c_int32, C.c_void_p, C.c_void_p], C.c_int),
    "astro_moe_unsorted_weighted_sum": ([C.c_void_p, C.c_void_p, C.c_int32, C.c_int32, C.c_int32,
                                         C.c_void_p, C.c_void_p], C.c_int),
    "astro_moe_combine_shared": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32,
                                  C.c_void_p, C.c_void_p], C.c_int),
    "astro_moe_shared_expert_workspace_bytes": ([C.POINTER(Layer), C.c_int32,
                                                 C.POINTER(C.c_size_t)], C.c_int),
    "astro_moe_shared_expert": ([C.POINTER(Layer), C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p,
                                 C.c_void_p, C.c_size_t, C.c_void_p], C.c_int),
    "astro_synth_words": ([C.c_void_p, C.c_int64, C.c_uint64, C.c_void_p], C.c_int),
    "astro_synth_uniform_bf16": ([C.c_void_p, C.c_int64, C.c_uint64, C.c_double, C.c_double,
                                  C.c_void_p], C.c_int),
    "astro_synth_affine_biases": ([C.c_void_p, C.c_void_p, C.c_int64, C.c_uint64, C.c_double,
                                   C.c_double, C.c_void_p], C.c_int),
    "astro_synth_normal_bf16": ([C.c_void_p, C.c_int64, C.c_uint64, C.c_double, C.c_void_p], C.c_int),
    "astro_synth_activations": ([C.c_void_p, C.c_int32, C.c_int32, C.c_uint64, C.c_void_p], C.c_int),
}

_lib = None


def lib():
    """Load libastro_moe.so; raises if it has not been built (no fallback path exists)."""
    global _lib
    if _lib is None:
        path = HOST_LIB or LIB_PATH
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: run __graft_entry__.build() "
                               "(python -m astronomical_amd.build) first")
        L = C.CDLL(path)
        for name, (args, res) in EXPORTS.items():
            f = getattr(L, name, None)
            if f is None and HOST_LIB:
                continue
            if f is None:
                raise RuntimeError(f"{path} does not export {name}: rebuild it")
            f.argtypes = args
            f.restype = res
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != OK:
        msg = lib().astro_moe_last_error().decode(errors="replace")
        raise AstroMoeError(status, msg)


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))
