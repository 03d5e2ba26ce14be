"""Host-side mirror of the reference's MoE operator API over the C ABI.

Function names, argument meaning and error behaviour follow the reference
(crates/model-serving/src/sparse_experts/*.rs, qwen3_5_moe/model/{routing,output_combination}.rs,
crates/runtime-integration/src/mlx_quantized_operations.rs).  Tensors are torch device
tensors used as plain HBM buffers: bf16 as ``torch.bfloat16``, uint32 indices and packed
codes as ``torch.int32`` bit patterns.  Every computation runs in libastro_moe.so on the
tensors' current HIP stream; errors raise ``AstroMoeError`` with the library's message.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from enum import Enum
from typing import Optional, Sequence

import numpy as np
import torch

from . import _lib
from ._lib import AstroMoeError, Affine, Layer, WorkspaceView, call
from .layout import AffineWeights, MoeLayerWeights

MINIMUM_SORTED_EXPERT_ASSIGNMENTS = 64  # routing.rs:13


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream(device=None):
    return C.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _bf16_dev(a, device="cuda") -> torch.Tensor:
    if isinstance(a, torch.Tensor):
        return a.to(device).contiguous().view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16)).to(device).view(torch.bfloat16)


def _u32_dev(a, device="cuda") -> torch.Tensor:
    if isinstance(a, torch.Tensor):
        return a.to(device).contiguous().view(torch.int32)
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(device)


def to_device(L: MoeLayerWeights, device="cuda") -> MoeLayerWeights:
    """Copy a host (numpy) layer to device tensors."""
    def conv(a):
        a = np.asarray(a)
        return _u32_dev(a, device) if a.dtype == np.uint32 else _bf16_dev(a, device)
    return L.map(conv)


def bf16_to_numpy(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def u32_to_numpy(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int32).cpu().numpy().view(np.uint32)


def affine_struct(w: Optional[AffineWeights]) -> Affine:
    if w is None:
        return Affine()
    return Affine(w.w.data_ptr(), w.scales.data_ptr(), w.biases.data_ptr(), int(w.w.shape[0]),
                  int(w.w.shape[1]), int(w.w.shape[2]) * 32 // w.bits, w.bits, w.group_size)


def layer_struct(L: MoeLayerWeights) -> Layer:
    s = Layer()
    s.hidden, s.num_experts, s.top_k = L.hidden, L.num_experts, L.top_k
    s.intermediate, s.shared_intermediate = L.intermediate, L.shared_intermediate
    s.normalize_top_k = int(bool(L.normalize_top_k))
    s.router_w = None if L.router_w is None else L.router_w.data_ptr()
    s.router_q = affine_struct(L.router_q)
    s.router_bias = None if L.router_bias is None else L.router_bias.data_ptr()
    s.gate_up = affine_struct(L.gate_up)
    s.gate = affine_struct(L.gate)
    s.up = affine_struct(L.up)
    s.down = affine_struct(L.down)
    s.shared_gate = affine_struct(L.shared_gate)
    s.shared_up = affine_struct(L.shared_up)
    s.shared_down = affine_struct(L.shared_down)
    s.shared_expert_gate = affine_struct(L.shared_expert_gate)
    s.slot_of_expert = None if L.slot_of_expert is None else L.slot_of_expert.data_ptr()
    return s


# ---------------------------------------------------------------- routing (routing.rs)

def qwen3_5_moe_route_experts(router_logits: torch.Tensor, expert_count_per_token: int,
                              should_normalize_scores: bool):
    """routing.rs:16-48 -> (selected_indices int32[..., k], selected_scores bf16[..., k])."""
    if router_logits.dim() < 2:
        raise AstroMoeError(_lib.INVALID_ARGUMENT, "route Qwen3.5-MoE sparse experts: router "
                            "logits must include token and expert dimensions")
    if router_logits.dtype != torch.bfloat16:
        raise AstroMoeError(_lib.UNSUPPORTED, "route Qwen3.5-MoE sparse experts: the kernels "
                            "take bfloat16 router logits")
    E = router_logits.shape[-1]
    lg = router_logits.contiguous()
    T = lg.numel() // max(E, 1)
    k = int(expert_count_per_token)
    shape = list(lg.shape[:-1]) + [max(k, 0)]
    idx = torch.empty(shape, dtype=torch.int32, device=lg.device)
    sc = torch.empty(shape, dtype=torch.bfloat16, device=lg.device)
    call("astro_moe_route_topk", _ptr(lg), T, E, k, int(bool(should_normalize_scores)), _ptr(idx),
         _ptr(sc), _stream(lg.device))
    return idx, sc


# ------------------------------------------------- sorting (assignment_sort.rs, permutation)

@dataclass
class SortedExpertAssignments:
    """assignment_sort.rs:13-17; the row gather (sorted_states) is fused into
    gather_qmm through ``token_rows`` instead of being materialised."""
    sorted_order: torch.Tensor     # sorted slot -> original slot
    sorted_indices: torch.Tensor   # expert id per sorted slot
    inverse_order: torch.Tensor    # original slot -> sorted slot
    expert_offsets: torch.Tensor   # [E+1]
    expert_count_per_token: int

    @property
    def token_rows(self) -> torch.Tensor:
        return torch.div(self.sorted_order, self.expert_count_per_token, rounding_mode="floor")


def sort_expert_assignments(selected_indices: torch.Tensor, num_experts: int) -> SortedExpertAssignments:
    """assignment_sort.rs:36-97: stable argsort by expert id, its inverse and the sorted ids."""
    ids = selected_indices.contiguous().view(torch.int32)
    if ids.dim() < 1:
        raise AstroMoeError(_lib.INVALID_ARGUMENT, "sort stacked expert assignments: selected "
                            "expert indices must include an expert dimension")
    k = int(ids.shape[-1]) if ids.dim() >= 2 else 1
    A = ids.numel()
    dev = ids.device
    so = torch.empty(A, dtype=torch.int32, device=dev)
    inv = torch.empty(A, dtype=torch.int32, device=dev)
    sid = torch.empty(A, dtype=torch.int32, device=dev)
    off = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    need = C.c_size_t()
    call("astro_moe_sort_workspace_bytes", A, num_experts, C.byref(need))
    ws = torch.empty(max(need.value, 1), dtype=torch.uint8, device=dev)
    call("astro_moe_sort_assignments", _ptr(ids), A, num_experts, _ptr(so), _ptr(inv), _ptr(sid),
         _ptr(off), _ptr(ws), need.value, _stream(dev))
    return SortedExpertAssignments(so, sid, inv, off, k)


def invert_assignment_order(sorted_order: Sequence[int]) -> list:
    """assignment_permutation.rs:10-42 (host)."""
    a = np.ascontiguousarray(np.asarray(sorted_order, dtype=np.uint32))
    out = np.empty_like(a)
    call("astro_moe_invert_assignment_order", C.c_void_p(a.ctypes.data), a.shape[0],
         C.c_void_p(out.ctypes.data))
    return out.tolist()


def gathered_indices_use_sorted_contract(assignments_were_sorted: bool) -> bool:
    """assignment_permutation.rs:44-48."""
    return bool(assignments_were_sorted)


# ------------------------------------------------- gathered projection (gathered_projection.rs)

class ExpertAssignmentOrder(Enum):
    ORIGINAL = 0
    SORTED_BY_EXPERT = 1

    def uses_sorted_indices(self) -> bool:
        return self is ExpertAssignmentOrder.SORTED_BY_EXPERT


def gather_expert_projection(activations: torch.Tensor, projection: AffineWeights,
                             selected_expert_indices: torch.Tensor,
                             assignment_order: ExpertAssignmentOrder = ExpertAssignmentOrder.ORIGINAL,
                             token_rows: Optional[torch.Tensor] = None) -> torch.Tensor:
    """gathered_projection.rs:84-131: out[r] = x[token_rows[r] or r] . deq(W[ids[r]])^T."""
    x = activations.contiguous().view(torch.bfloat16)
    ids = selected_expert_indices.contiguous().view(torch.int32).reshape(-1)
    rows = ids.numel()
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    tr = None if token_rows is None else token_rows.contiguous().view(torch.int32).reshape(-1)
    w = affine_struct(projection)
    out = torch.empty(rows, w.out_features, dtype=torch.bfloat16, device=x.device)
    if K != w.in_features:
        raise AstroMoeError(_lib.INVALID_ARGUMENT, "build affine gather_qmm: activation inner "
                            "dimension does not match the expanded quantized weight input")
    if tr is None and x2.shape[0] != rows:
        raise AstroMoeError(_lib.INVALID_ARGUMENT, "build affine gather_qmm: activation rows "
                            "must match the assignment count when no token rows are given")
    need = C.c_size_t()
    call("astro_moe_gather_qmm_workspace_bytes", rows, w.experts, C.byref(need))
    ws = torch.empty(max(need.value, 1), dtype=torch.uint8, device=x.device)
    call("astro_moe_gather_qmm", _ptr(x2), _ptr(tr), rows, C.byref(w), _ptr(ids),
         int(assignment_order.uses_sorted_indices()), _ptr(out), _ptr(ws), need.value,
         _stream(x.device))
    return out


def quantized_matmul_affine(activations: torch.Tensor, weights: AffineWeights) -> torch.Tensor:
    """mlx_quantized_operations.rs:49-96 (transpose = true)."""
    x = activations.contiguous().view(torch.bfloat16)
    w = affine_struct(weights)
    if x.shape[-1] != w.in_features:
        raise AstroMoeError(_lib.INVALID_ARGUMENT, "build affine quantized matmul: activation "
                            "inner dimension does not match the expanded quantized weight input")
    x2 = x.reshape(-1, x.shape[-1])
    out = torch.empty(x2.shape[0], w.out_features, dtype=torch.bfloat16, device=x.device)
    call("astro_moe_quantized_matmul", _ptr(x2), x2.shape[0], C.byref(w), _ptr(out), _stream(x.device))
    return out.reshape(*x.shape[:-1], w.out_features)


# ------------------------------------------------- MTP target verification (target_verification_quantized_linear.rs)

class TargetVerificationProjectionDispatch(Enum):
    """Qwen3_5TargetVerificationProjectionDispatch (target_verification_quantized_linear.rs:180-186):
    the arm the reference picks from the geometry.  Here one kernel serves both arms with the
    same token-local arithmetic; the classification is kept for callers that report it."""

    OPTIMIZED_METAL = "OptimizedMetal"
    TOKEN_LOCAL_MLX_FALLBACK = "TokenLocalMlxFallback"


@dataclass
class TargetVerificationProjection:
    """Qwen3_5TargetVerificationProjection (:188-207)."""

    projected_activations: torch.Tensor
    dispatch: TargetVerificationProjectionDispatch

    def into_projected_activations(self) -> torch.Tensor:
        return self.projected_activations


def target_verification_uses_optimized_dispatch(activation_dtype: torch.dtype, scale_dtype: torch.dtype,
                                                bias_dtype: torch.dtype, group_size: int, bits: int,
                                                input_dimension: int, output_dimension: int) -> bool:
    """target_verification_uses_optimized_dispatch (:332-356)."""
    return (bits in (4, 5) and group_size in (32, 64, 128) and input_dimension > 0
            and input_dimension % 512 == 0 and output_dimension > 0 and output_dimension % 8 == 0
            and activation_dtype == scale_dtype and bias_dtype == scale_dtype
            and activation_dtype in (torch.bfloat16, torch.float16))


_VERIFY_DTYPES = {torch.bfloat16: _lib.DTYPES.index("BF16"), torch.float16: _lib.DTYPES.index("F16")}


def qwen3_5_target_verification_quantized_linear(activations: torch.Tensor, packed_weight: torch.Tensor,
                                                 quantization_scales: torch.Tensor,
                                                 quantization_biases: torch.Tensor,
                                                 quantization_group_size: int,
                                                 quantization_bits: int) -> TargetVerificationProjection:
    """qwen3_5_target_verification_quantized_linear (:232-330): activations [B, T, K] (bf16 or
    f16), packed_weight [N, K * bits / 32] (uint32 bits as int32), scales / biases [N, K / g] of
    the activations' dtype -> [B, T, N] of that dtype.  Each token row's output has the bits of
    projecting that row alone."""
    op = "project Qwen3.5 target-verification tokens"
    a_shape, w_shape = tuple(activations.shape), tuple(packed_weight.shape)
    if len(a_shape) != 3 or min(a_shape) <= 0 or len(w_shape) != 2 or min(w_shape) <= 0:
        raise AstroMoeError(_lib.INVALID_ARGUMENT, f"{op}: target-verification arrays must have positive "
                            "rank-three activations and rank-two weights")
    if packed_weight.dtype != torch.int32 or quantization_group_size not in (32, 64, 128) \
            or quantization_bits not in (2, 3, 4, 5, 6, 8):
        raise AstroMoeError(_lib.INVALID_ARGUMENT, f"{op}: target-verification affine metadata is not "
                            "supported by MLX")
    K, N = a_shape[2], w_shape[0]
    expanded = w_shape[1] * 32 // quantization_bits if (w_shape[1] * 32) % quantization_bits == 0 else None
    affine_shape = (N, K // quantization_group_size)
    if expanded != K or K % quantization_group_size or tuple(quantization_scales.shape) != affine_shape \
            or tuple(quantization_biases.shape) != affine_shape:
        raise AstroMoeError(_lib.INVALID_ARGUMENT, f"{op}: target-verification affine arrays do not match "
                            "activation and weight geometry")
    dtype = activations.dtype
    if dtype not in _VERIFY_DTYPES or quantization_scales.dtype != dtype or quantization_biases.dtype != dtype:
        raise AstroMoeError(_lib.UNSUPPORTED, f"{op}: the verification kernel reads bfloat16 or float16 "
                            "activations, scales and biases")
    dispatch = (TargetVerificationProjectionDispatch.OPTIMIZED_METAL
                if target_verification_uses_optimized_dispatch(dtype, quantization_scales.dtype,
                                                               quantization_biases.dtype,
                                                               quantization_group_size, quantization_bits, K, N)
                else TargetVerificationProjectionDispatch.TOKEN_LOCAL_MLX_FALLBACK)
    x = activations.contiguous()
    w = Affine(packed_weight.data_ptr(), quantization_scales.contiguous().data_ptr(),
               quantization_biases.contiguous().data_ptr(), 1, N, K, quantization_bits, quantization_group_size)
    out = torch.empty(a_shape[0], a_shape[1], N, dtype=dtype, device=x.device)
    call("astro_moe_verification_quantized_linear", _ptr(x), a_shape[0], a_shape[1], K, C.byref(w),
         _VERIFY_DTYPES[dtype], _ptr(out), _stream(x.device))
    return TargetVerificationProjection(out, dispatch)


def apply_compiled_swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """mlx_compiled_swiglu.rs:44-89: silu(gate) * up in bf16."""
    g, u = gate.contiguous(), up.contiguous()
    if g.shape != u.shape:
        raise AstroMoeError(_lib.INVALID_ARGUMENT, "apply a compiled MLX SwiGLU graph: gate and "
                            "input shapes must match")
    out = torch.empty_like(g)
    call("astro_moe_swiglu", _ptr(g), _ptr(u), g.numel(), _ptr(out), _stream(g.device))
    return out


# ------------------------------------------------- reductions (weighted_sum.rs)

def sorted_expert_weighted_sum(sorted_expert_outputs: torch.Tensor, inverse_order: torch.Tensor,
                               selected_scores: torch.Tensor) -> torch.Tensor:
    """weighted_sum.rs:122-192: outputs [A, 1, D] (or [A, D]) in sorted order."""
    so = sorted_expert_outputs.contiguous()
    sc = selected_scores.contiguous()
    if sc.dtype != torch.bfloat16 or so.dtype != torch.bfloat16:
        raise AstroMoeError(_lib.INVALID_ARGUMENT, "reduce stacked expert outputs: sorted expert "
                            "outputs, inverse order, and scores have invalid shapes or dtypes")
    k = sc.shape[-1]
    A = sc.numel()
    T = A // k if k else (sc.numel())
    D = so.shape[-1]
    if so.numel() // max(D, 1) != A or inverse_order.numel() != A:
        raise AstroMoeError(_lib.INVALID_ARGUMENT, "reduce stacked expert outputs: sorted expert "
                            "outputs and inverse order must match selected scores")
    out = torch.empty(*sc.shape[:-1], D, dtype=so.dtype, device=so.device)
    call("astro_moe_sorted_weighted_sum", _ptr(so), _ptr(inverse_order.contiguous().view(torch.int32)),
         _ptr(sc), T, k, D, _ptr(out), _stream(so.device))
    return out


def unsorted_expert_weighted_sum(selected_expert_outputs: torch.Tensor,
                                 selected_scores: torch.Tensor) -> torch.Tensor:
    """weighted_sum.rs:94-120: outputs [..., k, D] * scores [..., k] summed over k."""
    o = selected_expert_outputs.contiguous()
    sc = selected_scores.contiguous()
    k = sc.shape[-1]
    D = o.shape[-1]
    T = sc.numel() // k if k else int(np.prod(sc.shape[:-1]))
    out = torch.empty(*sc.shape[:-1], D, dtype=o.dtype, device=o.device)
    call("astro_moe_unsorted_weighted_sum", _ptr(o), _ptr(sc), T, k, D, _ptr(out), _stream(o.device))
    return out


def combine_sparse_and_shared_experts(sparse_expert_output: torch.Tensor,
                                      shared_expert_output: torch.Tensor,
                                      shared_expert_gate_logits: torch.Tensor) -> torch.Tensor:
    """output_combination.rs:34-43: sparse + shared * sigmoid(gate)."""
    sp, so = sparse_expert_output.contiguous(), shared_expert_output.contiguous()
    z = shared_expert_gate_logits.contiguous()
    D = sp.shape[-1]
    T = sp.numel() // D
    if so.shape != sp.shape:
        raise AstroMoeError(_lib.INVALID_ARGUMENT, "combine Qwen3.5-MoE sparse and shared experts: "
                            "shared expert output must match the combined sparse-expert shape")
    if z.numel() != T:
        raise AstroMoeError(_lib.INVALID_ARGUMENT, "combine Qwen3.5-MoE sparse and shared experts: "
                            "shared expert gate must provide one logit per token")
    out = torch.empty_like(sp)
    call("astro_moe_combine_shared", _ptr(sp), _ptr(so), _ptr(z), T, D, _ptr(out), _stream(sp.device))
    return out


def qwen3_5_moe_combine_experts(selected_expert_outputs, selected_scores, shared_expert_output,
                                shared_expert_gate_logits):
    """output_combination.rs:7-32."""
    sparse = unsorted_expert_weighted_sum(selected_expert_outputs, selected_scores)
    return combine_sparse_and_shared_experts(sparse, shared_expert_output, shared_expert_gate_logits)


# ------------------------------------------------- the whole block (forward.rs:19-127)

class MoeBlock:
    """One resident MoE block: borrowed device weights + a reusable workspace."""

    def __init__(self, weights: MoeLayerWeights, device="cuda"):
        self.weights = weights
        self.device = torch.device(device)
        self._struct = layer_struct(weights)
        self._ws = None
        self._ws_tokens = -1

    def workspace_bytes(self, tokens: int) -> int:
        n = C.c_size_t()
        call("astro_moe_workspace_bytes", C.byref(self._struct), tokens, C.byref(n))
        return n.value

    def workspace(self, tokens: int) -> torch.Tensor:
        need = self.workspace_bytes(tokens)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(max(need, 1), dtype=torch.uint8, device=self.device)
        return self._ws

    def forward(self, x: torch.Tensor, out: Optional[torch.Tensor] = None,
                workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
        x2 = x.contiguous().view(torch.bfloat16).reshape(-1, self.weights.hidden)
        T = x2.shape[0]
        y = out if out is not None else torch.empty_like(x2)
        ws = workspace if workspace is not None else self.workspace(T)
        call("astro_moe_block_forward", C.byref(self._struct), _ptr(x2), T, _ptr(y), _ptr(ws),
             ws.numel(), _stream(self.device))
        return y

    __call__ = forward

    def verification_workspace_bytes(self, tokens: int) -> int:
        n = C.c_size_t()
        call("astro_moe_verification_workspace_bytes", C.byref(self._struct), tokens, C.byref(n))
        return n.value

    def target_verification_forward(self, x: torch.Tensor, out: Optional[torch.Tensor] = None,
                                    workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
        """forward_moe_resident_target_verification (resident_execution.rs:146-208): the block
        over an MTP verification window, each output row bit-equal to the one-token block of
        its row."""
        x2 = x.contiguous().view(torch.bfloat16).reshape(-1, self.weights.hidden)
        T = x2.shape[0]
        y = out if out is not None else torch.empty_like(x2)
        need = self.verification_workspace_bytes(T)
        ws = workspace
        if ws is None or ws.numel() < need:
            ws = torch.empty(max(need, 1), dtype=torch.uint8, device=self.device)
        call("astro_moe_block_forward_verification", C.byref(self._struct), _ptr(x2), T, _ptr(y), _ptr(ws),
             ws.numel(), _stream(self.device))
        return y

    def decoder_feed_forward(self, hidden: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                             attention_out: Optional[torch.Tensor] = None,
                             out: Optional[torch.Tensor] = None, residual: Optional[torch.Tensor] = None,
                             workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
        """The feed-forward half of a decoder layer around this block
        (decoder_layer_forward.rs:111-174): r = hidden + attention_out, n = rms_norm(r),
        out = r + MoE(n), all bf16; `residual` (optional) receives r."""
        h2 = hidden.contiguous().view(torch.bfloat16).reshape(-1, self.weights.hidden)
        T = h2.shape[0]
        a2 = None if attention_out is None else attention_out.contiguous().view(torch.bfloat16).reshape(T, -1)
        y = out if out is not None else torch.empty_like(h2)
        n = C.c_size_t()
        call("astro_moe_decoder_ffn_workspace_bytes", C.byref(self._struct), T, C.byref(n))
        ws = workspace
        if ws is None or ws.numel() < n.value:
            ws = torch.empty(max(n.value, 1), dtype=torch.uint8, device=self.device)
        w = norm_weight.contiguous().view(torch.bfloat16)
        call("astro_moe_decoder_ffn_forward", C.byref(self._struct), _ptr(h2), _ptr(a2), _ptr(w), float(eps), T,
             _ptr(y), _ptr(residual), _ptr(ws), ws.numel(), _stream(self.device))
        return y

    def forward_attributed(self, x: torch.Tensor, out: Optional[torch.Tensor] = None,
                           workspace: Optional[torch.Tensor] = None):
        """forward plus per-stage device milliseconds (synchronises the stream)."""
        x2 = x.contiguous().view(torch.bfloat16).reshape(-1, self.weights.hidden)
        T = x2.shape[0]
        y = out if out is not None else torch.empty_like(x2)
        ws = workspace if workspace is not None else self.workspace(T)
        ms = (C.c_float * len(_lib.STAGES))()
        call("astro_moe_block_forward_attributed", C.byref(self._struct), _ptr(x2), T, _ptr(y),
             _ptr(ws), ws.numel(), _stream(self.device), ms)
        return y, dict(zip(_lib.STAGES, [float(v) for v in ms]))

    def trace(self, tokens: int, workspace: Optional[torch.Tensor] = None) -> dict:
        """Intermediates of the last forward with `tokens` tokens (host numpy copies)."""
        v = WorkspaceView()
        call("astro_moe_workspace_layout", C.byref(self._struct), tokens, C.byref(v))
        ws = workspace if workspace is not None else self._ws
        torch.cuda.synchronize(self.device)
        raw = ws[: v.total_bytes].cpu().numpy()
        L = self.weights
        T, E, k, H, I = tokens, L.num_experts, L.top_k, L.hidden, L.intermediate
        A = T * k
        # the sort buckets page slots when the layer is a compact page
        capacity = (L.gate_up if L.gate_up is not None else L.gate).experts
        E_sort = max(E, capacity)

        def get(off, n, dt):
            return raw[off: off + n * np.dtype(dt).itemsize].view(dt).copy()
        out = dict(
            sorted_path=bool(v.sorted_path),
            logits=get(v.logits, T * E, np.uint16).reshape(T, E),
            indices=get(v.indices, A, np.uint32).reshape(T, k),
            scores=get(v.scores, A, np.uint16).reshape(T, k),
            sorted_order=get(v.sorted_order, A, np.uint32),
            inverse_order=get(v.inverse_order, A, np.uint32),
            sorted_ids=get(v.sorted_ids, A, np.uint32),
            expert_offsets=get(v.expert_offsets, E_sort + 1, np.uint32),
            activated_sorted=_unpair(get(v.activated, A * v.activated_ld, np.uint16).reshape(A, v.activated_ld)[:, :I],
                                     bool(v.activated_paired)),
            expert_out_sorted=get(v.expert_out, A * H, np.uint16).reshape(A, H),
            sparse=get(v.sparse, T * H, np.uint16).reshape(T, H))
        if L.shared_intermediate:
            out["shared_out"] = get(v.shared_out, T * H, np.uint16).reshape(T, H)
            out["shared_gate_logits"] = get(v.shared_gate_logits, T, np.uint16)
        if v.sorted_path and v.max_tiles:
            n_tiles = int(get(v.tile_count, 1, np.uint32)[0])
            out["tile_expert"] = get(v.tile_expert, v.max_tiles, np.uint32)[:n_tiles]
            out["tile_row0"] = get(v.tile_row0, v.max_tiles, np.uint32)[:n_tiles]
        if L.slot_of_expert is not None:
            out["expert_slots"] = get(v.expert_slots, A, np.uint32).reshape(T, k)
            out["missing_slots"] = int(get(v.missing_slots, 1, np.uint32)[0])
        return out


def _unpair(rows: np.ndarray, paired: bool) -> np.ndarray:
    """Activated rows in natural order: a paired row's 8-element chunks hold 0 4 1 5 2 6 3 7."""
    if not paired:
        return rows
    n = rows.shape[1]
    c = rows.reshape(rows.shape[0], n // 8, 8)
    return c[:, :, [0, 2, 4, 6, 1, 3, 5, 7]].reshape(rows.shape[0], n)


def router_logits(weights: MoeLayerWeights, x: torch.Tensor) -> torch.Tensor:
    """forward.rs:52-93 (+ the optional logit bias)."""
    s = layer_struct(weights)
    x2 = x.contiguous().view(torch.bfloat16).reshape(-1, weights.hidden)
    out = torch.empty(x2.shape[0], weights.num_experts, dtype=torch.bfloat16, device=x.device)
    call("astro_moe_router_logits", C.byref(s), _ptr(x2), x2.shape[0], _ptr(out), _stream(x.device))
    return out


def shared_expert(weights: MoeLayerWeights, x: torch.Tensor):
    """resident_execution.rs:360-382 -> (shared_out bf16 [T, H], gate_logits bf16 [T])."""
    s = layer_struct(weights)
    x2 = x.contiguous().view(torch.bfloat16).reshape(-1, weights.hidden)
    T = x2.shape[0]
    need = C.c_size_t()
    call("astro_moe_shared_expert_workspace_bytes", C.byref(s), T, C.byref(need))
    ws = torch.empty(max(need.value, 1), dtype=torch.uint8, device=x.device)
    so = torch.empty(T, weights.hidden, dtype=torch.bfloat16, device=x.device)
    z = torch.empty(T, dtype=torch.bfloat16, device=x.device)
    call("astro_moe_shared_expert", C.byref(s), _ptr(x2), T, _ptr(so), _ptr(z), _ptr(ws),
         need.value, _stream(x.device))
    return so, z


# ------------------------------------------------------ paged callers (paged_execution.rs)

SLOT_ABSENT = 0xFFFFFFFF
_REMAP_OP = "remap Qwen3.5-MoE expert page slots"
_SPLIT_OP = "build Qwen3.5-MoE split expert page route"


def qwen3_5_moe_remap_expert_page_slots(selected_indices: torch.Tensor,
                                        page_slot_by_global_expert_id: torch.Tensor) -> torch.Tensor:
    """split_page_route.rs:79-105: page slot of every selected expert (int32, same shape).
    Like the reference, refuses a routed expert the page does not hold; the check reads the
    device's absent-expert count back (one stream synchronisation)."""
    ids = selected_indices.contiguous().view(torch.int32)
    m = page_slot_by_global_expert_id.contiguous().view(torch.int32)
    slots = torch.empty_like(ids)
    missing = torch.zeros(1, dtype=torch.int32, device=ids.device)
    call("astro_moe_remap_expert_slots", _ptr(ids), ids.numel(), _ptr(m), m.numel(), _ptr(slots),
         _ptr(missing), _stream(ids.device))
    if int(missing.item()):
        raise AstroMoeError(_lib.INVALID_ARGUMENT,
                            f"{_REMAP_OP}: a routed expert is absent from the streamed page manifest")
    return slots


def forward_moe_with_streamed_weights(hidden_states: torch.Tensor, page: MoeLayerWeights,
                                      page_slot_indices: torch.Tensor,
                                      selected_scores: torch.Tensor) -> torch.Tensor:
    """paged_execution.rs:207-281: the sparse expert output bf16 [T, H] of T tokens with
    page_slot_indices / selected_scores [T, kk] against the page's routed arrays."""
    s = layer_struct(page)
    x2 = hidden_states.contiguous().view(torch.bfloat16).reshape(-1, page.hidden)
    T = x2.shape[0]
    slots = page_slot_indices.contiguous().view(torch.int32).reshape(T, -1)
    sc = selected_scores.contiguous().view(torch.bfloat16).reshape(T, -1)
    kk = slots.shape[1]
    need = C.c_size_t()
    call("astro_moe_streamed_sparse_workspace_bytes", C.byref(s), T, kk, C.byref(need))
    ws = torch.empty(max(need.value, 1), dtype=torch.uint8, device=x2.device)
    out = torch.empty(T, page.hidden, dtype=torch.bfloat16, device=x2.device)
    call("astro_moe_streamed_sparse_forward", C.byref(s), _ptr(x2), T, _ptr(slots), _ptr(sc), kk,
         _ptr(out), _ptr(ws), need.value, _stream(x2.device))
    return out


def rms_norm(hidden: torch.Tensor, weight: torch.Tensor, eps: float,
             attention_out: Optional[torch.Tensor] = None, residual_out: Optional[torch.Tensor] = None
             ) -> torch.Tensor:
    """MlxRuntime::rms_norm (mlx_operations.rs:91-101) of hidden (+ attention_out, the decoder's
    attention residual, written to residual_out when given), bf16 [..., H]."""
    H = hidden.shape[-1]
    h2 = hidden.contiguous().view(torch.bfloat16).reshape(-1, H)
    a2 = None if attention_out is None else attention_out.contiguous().view(torch.bfloat16).reshape(-1, H)
    out = torch.empty_like(h2)
    call("astro_moe_add_rms_norm", _ptr(h2), _ptr(a2), _ptr(weight.contiguous().view(torch.bfloat16)), float(eps),
         h2.shape[0], H, _ptr(residual_out), _ptr(out), _stream(h2.device))
    return out.reshape(hidden.shape)


def route_laguna_experts(router_logits: torch.Tensor, experts_per_token: int,
                         correction_bias: Optional[torch.Tensor] = None, router_logit_softcap: float = 0.0,
                         normalize: bool = True):
    """route_laguna_experts (laguna/moe/router.rs:29-94): (selected indices int32 [..., k],
    fp32 scores [..., k]) in the order of the CPU selection (router_selection.rs:59-116)."""
    lg = router_logits.contiguous().view(torch.bfloat16)
    E = lg.shape[-1]
    T = lg.numel() // max(E, 1)
    shape = tuple(lg.shape[:-1]) + (experts_per_token,)
    idx = torch.empty(shape, dtype=torch.int32, device=lg.device)
    sc = torch.empty(shape, dtype=torch.float32, device=lg.device)
    bias = None if correction_bias is None else correction_bias.contiguous().to(torch.float32)
    call("astro_moe_route_laguna", _ptr(lg), T, E, experts_per_token, _ptr(bias), float(router_logit_softcap),
         int(normalize), _ptr(idx), _ptr(sc), _stream(lg.device))
    return idx, sc


def add(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """MlxRuntime::add of two bf16 arrays of one shape (fp32 sum, rounded to nearest even)."""
    a2, b2 = a.contiguous().view(torch.bfloat16), b.contiguous().view(torch.bfloat16)
    if a2.shape != b2.shape:
        raise AstroMoeError(_lib.INVALID_ARGUMENT, "add: operands must have one shape")
    out = torch.empty_like(a2)
    call("astro_moe_add", _ptr(a2), _ptr(b2), a2.numel(), _ptr(out), _stream(a2.device))
    return out


def selftest_bf16_rounding(device: str | torch.device = "cuda") -> int:
    """Fp32 bit patterns (of all 2^32) on which the library's bf16 rounding differs from
    round-to-nearest-even on the bit pattern; 0 when they agree everywhere."""
    count = torch.zeros(1, dtype=torch.int64, device=device)
    call("astro_moe_selftest_bf16_rounding", _ptr(count), _stream(count.device))
    return int(count.item())


@dataclass
class Qwen3_5MoESplitPageRoute:
    """split_page_route.rs:11-16."""
    retained_page_slot_indices: torch.Tensor
    retained_scores: torch.Tensor
    missing_page_slot_indices: torch.Tensor
    missing_scores: torch.Tensor

    @staticmethod
    def build(selected_indices: torch.Tensor, selected_scores: torch.Tensor,
              retained_assignment_positions: Sequence[int], missing_assignment_positions: Sequence[int],
              retained_page_slot_by_expert: torch.Tensor,
              missing_page_slot_by_expert: torch.Tensor) -> "Qwen3_5MoESplitPageRoute":
        """split_page_route.rs:20-73, with validate_split_page_route (:107-150) on the host."""
        n = selected_indices.numel()
        ret, mis = list(retained_assignment_positions), list(missing_assignment_positions)
        if (n == 0 or selected_scores.numel() != n or not ret or not mis or len(ret) + len(mis) != n):
            raise AstroMoeError(_lib.INVALID_ARGUMENT, f"{_SPLIT_OP}: selected indices, scores, and "
                                "non-empty route sides must cover the same assignments")
        covered = [False] * n
        for p in ret + mis:
            if not 0 <= p < n:
                raise AstroMoeError(_lib.INVALID_ARGUMENT, f"{_SPLIT_OP}: a route assignment position "
                                    "exceeds the selected assignment count")
            if covered[p]:
                raise AstroMoeError(_lib.INVALID_ARGUMENT, f"{_SPLIT_OP}: a route assignment position "
                                    "appears more than once")
            covered[p] = True
        ids = selected_indices.contiguous().view(torch.int32).reshape(-1)
        sc = selected_scores.contiguous().view(torch.bfloat16).reshape(-1)
        sides = []
        for pos, m in ((ret, retained_page_slot_by_expert), (mis, missing_page_slot_by_expert)):
            p = torch.tensor(pos, dtype=torch.int32, device=ids.device)
            side_ids = torch.empty(len(pos), dtype=torch.int32, device=ids.device)
            side_sc = torch.empty(len(pos), dtype=torch.bfloat16, device=ids.device)
            call("astro_moe_gather_assignments", _ptr(ids), _ptr(sc), _ptr(p), len(pos), _ptr(side_ids),
                 _ptr(side_sc), _stream(ids.device))
            sides += [qwen3_5_moe_remap_expert_page_slots(side_ids, m), side_sc]
        return Qwen3_5MoESplitPageRoute(*sides)


def forward_moe_split_paged(hidden_states: torch.Tensor, weights: MoeLayerWeights,
                            retained_page: MoeLayerWeights, missing_page: MoeLayerWeights,
                            selected_indices: torch.Tensor, selected_scores: torch.Tensor,
                            retained_assignment_positions: Sequence[int],
                            missing_assignment_positions: Sequence[int]) -> torch.Tensor:
    """forward_moe_split_paged_with_performance_attribution (paged_execution.rs:147-205) for
    one decode token: the retained and missing pages each run the streamed sparse graph over
    their side of the route, the partial outputs are added, then the shared expert of
    `weights` and the shared combine.  Pages carry their slot maps in slot_of_expert."""
    route = Qwen3_5MoESplitPageRoute.build(
        selected_indices, selected_scores, retained_assignment_positions, missing_assignment_positions,
        retained_page.slot_of_expert, missing_page.slot_of_expert)
    x2 = hidden_states.contiguous().view(torch.bfloat16).reshape(-1, weights.hidden)
    retained = forward_moe_with_streamed_weights(x2, retained_page, route.retained_page_slot_indices.reshape(1, -1),
                                                 route.retained_scores.reshape(1, -1))
    missing = forward_moe_with_streamed_weights(x2, missing_page, route.missing_page_slot_indices.reshape(1, -1),
                                                route.missing_scores.reshape(1, -1))
    sparse = add(retained, missing)
    if not weights.shared_intermediate:
        return sparse
    so, z = shared_expert(weights, x2)
    return combine_sparse_and_shared_experts(sparse, so, z)
