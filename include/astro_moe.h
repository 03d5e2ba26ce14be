/*
 * astro_moe — MI355X (gfx950) sorted mixture-of-experts block behind a plain C ABI.
 *
 * This is the drop-in seam for the reference's MoE block.  The reference reaches the
 * block through Qwen3_5Model::forward_qwen3_5_moe
 * (crates/model-serving/src/qwen3_5_moe/model/forward.rs:19-28) and every operation
 * below it through the MLX-C C ABI bound in crates/runtime-integration/src/raw.rs:1-11.
 * Each entry point below names the reference function it replaces.
 *
 * Conventions (mirroring MLX-C, crates/runtime-integration/src/mlx_runtime/error_handling.rs:19-62):
 *  - every call returns an int status, 0 = success;
 *  - on failure astro_moe_last_error() returns a thread-local message of the form
 *    "<operation>: <description>"; a too-small workspace carries the marker
 *    "ASTRONOMICAL_MLX_ACTIVE_MEMORY_LIMIT_EXCEEDED active_bytes=0 allocation_bytes=<needed>
 *    allowed_bytes=<given>" so classify_mlx_error (error_handling.rs:57-62, :81-122) still
 *    returns ActiveMemoryLimitExceeded;
 *  - bf16 tensors are uint16_t bit patterns; packed affine weights are uint32_t in MLX
 *    layout (element j of a row = bits [j*b, j*b+b) of the row's little-endian bit
 *    stream); scales/biases are bf16;
 *  - all pointers are device pointers (HBM) unless stated; the caller owns every buffer
 *    and the library never allocates on the hot path — scratch comes from `workspace`;
 *  - `stream` is a hipStream_t (NULL = the default stream); every launch is
 *    asynchronous on it; no global mutable state besides the thread-local error.
 *  - No C++ exception crosses this ABI.
 */
#ifndef ASTRO_MOE_H
#define ASTRO_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ASTRO_MOE_ABI_VERSION 6

enum astro_moe_status {
  ASTRO_MOE_OK = 0,
  ASTRO_MOE_INVALID_ARGUMENT = 1,      /* geometry, dtype contract or null pointer */
  ASTRO_MOE_UNSUPPORTED = 2,           /* valid for MLX, not implemented by the kernels */
  ASTRO_MOE_WORKSPACE_TOO_SMALL = 3,   /* message carries the active-memory marker */
  ASTRO_MOE_HIP_ERROR = 4,             /* a HIP runtime call failed */
};

/*
 * One stacked affine projection in MLX layout (gathered_projection.rs:50-71,
 * StackedExpertProjection::Affine): w [experts][out][in*bits/32] u32,
 * scales/biases [experts][out][in/group] bf16.  experts == 1 for a plain quantized
 * linear (router, shared expert).  Kernels implement bits in {4, 8} and group in
 * {32, 64, 128}; other MLX widths return ASTRO_MOE_UNSUPPORTED.
 */
typedef struct astro_moe_affine {
  const uint32_t *w;
  const uint16_t *scales;
  const uint16_t *biases;
  int32_t experts;
  int32_t out_features;
  int32_t in_features;
  int32_t bits;
  int32_t group_size;
} astro_moe_affine;

/*
 * Borrowed weights of one block (Qwen3_5MoEFeedForwardWeights, feed_forward_weights.rs:17-24,
 * and the resident expert arrays, resident_expert_layer_weights.rs:12-16).  Exactly one
 * of router_w / router_q.w is set.  gate_up.w set selects the fused resident layout
 * [E][2I][H*b/32] (resident_gate_up_fusion.rs:221-260); otherwise gate and up are
 * separate pages.  shared_intermediate == 0 means no shared expert.
 */
typedef struct astro_moe_layer {
  int32_t hidden;              /* H */
  int32_t num_experts;         /* E */
  int32_t top_k;               /* k */
  int32_t intermediate;        /* I */
  int32_t shared_intermediate; /* Is */
  int32_t normalize_top_k;     /* norm_topk_prob (config_document.rs:145) */
  const uint16_t *router_w;    /* bf16 [E][H] (unquantized router, forward.rs:59-91) */
  astro_moe_affine router_q;   /* affine router (forward.rs:53-58) */
  const uint16_t *router_bias; /* optional bf16 [E] added to the logits (benchmark skew only) */
  astro_moe_affine gate_up;
  astro_moe_affine gate;
  astro_moe_affine up;
  astro_moe_affine down;                /* [E][H][I*b/32] */
  astro_moe_affine shared_gate;         /* [1][Is][H*b/32] */
  astro_moe_affine shared_up;
  astro_moe_affine shared_down;         /* [1][H][Is*b/32] */
  astro_moe_affine shared_expert_gate;  /* [1][1][H*b/32] */
  /* Compact paged pages (forward_moe_paged_with_performance_attribution,
   * paged_execution.rs:98-139; page_slot_by_global_expert_id,
   * quantized_expert_manifest.rs:212-220): when set, u32 [num_experts] maps each global
   * expert id to its slot in the routed arrays above, whose `experts` is then the page's slot
   * count; 0xffffffff marks an expert the page does not hold.  Routing is unchanged; the
   * assignments are sorted and computed by slot.  The reference refuses a routed expert absent
   * from the page on the host; here each one counts into the workspace word
   * astro_moe_workspace_view.missing_slots (read it after the stream completes) and reads
   * slot 0.  NULL: resident arrays indexed by expert id. */
  const uint32_t *slot_of_expert;
} astro_moe_layer;

/* Byte offsets of the block's intermediates inside the workspace, valid after
 * astro_moe_block_forward with the same layer and token count (for inspection and
 * tests; the hot path never reads this). Offsets are from the workspace base. */
typedef struct astro_moe_workspace_view {
  size_t total_bytes;
  int32_t sorted_path;       /* 1 when T*k >= 64 (routing.rs:13) */
  size_t logits;             /* bf16 [T][E] */
  size_t indices;            /* u32 [T][k] */
  size_t scores;             /* bf16 [T][k] */
  size_t sorted_order;       /* u32 [A]: sorted slot -> original slot */
  size_t inverse_order;      /* u32 [A]: original slot -> sorted slot */
  size_t sorted_ids;         /* u32 [A] */
  size_t expert_offsets;     /* u32 [E+1] */
  size_t activated;          /* bf16 [A][activated_ld], sorted order */
  size_t activated_ld;       /* elements per activated row (>= I) */
  size_t expert_out;         /* bf16 [A][H], sorted order */
  size_t sparse;             /* bf16 [T][H] */
  size_t shared_out;         /* bf16 [T][H] */
  size_t shared_gate_logits; /* bf16 [T] */
  size_t expert_slots;       /* u32 [T][k] page slots (slot_of_expert set; else 0) */
  size_t missing_slots;      /* u32: routed experts absent from the page (slot_of_expert set) */
  /* Sorted path only (0 on the decode path): the grouped GEMMs' tile table written by the
   * sort -- u32 tile_expert[max_tiles], u32 tile_row0[max_tiles] (first sorted row of the
   * tile), u32 tile_count (tiles in use).  Tiles hold up to 64 rows of one expert; every
   * tile of more than 32 rows is listed before the smaller last tiles. */
  size_t tile_expert;
  size_t tile_row0;
  size_t tile_count;
  size_t max_tiles;          /* entries of tile_expert / tile_row0 (a count, not an offset) */
  /* 1 when the activated rows are stored in the 4-bit codes' pairing: each 8-element chunk
   * holds elements 0 4 1 5 2 6 3 7 (exact-code GEMMs, with a 256-byte aligned workspace) */
  size_t activated_paired;
} astro_moe_workspace_view;

const char *astro_moe_last_error(void);
int astro_moe_abi_version(void);

/* Workspace sizing for astro_moe_block_forward (host-only, no GPU call). */
int astro_moe_workspace_bytes(const astro_moe_layer *layer, int32_t tokens, size_t *bytes);
int astro_moe_workspace_layout(const astro_moe_layer *layer, int32_t tokens,
                               astro_moe_workspace_view *view);

/*
 * Whole block, y = MoE(x): replaces Qwen3_5Model::forward_qwen3_5_moe with the
 * resident owner (forward.rs:19-127 -> resident_execution.rs:70-143, :352-400).
 * x, y: bf16 [tokens][H].  The residual add stays with the caller
 * (decoder_layer_forward.rs:172-173).
 */
int astro_moe_block_forward(const astro_moe_layer *layer, const uint16_t *x, int32_t tokens,
                            uint16_t *y, void *workspace, size_t workspace_bytes,
                            void *stream);

/*
 * astro_moe_block_forward without a workspace argument and without any allocation: no
 * counterpart in the reference.  It is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * block's intermediates live in a static device array of ASTRO_MOE_STATIC_SCRATCH_BYTES per
 * GPU, held from the first call on that GPU until the process ends; a call whose workspace
 * (astro_moe_workspace_bytes) exceeds it fails with ASTRO_MOE_WORKSPACE_TOO_SMALL.  Every
 * call on one GPU shares that array: calls that overlap on one GPU (two streams, two host
 * threads) race, so serialise them.  The first call on a device must not happen during
 * graph capture (it looks up the array's address once per device).
 */
#define ASTRO_MOE_STATIC_SCRATCH_BYTES ((size_t)32 << 20)
int astro_moe_block_forward_no_alloc(const astro_moe_layer *layer, const uint16_t *x, int32_t tokens,
                                     uint16_t *y, void *stream);

/*
 * The same forward with per-stage device times, the counterpart of the reference's
 * PerformanceAttribution operation timers (crates/model-serving/src/performance_attribution.rs:1-80,
 * performance_attribution/catalog.rs:54,89-91) — but measuring device time rather than
 * graph construction.  stage_ms[ASTRO_MOE_STAGES] receives: router projection, route
 * (softmax/top-k), sort (assignment preparation; with 4-bit gate/up also x's group sums and
 * its copy in the codes' pairing), gate/up + SwiGLU, down (gathered expert execution), shared
 * expert, combine (weighted reduction).  On the sorted path the shared expert's gate/up and
 * down projections run inside the gate/up and down launches (their tiles come before the
 * routed ones), so its stage holds the output gate only.  A stage that is one kernel is
 * timed by events attached to that kernel's dispatch; other stages by event records around
 * their launches.  The decode path (tokens * top_k <= 64) runs three kernels and reports
 * them as router, gate/up (which also runs the shared expert's gate/up, the routing and
 * the sort) and down (which also runs the shared expert's down projection and the
 * combine); its other stages read 0.  Synchronises the stream; not for the hot path.
 */
#define ASTRO_MOE_STAGES 7
int astro_moe_block_forward_attributed(const astro_moe_layer *layer, const uint16_t *x,
                                       int32_t tokens, uint16_t *y, void *workspace,
                                       size_t workspace_bytes, void *stream, float *stage_ms);

/*
 * The block over an MTP target-verification window (forward_moe_resident_target_verification,
 * resident_execution.rs:146-208): token rows stay unsorted, so output row t has the bits of
 * astro_moe_block_forward on row t alone, whatever the window length (the exact rollback
 * boundary after a rejected draft).  Same arguments as astro_moe_block_forward; the
 * workspace is astro_moe_verification_workspace_bytes(layer, tokens).
 */
int astro_moe_verification_workspace_bytes(const astro_moe_layer *layer, int32_t tokens, size_t *bytes);
int astro_moe_block_forward_verification(const astro_moe_layer *layer, const uint16_t *x, int32_t tokens,
                                         uint16_t *y, void *workspace, size_t workspace_bytes, void *stream);

/* Router projection logits = x·W_rᵀ (bf16 out, fp32 accumulate), plus router_bias if
 * set: forward.rs:52-93 (matmul or quantized_linear). */
int astro_moe_router_logits(const astro_moe_layer *layer, const uint16_t *x, int32_t tokens,
                            uint16_t *logits, void *stream);

/* qwen3_5_moe_route_experts (routing.rs:16-48): softmax, top-k, optional
 * renormalisation.  indices u32 [T][k] (ascending in (probability, index)),
 * scores bf16 [T][k]. */
int astro_moe_route_topk(const uint16_t *logits, int32_t tokens, int32_t experts,
                         int32_t top_k, int32_t normalize, uint32_t *indices,
                         uint16_t *scores, void *stream);

/* sort_expert_assignments (assignment_sort.rs:36-97) minus the row gather, which the
 * gathered matmul fuses into its activation load: sorted_order = stable argsort(ids),
 * inverse_order, sorted_ids, expert_offsets [E+1]. */
int astro_moe_sort_workspace_bytes(int32_t assignments, int32_t experts, size_t *bytes);
int astro_moe_sort_assignments(const uint32_t *ids, int32_t assignments, int32_t experts,
                               uint32_t *sorted_order, uint32_t *inverse_order,
                               uint32_t *sorted_ids, uint32_t *expert_offsets,
                               void *workspace, size_t workspace_bytes, void *stream);

/* invert_assignment_order (assignment_permutation.rs:10-42); HOST pointers, no GPU. */
int astro_moe_invert_assignment_order(const uint32_t *sorted_order, int32_t n,
                                      uint32_t *inverse_order);

/*
 * gather_expert_projection / MlxRuntime::gather_quantized_matmul_affine
 * (gathered_projection.rs:84-131, mlx_quantized_operations.rs:100-157, transpose = true):
 * out[r] = x[x_rows ? x_rows[r] : r] · deq(W[ids[r]])ᵀ, bf16 [rows][out_features].
 * sorted_indices is the caller's promise that ids ascend (gathered_projection.rs:18-43);
 * results do not depend on it.
 */
int astro_moe_gather_qmm_workspace_bytes(int32_t rows, int32_t experts, size_t *bytes);
int astro_moe_gather_qmm(const uint16_t *x, const uint32_t *x_rows, int32_t rows,
                         const astro_moe_affine *w, const uint32_t *ids,
                         int32_t sorted_indices, uint16_t *out, void *workspace,
                         size_t workspace_bytes, void *stream);

/* quantized_matmul_affine (mlx_quantized_operations.rs:49-96) for w.experts == 1. */
int astro_moe_quantized_matmul(const uint16_t *x, int32_t rows, const astro_moe_affine *w,
                               uint16_t *out, void *stream);

/* apply_compiled_swiglu (mlx_compiled_swiglu.rs:44-89): silu(gate) * up, bf16. */
int astro_moe_swiglu(const uint16_t *gate, const uint16_t *up, int64_t n, uint16_t *out,
                     void *stream);

/* sorted_expert_weighted_sum (weighted_sum.rs:16-33, :122-192). */
int astro_moe_sorted_weighted_sum(const uint16_t *sorted_outputs, const uint32_t *inverse_order,
                                  const uint16_t *scores, int32_t tokens, int32_t top_k,
                                  int32_t dim, uint16_t *out, void *stream);

/* unsorted_expert_weighted_sum (weighted_sum.rs:94-120): outputs [T][k][D]. */
int astro_moe_unsorted_weighted_sum(const uint16_t *outputs, const uint16_t *scores,
                                    int32_t tokens, int32_t top_k, int32_t dim,
                                    uint16_t *out, void *stream);

/* combine_sparse_and_shared_experts (output_combination.rs:34-43). */
int astro_moe_combine_shared(const uint16_t *sparse, const uint16_t *shared_out,
                             const uint16_t *gate_logits, int32_t tokens, int32_t dim,
                             uint16_t *out, void *stream);

/* Shared expert of combine_resident_sparse_and_shared_experts (resident_execution.rs:360-382):
 * shared_out = down(swiglu(gate(x), up(x))), gate_logits = shared_expert_gate(x). */
int astro_moe_shared_expert_workspace_bytes(const astro_moe_layer *layer, int32_t tokens,
                                            size_t *bytes);
int astro_moe_shared_expert(const astro_moe_layer *layer, const uint16_t *x, int32_t tokens,
                            uint16_t *shared_out, uint16_t *gate_logits, void *workspace,
                            size_t workspace_bytes, void *stream);

/*
 * Paged callers (paged_execution.rs; split_page_route.rs).  The resident block above takes
 * compact pages through slot_of_expert.  A split-page decode step (retained page + miss page,
 * forward_moe_split_paged_with_performance_attribution, paged_execution.rs:147-205) composes:
 *   for each side: astro_moe_gather_assignments (its positions) -> astro_moe_remap_expert_slots
 *   (its page map) -> astro_moe_streamed_sparse_forward (its page, T = 1, per_token = the
 *   side's assignment count); then astro_moe_add of the two partial outputs,
 *   astro_moe_shared_expert and astro_moe_combine_shared.
 */

/* qwen3_5_moe_remap_expert_page_slots (split_page_route.rs:79-105): slots[a] =
 * slot_of_expert[expert_ids[a]], a < n.  The reference rejects a routed expert absent from
 * the page (slot 0xffffffff) on the host; here each absent or out-of-range id adds 1 to
 * *missing_count (a device word the caller zeroes first; may be NULL) and maps to slot 0, so
 * every later access stays inside the page. */
int astro_moe_remap_expert_slots(const uint32_t *expert_ids, int32_t n, const uint32_t *slot_of_expert,
                                 int32_t experts, uint32_t *slots, uint32_t *missing_count, void *stream);

/* The take of one route side in Qwen3_5MoESplitPageRoute::build (split_page_route.rs:28-55):
 * out_ids[i] = ids[positions[i]], out_scores[i] = scores[positions[i]], i < n (either output
 * may be NULL).  validate_split_page_route (split_page_route.rs:107-150) stays with the
 * caller, which holds the positions on the host. */
int astro_moe_gather_assignments(const uint32_t *ids, const uint16_t *scores, const uint32_t *positions,
                                 int32_t n, uint32_t *out_ids, uint16_t *out_scores, void *stream);

/* forward_moe_with_streamed_weights (paged_execution.rs:207-281): the sparse expert output
 * [T][H] of T tokens with per_token assignments each -- page slots u32 [T][per_token], scores
 * bf16 [T][per_token] -- against the routed arrays of `page` (gate_up or gate/up, and down;
 * `experts` = the page's slots; hidden and intermediate set; router, shared expert and
 * slot_of_expert are not read).  Sorted by slot with the sorted rounding iff
 * T * per_token >= 64 (routing.rs:13), else the unsorted rounding. */
int astro_moe_streamed_sparse_workspace_bytes(const astro_moe_layer *page, int32_t tokens,
                                              int32_t per_token, size_t *bytes);
int astro_moe_streamed_sparse_forward(const astro_moe_layer *page, const uint16_t *x, int32_t tokens,
                                      const uint32_t *slots, const uint16_t *scores, int32_t per_token,
                                      uint16_t *sparse, void *workspace, size_t workspace_bytes,
                                      void *stream);

/* MlxRuntime::add of the two partial sparse outputs (paged_execution.rs:189-191):
 * out = bf16(float(a) + float(b)), round to nearest even. */
int astro_moe_add(const uint16_t *a, const uint16_t *b, int64_t n, uint16_t *out, void *stream);

/*
 * ------------------------------------------------------------------ the decoder step around the block
 * The feed-forward half of a Qwen3.5 decoder layer (forward_decoder_layer_attention's tail and
 * forward_decoder_layer_feed_forward, decoder_layer_forward.rs:111-174):
 *   r = bf16(hidden + attention_out)                    (attention_residual; attention_out NULL: r = hidden)
 *   n = bf16(w * bf16(r * rsqrt(mean(r^2) + eps)))      (mlx_fast_rms_norm, fp32 inside)
 *   out = bf16(r + MoE(n))
 * All bf16 [tokens][hidden]; w bf16 [hidden]; hidden <= 8192.
 */
int astro_moe_add_rms_norm(const uint16_t *hidden, const uint16_t *attention_out, const uint16_t *norm_weight,
                           float eps, int32_t tokens, int32_t hidden_size, uint16_t *residual_out,
                           uint16_t *normed_out, void *stream);
int astro_moe_decoder_ffn_workspace_bytes(const astro_moe_layer *layer, int32_t tokens, size_t *bytes);
/* residual_out (nullable) receives r. */
int astro_moe_decoder_ffn_forward(const astro_moe_layer *layer, const uint16_t *hidden,
                                  const uint16_t *attention_out, const uint16_t *norm_weight, float eps,
                                  int32_t tokens, uint16_t *out, uint16_t *residual_out, void *workspace,
                                  size_t workspace_bytes, void *stream);

/*
 * Laguna's sigmoid router, the second router family over the same sparse experts:
 * route_laguna_experts (laguna/moe/router.rs:29-94), emitted in the order of the reference's
 * CPU selection select_laguna_router_experts (router_selection.rs:59-116).  Per token: fp32
 * logit l (tanh-softcapped, l = tanh(l / softcap) * softcap, when softcap > 0), score
 * s = sigmoid(l); the top_k experts of largest s + correction_bias (f32 total order, ties to the
 * lower expert id) in that descending order; scores = their unbiased s, divided by their
 * in-order fp32 sum when normalize and the sum is positive.  logits bf16 [tokens][experts];
 * correction_bias fp32 [experts] or NULL; indices u32 [tokens][top_k]; scores fp32 [tokens][top_k].
 */
int astro_moe_route_laguna(const uint16_t *logits, int32_t tokens, int32_t experts, int32_t top_k,
                           const float *correction_bias, double softcap, int32_t normalize,
                           uint32_t *indices, float *scores, void *stream);

/*
 * ------------------------------------------------------------------ expert pages from safetensors
 * Host-side I/O; no kernel runs.  The checkpoint keeps each projection of a layer as three
 * rank-3 tensors "<layer_prefix>.switch_mlp.<proj>.<param>" (proj: gate_proj, up_proj,
 * down_proj; param: weight (U32 codes), scales, biases), each [experts, out, inner] and
 * possibly in different shard files.  The loader reads exactly the byte intervals of the
 * selected experts (never a whole shard) and writes them, unchanged, into the caller's
 * buffers in the MLX affine layout the block reads.
 */
enum astro_moe_dtype {  /* the safetensors dtypes MLX 0.32 reads (safetensors_header.rs:23-38) */
  ASTRO_MOE_DTYPE_BOOL = 0, ASTRO_MOE_DTYPE_I8, ASTRO_MOE_DTYPE_U8, ASTRO_MOE_DTYPE_F8_E4M3,
  ASTRO_MOE_DTYPE_F8_E5M2, ASTRO_MOE_DTYPE_I16, ASTRO_MOE_DTYPE_U16, ASTRO_MOE_DTYPE_F16,
  ASTRO_MOE_DTYPE_BF16, ASTRO_MOE_DTYPE_I32, ASTRO_MOE_DTYPE_U32, ASTRO_MOE_DTYPE_F32,
  ASTRO_MOE_DTYPE_I64, ASTRO_MOE_DTYPE_U64
};

#define ASTRO_MOE_PATH_MAX 1024

/* One full expert tensor of a layer: quantized_expert_manifest.rs:300-315 (QuantizedTensorSource). */
typedef struct astro_moe_tensor_source {
  char source_file[ASTRO_MOE_PATH_MAX];  /* shard path */
  int32_t dtype;                         /* astro_moe_dtype */
  int64_t shape[3];                      /* [expert capacity, out, inner] */
  uint64_t file_offset;                  /* file-relative offset of expert 0 */
  uint64_t bytes_per_expert;
  uint64_t file_size;
} astro_moe_tensor_source;

/* Startup-validated layer plan: quantized_expert_manifest.rs:317-326 plus the resident gate/up
 * fusion decision (resident_gate_up_fusion.rs:109-163). */
typedef struct astro_moe_expert_layer_plan {
  astro_moe_tensor_source src[3][3];  /* [gate_proj, up_proj, down_proj][weight, scales, biases] */
  int32_t expert_capacity;
  int32_t bits[3], group_size[3];     /* per projection */
  int32_t gate_up_fusable;            /* 1: gate and up may be concatenated on the output axis */
  char gate_up_separate_reason[96];   /* why not, when gate_up_fusable == 0 */
} astro_moe_expert_layer_plan;

/* One read of a selected-expert run: source_manifests.rs:46-58 (QuantizedExpertSourceInterval).
 * virtual_offset is the run's offset inside its tensor's compact page payload. */
typedef struct astro_moe_page_interval {
  int32_t projection, parameter;      /* src indices */
  int32_t expert_start, expert_count, first_page_slot;
  uint64_t file_offset, byte_count, virtual_offset;
} astro_moe_page_interval;

/* Parses the safetensors framing of `path` (8-byte little-endian length, JSON header of at most
 * 64 MiB) with every check of parse_safetensors_header (safetensors_header.rs:171-276), then
 * looks up one tensor.  shape receives the first 8 dimensions and rank the tensor's full rank;
 * file_offset is file-relative. */
int astro_moe_safetensors_tensor(const char *path, const char *tensor_name, int32_t *dtype,
                                 int32_t *rank, int64_t *shape, uint64_t *file_offset,
                                 uint64_t *byte_count);

/* build_quantized_expert_layer_plan (quantized_expert_layer_plan.rs:29-214): weight_map pairs
 * tensor names with shard file names relative to model_dir (model.safetensors.index.json);
 * bits / group_size are the quantization profile of each projection. */
int astro_moe_build_expert_layer_plan(const char *model_dir, const char *const *map_tensor_names,
                                      const char *const *map_shard_files, int32_t map_len,
                                      const char *layer_prefix, const int32_t bits[3],
                                      const int32_t group_size[3], astro_moe_expert_layer_plan *plan);

/* build_quantized_expert_page_manifest_from_plan (quantized_expert_manifest.rs:401-418):
 * validates expert_ids (non-empty, strictly ascending, below the capacity), fills
 * slot_of_expert[capacity] (0xffffffff where absent) and, when intervals is non-null, the
 * reads of every tensor's contiguous selected runs (9 * n at most); payload_bytes = compact
 * page bytes over all 9 tensors. */
int astro_moe_build_expert_page_manifest(const astro_moe_expert_layer_plan *plan,
                                         const int32_t *expert_ids, int32_t n, uint32_t *slot_of_expert,
                                         astro_moe_page_interval *intervals, int32_t max_intervals,
                                         int32_t *n_intervals, uint64_t *payload_bytes);

/* load_quantized_expert_page (bounded_expert_reader.rs:35-117) and, with fuse_gate_up, the
 * resident concatenation of gate and up on the output axis (resident_gate_up_fusion.rs:221-260).
 * dst[p][q] receives tensor src[p][q] of the selected experts, [n, out, inner] in page-slot
 * order; with fuse_gate_up (requires plan->gate_up_fusable) dst[0][q] receives
 * [n, 2 * out, inner] = each expert's gate rows then its up rows and dst[1][*] is unused.
 * dst_on_device: destinations are HIP device memory, written through `staging` (pinned host
 * memory of staging_bytes >= 1 MiB; null: the call allocates and frees its own) on `stream`,
 * which is synchronized before returning; otherwise host memory.  bytes_read = file bytes read. */
int astro_moe_load_expert_page(const astro_moe_expert_layer_plan *plan, const int32_t *expert_ids,
                               int32_t n, int32_t fuse_gate_up, void *const *dst, int32_t dst_on_device,
                               void *staging, size_t staging_bytes, void *stream, uint64_t *bytes_read);

/*
 * ------------------------------------------------------------------ multi-token QMV for MTP verification
 * qwen3_5_target_verification_quantized_linear (qwen3_5/model/target_verification_quantized_linear.rs:
 * 232-330), the quantized linear of an MTP target-verification window (router, shared expert,
 * attention and logits projections; :453-488):
 *   out[b][t][n] = sum_k activations[b][t][k] * (s[n][k/g] * q[n][k] + b[n][k/g])
 * activations [batch][tokens][in_features], out [batch][tokens][w.out_features], and w's scales and
 * biases all of `dtype` (ASTRO_MOE_DTYPE_BF16 or ASTRO_MOE_DTYPE_F16); w.experts == 1, codes u32
 * [out_features][in_features * bits / 32] LSB-first.  fp32 accumulation, one rounding to dtype.
 * Every output row equals the one-token projection of its own activation row bit for bit (the
 * reference's token-local contract, :333-356); for bf16 that is astro_moe_quantized_matmul of
 * that row.  Errors: validate_target_verification_projection (:378-447), then status 2 for
 * 2/3/6-bit codes, dtypes other than bf16/f16, in_features not a multiple of 128, or
 * activations or codes not 16-byte aligned.
 */
int astro_moe_verification_quantized_linear(const void *activations, int32_t batch, int32_t tokens,
                                            int32_t in_features, const astro_moe_affine *w, int32_t dtype,
                                            void *out, void *stream);

/*
 * Seeded synthetic inputs for benchmarks and tests (no counterpart in the reference):
 * device-side version of astronomical_amd/synthetic.py.  key = stream key of the tensor.
 */
int astro_synth_words(uint32_t *out, int64_t n, uint64_t key, void *stream);
int astro_synth_uniform_bf16(uint16_t *out, int64_t n, uint64_t key, double lo, double hi,
                             void *stream);
int astro_synth_affine_biases(uint16_t *out, const uint16_t *scales, int64_t n, uint64_t key,
                              double center, double noise, void *stream);
int astro_synth_normal_bf16(uint16_t *out, int64_t n, uint64_t key, double scale, void *stream);
int astro_synth_activations(uint16_t *out, int32_t tokens, int32_t hidden, uint64_t key,
                            void *stream);

/*
 * Self-test of the fp32 -> bf16 rounding every kernel uses (no counterpart in the reference):
 * the kernels round with gfx950's conversion instruction; this runs it on all 2^32 fp32 bit
 * patterns against IEEE round-to-nearest-even on the bit pattern (NaN kept quiet) and stores
 * the number of patterns that differ into *mismatches (device memory, one uint64_t; 0 means
 * the library's bf16 results are those of the bit-pattern rounding).  Asynchronous on stream.
 */
int astro_moe_selftest_bf16_rounding(uint64_t *mismatches, void *stream);

#ifdef __cplusplus
}
#endif
#endif
