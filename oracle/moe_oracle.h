/*
 * CPU oracle for the sorted mixture-of-experts block — TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the reference op graph
 * (crates/model-serving/src/qwen3_5_moe/model/{forward,routing,resident_execution,
 * output_combination}.rs and crates/model-serving/src/sparse_experts/ files), with the
 * reference's dtype flow: every MLX primitive returns a tensor rounded to its output
 * dtype (bf16 here), reductions inside a primitive accumulate in fp32.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, and only as the checker / the timed CPU baseline. The product path never
 * links it.
 *
 * bf16 values are carried as uint16_t bit patterns; packed affine weights as uint32_t.
 */
#ifndef ASTRO_MOE_ORACLE_H
#define ASTRO_MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  ORC_OK = 0,
  ORC_ERR_GEOMETRY = 1,
  ORC_ERR_UNSUPPORTED = 2,
  ORC_ERR_DUPLICATE = 3,
  ORC_ERR_OUT_OF_RANGE = 4,
  ORC_ERR_MISSING = 5,
};

/* One MLX affine projection: w [experts][out][in*bits/32] u32, scales/biases
 * [experts][out][in/group] bf16.  experts == 1 for a plain quantized linear. */
typedef struct orc_affine {
  const uint32_t *w;
  const uint16_t *scales;
  const uint16_t *biases;
  int32_t experts;
  int32_t out_features;
  int32_t in_features;
  int32_t bits;
  int32_t group_size;
} orc_affine;

typedef struct orc_layer {
  int32_t hidden;              /* H */
  int32_t num_experts;         /* E */
  int32_t top_k;               /* k */
  int32_t intermediate;        /* I */
  int32_t shared_intermediate; /* Is, 0 = no shared expert */
  int32_t normalize_top_k;     /* norm_topk_prob */
  const uint16_t *router_w;    /* bf16 [E][H]; NULL selects router_q */
  orc_affine router_q;         /* affine router, experts = 1, out = E */
  const uint16_t *router_bias; /* optional bf16 [E] added to logits (harness only) */
  orc_affine gate_up;          /* fused [E][2I][..]; w == NULL selects gate/up */
  orc_affine gate;
  orc_affine up;
  orc_affine down;             /* [E][H][I*b/32] */
  orc_affine shared_gate;      /* [1][Is][H*b/32] */
  orc_affine shared_up;
  orc_affine shared_down;      /* [1][H][Is*b/32] */
  orc_affine shared_expert_gate; /* [1][1][H*b/32] */
} orc_layer;

/* Intermediates of one block forward, all optional (NULL = not recorded). */
typedef struct orc_trace {
  uint16_t *logits;        /* [T][E] */
  uint16_t *probabilities; /* [T][E] */
  uint32_t *indices;       /* [T][k] */
  uint16_t *scores;        /* [T][k] */
  uint32_t *sorted_order;  /* [A]   (sorted path only) */
  uint32_t *inverse_order; /* [A] */
  uint32_t *sorted_ids;    /* [A] */
  uint32_t *expert_offsets;/* [E+1] */
  uint16_t *activated;     /* [A][I] in original assignment order */
  uint16_t *expert_out;    /* [A][H] in original assignment order */
  uint16_t *sparse;        /* [T][H] */
  uint16_t *shared_out;    /* [T][H] */
  uint16_t *shared_gate_logits; /* [T] */
  int32_t used_sorted_path;
} orc_trace;

/* scalar helpers */
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
float orc_expf(float x);
void orc_set_threads(int threads);
int orc_get_threads(void);

/* stage functions (reference rows 1..12) */
void orc_router_logits(const uint16_t *x, const uint16_t *w, int32_t T, int32_t H,
                       int32_t E, uint16_t *logits);
/* MLX CPU argpartition (argpartition.cc): idx = 0..n-1 after std::nth_element at kth with the
 * (value, index) comparator over bf16 values v. */
void orc_argpartition_bf16(const uint16_t *v, int32_t n, int32_t kth, uint32_t *idx);
/* a rank permutation that drives std::nth_element(n, kth) into its heap selection (test input) */
void orc_adversarial_ranks(int32_t n, int32_t kth, int32_t *ranks);
int orc_route_topk(const uint16_t *logits, int32_t T, int32_t E, int32_t k,
                   int32_t normalize, uint32_t *indices, uint16_t *scores,
                   uint16_t *probabilities);
int orc_sort_assignments(const uint32_t *ids, int32_t A, int32_t E,
                         uint32_t *sorted_order, uint32_t *inverse_order,
                         uint32_t *sorted_ids, uint32_t *expert_offsets);
int orc_invert_assignment_order(const uint32_t *sorted_order, int32_t n,
                                uint32_t *inverse_order);
int orc_dequantize(const orc_affine *w, int32_t expert, uint16_t *out_bf16);
int orc_qmm(const uint16_t *x, int32_t M, const orc_affine *w, int32_t expert,
            uint16_t *y);
int orc_verification_quantized_linear(const uint16_t *x, int32_t rows, const orc_affine *w, int32_t f16,
                                      uint16_t *y);
int orc_gather_qmm(const uint16_t *x, const uint32_t *x_rows, int32_t rows,
                   const orc_affine *w, const uint32_t *ids, uint16_t *y);
void orc_swiglu(const uint16_t *gate, const uint16_t *up, int64_t n, uint16_t *out);
void orc_sorted_weighted_sum(const uint16_t *sorted_out, const uint32_t *inverse_order,
                             const uint16_t *scores, int32_t T, int32_t k, int32_t D,
                             uint16_t *y);
void orc_unsorted_weighted_sum(const uint16_t *out, const uint16_t *scores, int32_t T,
                               int32_t k, int32_t D, uint16_t *y);
void orc_combine_shared(const uint16_t *sparse, const uint16_t *shared_out,
                        const uint16_t *gate_logits, int32_t T, int32_t D, uint16_t *y);

/* the decoder step around the block and Laguna's sigmoid router */
int orc_add_rms_norm(const uint16_t *h, const uint16_t *a, const uint16_t *w, float eps, int32_t T,
                     int32_t H, uint16_t *r_out, uint16_t *n_out);
int orc_laguna_route(const uint16_t *logits, int32_t T, int32_t E, int32_t k, const float *bias,
                     float softcap, int32_t normalize, uint32_t *indices, float *scores);

/* whole block; logits_override (bf16 [T][E], may be NULL) replaces the router
 * projection so routing can be compared on identical logits. */
int orc_moe_block_forward(const orc_layer *L, const uint16_t *x, int32_t T,
                          const uint16_t *logits_override, uint16_t *y,
                          orc_trace *trace);
int orc_decoder_ffn_forward(const orc_layer *L, const uint16_t *h, const uint16_t *a, const uint16_t *w,
                            float eps, int32_t T, uint16_t *out, uint16_t *r_out);

#ifdef __cplusplus
}
#endif
#endif
